"""Q8_0 codec (M22 / Q8Parts) golden cases: small files of Q8_0 tensors, shared by make_q8_golden.py
and the tests, which regenerate the files instead of storing them.

A case file is a header stand-in followed by 32-byte aligned Q8_0 tensors with small gaps; its layout
has the reference's Q8_0 form (gpu2.py:316-320): tensors by offset as [offset, bytes, row length,
group], the group being the tensor name without "blk.N." and ".weight".

Tensor kinds:
  "normal"  Gaussian weights with per-column scales and biases (column factors, sign classes);
  "embd"    token embeddings: most rows a mix of two earlier rows plus noise (row prediction finds
            them), duplicate rows (references), all-zero rows, loud rows;
  "odd"     like normal, plus hand-made blocks: weights of -128, a zero scale with non-zero weights,
            a negative scale, a subnormal scale;
  "embd_bad" like embd, plus blocks whose fp16 scale is +inf, -inf or NaN (a damaged file): the
            planner's row and column statistics become NaN, and its int8 side values of NaN are 0.
"""
import numpy as np

CASES = [  # (name, [(tensor name, rows, row length, kind)], options)
    ("mixed", [("token_embd.weight", 2300, 128, "embd"), ("blk.0.attn_q.weight", 96, 256, "normal"),
               ("blk.0.ffn_up.weight", 128, 512, "odd"), ("blk.1.attn_q.weight", 96, 256, "dups"),
               ("output.weight", 64, 128, "normal")], {}),
    ("small_slices", [("token_embd.weight", 600, 256, "embd"), ("blk.0.ffn_down.weight", 300, 384, "normal"),
                      ("blk.1.ffn_down.weight", 40, 384, "odd")], {"stat_elems": 8192}),
    ("no_pred", [("token_embd.weight", 200, 256, "embd"), ("blk.0.attn_k.weight", 70, 128, "dups")], {}),
    ("parts", [("blk.0.attn_v.weight", 64, 256, "normal"), ("token_embd.weight", 700, 128, "embd"),
               ("blk.0.ffn_gate.weight", 96, 512, "odd"), ("blk.1.attn_v.weight", 64, 256, "dups")],
     {"part_bytes": 80000}),
    ("bad_scales", [("token_embd.weight", 400, 128, "embd_bad"), ("blk.0.attn_q.weight", 64, 256, "normal")], {}),
]


def group_of(name):
    """blk.13.ffn_up.weight -> ffn_up; token_embd.weight -> token_embd (codecs_gguf.py:163-166)"""
    p = name.split(".")
    return p[2] if p[0] == "blk" else p[0]


def q8_blocks(x):
    """float32 (rows, C) -> Q8_0 bytes (rows * C / 32, 34): d = amax / 127 as fp16, q = round(x / d)"""
    b = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(b).max(1)
    d = (amax / 127).astype(np.float32)
    idv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1), 0).astype(np.float32)
    v = b * idv[:, None]
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127).astype(np.int8)
    out = np.zeros((len(b), 34), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out


def _weights(g, rows, C, kind):
    cs = np.exp(g.normal(0, 0.5, C)).astype(np.float32)
    x = (g.normal(0, 0.02, (rows, C)) * cs + 0.004 * g.normal(0, 1, C) * cs).astype(np.float32)
    if kind.startswith("embd"):
        for r in range(40, rows):
            if g.random() < 0.7:
                p1, p2 = g.integers(0, r, 2)
                a, b = g.normal(0.7, 0.2), g.normal(0.3, 0.2)
                x[r] = a * x[p1] + b * x[p2] + 0.4 * x[r]
        x[100:104] = x[20]
        x[150:152] = 0.0
        x[7] *= 50.0
        x[rows - 1] = x[rows // 2]
    if kind == "dups":
        x[5:9] = x[2]
        x[rows - 1] = x[0]
    return x


def _tensor(g, rows, C, kind):
    blk = q8_blocks(_weights(g, rows, C, kind))
    if kind == "odd":
        blk[3, 2 + 5] = 0x80                                  # a weight of -128
        blk[4, :2] = 0                                        # zero scale, non-zero weights
        blk[5, :2] = np.frombuffer(np.float16(-0.01).tobytes(), np.uint8)      # negative scale
        blk[6, :2] = (3, 0)                                   # subnormal scale
        blk[7, 2:] = 0                                        # all-zero weights
        blk[8, 2:] = 0x7f                                     # ties for the maximum
    if kind == "embd_bad":
        nb = C // 32
        blk[60 * nb + 1, :2] = (0x00, 0x7c)                   # +inf
        blk[61 * nb, :2] = (0x00, 0xfc)                       # -inf
        blk[62 * nb + 2, :2] = (0x01, 0x7e)                   # NaN
        blk[63 * nb + 3, :2] = (0x00, 0x7c)
        blk[63 * nb + 3, 2:] = 0                              # +inf times zero weights
    return blk


def case_file(name):
    """(file bytes, layout, options) of case `name`"""
    k = [c[0] for c in CASES].index(name)
    _, tensors, opts = CASES[k]
    g = np.random.Generator(np.random.PCG64(0x0880 + k))
    parts = [g.integers(0, 256, 160, dtype=np.uint8).tobytes()]
    pos = 160
    t = []
    for tname, rows, C, kind in tensors:
        pad = (-pos) % 32 + 32 * int(g.integers(0, 3))
        parts.append(g.integers(0, 256, pad, dtype=np.uint8).tobytes())
        pos += pad
        b = _tensor(g, rows, C, kind).tobytes()
        t.append([pos, len(b), C, group_of(tname)])
        parts.append(b)
        pos += len(b)
    parts.append(g.integers(0, 256, 40, dtype=np.uint8).tobytes())
    data = b"".join(parts)
    return data, {"size": len(data), "t": t}, opts
