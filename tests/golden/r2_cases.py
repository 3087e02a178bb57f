"""R2 golden cases: small files of 2-D BF16 tensors (shared by make_r2_golden.py and the tests, which
regenerate the files instead of storing them).

A case file is a few tensors laid out as in a GGUF (a header, 32-byte aligned tensors, small
gaps holding other data); the layout has the R2 form (bf16v2.py:182-188): tensors by offset as
[offset, bytes, row length, "bf16"], each tensor's role index (its name without "blk.N."), in order
of first appearance.
"""
import re

import numpy as np

from seedpack_amd import synth

CASES = [  # (name, [(tensor name, rows, row length, distribution)], group bytes)
    ("single", [("blk.0.ffn_down.weight", 48, 1024, "normal")], 400 << 20),
    ("roles", [("blk.0.ffn_up.weight", 40, 512, "normal"), ("blk.0.attn_q.weight", 24, 768, "student"),
               ("blk.1.ffn_up.weight", 40, 512, "normal"), ("blk.1.attn_q.weight", 24, 768, "student"),
               ("output_norm.weight", 1, 512, "normal")], 64 << 10),
    ("embd_dups", [("token_embd.weight", 300, 256, "dups")], 400 << 20),
    ("wide", [("blk.0.ffn_gate.weight", 6, 6144, "student"), ("blk.0.ffn_up.weight", 6, 6144, "bias")], 400 << 20),
]


def role(name):
    return re.sub(r"blk\.\d+\.", "", name)


def _tensor(g, rows, rl, dist):
    if dist == "normal":
        return synth.normal_bf16(g, (rows, rl), 0.02)
    if dist == "student":
        return synth.student_t_bf16(g, (rows, rl))
    if dist == "bias":                       # columns with a mean: the sign context's classes
        x = g.normal(0, 0.02, (rows, rl)) + np.linspace(-0.05, 0.05, rl)[None, :]
        return synth.bf16_bits(x.astype(np.float32))
    # duplicate and all-zero rows (untrained embeddings), a loud row, a constant column
    x = g.normal(0, 0.02, (rows, rl)).astype(np.float32)
    x[10:20] = x[0]
    x[50:53] = 0.0
    x[200] = x[3]
    x[7] *= 500.0
    x[:, 5] = 0.01
    b = synth.bf16_bits(x)
    b[120] = b[121]
    return b


def case_file(name):
    """(file bytes, R2 layout, group bytes) of case `name`"""
    k = [c[0] for c in CASES].index(name)
    _, tensors, group_bytes = CASES[k]
    g = np.random.Generator(np.random.PCG64(0x2B2 + k))
    parts = [g.integers(0, 256, 96, dtype=np.uint8).tobytes()]        # header stand-in
    pos = 96
    t, roles, rix = [], [], []
    for tname, rows, rl, dist in tensors:
        pad = (-pos) % 32
        parts.append(b"\0" * pad); pos += pad
        b = _tensor(g, rows, rl, dist).reshape(-1)
        if rows > 1:
            if role(tname) not in roles:
                roles.append(role(tname))
            t.append([pos, b.nbytes, rl, "bf16"]); rix.append(roles.index(role(tname)))
        parts.append(b.tobytes()); pos += b.nbytes
        gap = g.integers(0, 256, 40, dtype=np.uint8).tobytes()          # other data between tensors
        parts.append(gap); pos += len(gap)
    data = b"".join(parts)
    return data, {"size": len(data), "t": t, "role": rix, "nroles": len(roles)}, group_bytes
