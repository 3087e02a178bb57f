"""Seeded synthetic inputs of the benchmark configurations (BF16 weights + imatrix).

Values are drawn in float64 with numpy's PCG64 at seed 0x5EED0000 + 16*config + tensor, cast to
float32 and rounded to BF16 with round-to-nearest-even, (u + 0x7FFF + ((u >> 16) & 1)) >> 16 -- the
rounding the reference applies to float tensors (seedpack/repo2.py:46-48). An imatrix is one
LogNormal(0, 1) float32 per input column.
"""
import numpy as np

SEED0 = 0x5EED0000


def rng(config, tensor=0):
    return np.random.Generator(np.random.PCG64(SEED0 + 16 * config + tensor))


def bf16_bits(x):
    """float32 -> bf16 bits (uint16), round to nearest even"""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(g, shape, std, outlier_frac=0.0, outlier_std=0.5):
    x = g.normal(0.0, std, size=shape)
    if outlier_frac:
        n = x.size
        k = int(round(n * outlier_frac))
        idx = g.choice(n, size=k, replace=False)
        x.reshape(-1)[idx] = g.normal(0.0, outlier_std, size=k)
    return bf16_bits(x.astype(np.float32))


def student_t_bf16(g, shape, df=5, std=0.015):
    x = g.standard_t(df, size=shape) * (std / np.sqrt(df / (df - 2.0)))
    return bf16_bits(x.astype(np.float32))


def imatrix(g, ncols):
    return g.lognormal(0.0, 1.0, size=ncols).astype(np.float32)


# config -> tensors (name, rows, cols); cols = n_per_row, rows back to back (row-major)
SHAPES = {
    1: [("blk.0.ffn_up", 3072, 1024)],
    2: [("token_embd", 151936, 1024), ("blk.0.ffn_down", 1024, 3072)],
    3: [("blk.0.ffn_up", 4096, 12288), ("blk.0.ffn_down", 12288, 4096)],
}

TYPES = {
    1: [8, 2],                          # Q8_0, Q4_0 (no imatrix)
    2: [10, 11, 12, 13, 14],            # Q2_K .. Q6_K
    3: [23, 18, 17, 16, 19, 29],        # IQ4_XS, IQ3_XXS, IQ2_XS, IQ2_XXS, IQ1_S, IQ1_M
}


def tensor(config, index, rows=None):
    """(bf16 bits (rows, cols), imatrix or None) of tensor `index` of a config; `rows` takes the
    first rows only (same generator stream)"""
    name, r, c = SHAPES[config][index]
    g = rng(config, index)
    r = r if rows is None else min(rows, r)
    if config == 1:
        w = normal_bf16(g, (r, c), 0.02, outlier_frac=0.001)
        return w, None
    if config == 2:
        w = normal_bf16(g, (r, c), 0.02)
    else:
        w = student_t_bf16(g, (r, c))
    return w, imatrix(g, c)


# ------------------------------------------------------------------ synthetic model repositories

def qwen_tensors(layers=36, hidden=4096, ffn=12288, kv=1024, vocab=151936, norms=True):
    """the tensors of a Qwen3.5-9B-shaped BF16 GGUF in llama.cpp's order: (name, ggml shape (row
    length first), type) -- 2-D matrices BF16, norms F32"""
    out = [("token_embd.weight", (hidden, vocab), 30)]
    for b in range(layers):
        p = f"blk.{b}."
        if norms:
            out.append((p + "attn_norm.weight", (hidden,), 0))
        out += [(p + "attn_q.weight", (hidden, hidden), 30), (p + "attn_k.weight", (hidden, kv), 30),
                (p + "attn_v.weight", (hidden, kv), 30), (p + "attn_output.weight", (hidden, hidden), 30)]
        if norms:
            out.append((p + "ffn_norm.weight", (hidden,), 0))
        out += [(p + "ffn_gate.weight", (hidden, ffn), 30), (p + "ffn_up.weight", (hidden, ffn), 30),
                (p + "ffn_down.weight", (ffn, hidden), 30)]
    if norms:
        out.append(("output_norm.weight", (hidden,), 0))
    out.append(("output.weight", (hidden, vocab), 30))
    return out


def bpe_tokenizer(nmerge, nspecial=8, seed=0x70C):
    """(tokens, merges) of a synthetic byte-level BPE vocabulary: 256 byte tokens (no spaces), nmerge
    merged tokens (token 256 + k is the concatenation of the pair merge rule k names), special tokens"""
    g = np.random.Generator(np.random.PCG64(seed))
    toks = [(chr(33 + i) if i < 94 else chr(0x100 + i)).encode() for i in range(256)]
    merges = []
    for k in range(nmerge):
        hi = 256 + k
        a = int(g.integers(0, hi))
        b = int(g.integers(0, min(hi, 256 + k // 2 + 1)))
        toks.append(toks[a] + toks[b])
        merges.append(toks[a] + b" " + toks[b])
    return toks + [f"<|special_{j}|>".encode() for j in range(nspecial)], merges


def q4_k_m(name):
    """a Q4_K_M-like mix: Q6_K for attn_v, ffn_down and output, Q4_K elsewhere"""
    return 14 if any(k in name for k in ("attn_v", "ffn_down", "output.")) else 12


def write_repo(root, tensors, files, per_million=10000, nmerge=20000, seed=0x5EED0400, stream=None, log=None):
    """a synthetic model repository in directory `root`: model-BF16.gguf (the tensors, BF16 N(0, 0.02)
    from a counter-based generator on the device, F32 norms near 1, a BPE tokenizer), imatrix.dat (one
    LogNormal(0, 1) value per input column of every matrix), README.md, and per entry of `files`
    {name: type_of(tensor name) -> ggml type} a quantized GGUF made by this library's quantizers with
    the imatrix, per_million / 10^6 of its blocks carrying one changed byte. -> {file name: bytes}"""
    import os

    from . import device as dev
    from . import gguf
    from . import imatrix as imx
    from ._lib import check, lib
    from .gpuquant import GPUQuant
    from .requant import QFUN
    os.makedirs(root, exist_ok=True)
    st = stream.handle if stream is not None else None
    g = np.random.Generator(np.random.PCG64(seed))
    toks, merges = bpe_tokenizer(nmerge, seed=seed + 1)
    kv = {"general.architecture": "qwen35", "general.name": "synthetic Qwen3.5-9B-shaped", "general.alignment": 32,
          "qwen35.block_count": sum(1 for n, s, t in tensors if n.endswith("attn_q.weight")),
          "tokenizer.ggml.model": "gpt2", "tokenizer.ggml.tokens": toks, "tokenizer.ggml.token_type": [1] * len(toks),
          "tokenizer.ggml.merges": merges, "tokenizer.ggml.eos_token_id": len(toks) - 1}
    mats = [(n, s) for n, s, t in tensors if len(s) == 2]
    imx_h = {n: imatrix(g, s[0]) for n, s in mats}
    sizes = {}
    with open(os.path.join(root, "imatrix.dat"), "wb") as f:
        f.write(imx.write_dat(imx_h, ncall=1, chunk_count=125, dataset="synthetic.txt"))
    with open(os.path.join(root, "README.md"), "w") as f:
        f.write("synthetic repository: weights N(0, 0.02), quant files made from them with 1% of blocks changed\n")
    # the base, kept on the device for the quantizers
    head, where, size = gguf.header_bytes({**kv, "general.file_type": 32}, tensors)
    base = dev.DeviceArray(size, np.uint8).zero(st)
    host = dev.pinned(size)
    host[:len(head)] = np.frombuffer(head, np.uint8)
    check(lib().spa_memcpy_h2d(base.ptr, host.ctypes.data, len(head), st))
    norms = {}
    for k, ((n, s, t), (off, nb)) in enumerate(zip(tensors, where)):
        if t == 30:
            check(lib().spa_synth_normal_bf16(base.ptr + off, nb // 2, seed + 16 * k, 0.02, st))
        else:
            norms[n] = (1.0 + 0.02 * g.standard_normal(nb // 4)).astype(np.float32)
            host[off:off + nb] = norms[n].view(np.uint8)
            check(lib().spa_memcpy_h2d(base.ptr + off, host[off:].ctypes.data, nb, st))
    check(lib().spa_memcpy_d2h(host.ctypes.data, base.ptr, size, st))
    with open(os.path.join(root, "model-BF16.gguf"), "wb") as f:
        f.write(memoryview(host))
    sizes["model-BF16.gguf"] = size
    del host
    imx_d = {n: dev.DeviceArray.from_host(v, st) for n, v in imx_h.items()}
    gq = GPUQuant(stream=st)
    specs = []
    for fname, type_of in files.items():
        qt = [(n, s, type_of(n) if len(s) == 2 else t) for n, s, t in tensors]
        specs.append((fname, qt) + gguf.header_bytes({**kv, "general.file_type": 15, "quantize.imatrix.file": "imatrix.dat",
                                                      "quantize.imatrix.chunks_count": 125}, qt))
    staging = dev.pinned(max((sp[4] for sp in specs), default=1))      # one page-locked buffer for every file
    for fi, (fname, qt, qhead, qwhere, qsize) in enumerate(specs):
        out = staging[:qsize]
        out[:] = 0
        out[:len(qhead)] = np.frombuffer(qhead, np.uint8)
        for k, ((n, s, t), (off, nb)) in enumerate(zip(qt, qwhere)):
            if len(s) == 1:
                out[off:off + nb] = norms[n].view(np.uint8)
                continue
            boff = where[k][0]
            y = gq.quantize_tensors(t, [(base.view(boff, (s[0] * s[1],), np.uint16), s[0])], [imx_d[n]], device=True)[0]
            bs = QFUN[t][2]
            check(lib().spa_perturb_blocks(y.ptr, y.nbytes // bs, bs, per_million, seed + 100003 * (fi + 1) + k, st))
            check(lib().spa_memcpy_d2h(out[off:].ctypes.data, y.ptr, nb, st))
            del y
        with open(os.path.join(root, fname), "wb") as f:
            f.write(memoryview(out))
        sizes[fname] = qsize
        if log:
            log(f"synthetic repo: {fname} {qsize:,} B")
    return sizes
