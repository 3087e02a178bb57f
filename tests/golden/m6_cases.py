"""Inputs of the M6 and rANS golden cases (tests/golden/make_m6_golden.py writes the expected outputs).

M6: synthetic Q8_0 GGUFs (numpy-made blocks: scale max|x| / 127 as fp16, weights rounded): tensors of
several groups and row lengths, rows of very different scales, a zero row and zero blocks, an F32
tensor and metadata in the rest bytes, segments of 512 blocks that cut rows and tensors.
rANS: seeded symbol streams with one context, 64 contexts, an order-1 context with period, and a
context that holds a single symbol (frequency 2^14)."""
import numpy as np

from seedpack_amd import gguf

Q8_0, F32 = 8, 0
CASES = ["mixed", "one"]
RANS_CASES = ["o0", "ctx", "o1", "single"]


def q8_blocks(x):
    """float32 rows -> Q8_0 blocks (n, 34)"""
    xb = np.asarray(x, np.float32).reshape(-1, 32)
    d = (np.abs(xb).max(1) / np.float32(127)).astype(np.float32)
    inv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, 1), np.float32(0)).astype(np.float32)
    q = np.clip(np.rint(xb * inv[:, None]), -128, 127).astype(np.int8)
    out = np.zeros((len(xb), 34), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out


def _file(kv, tensors):
    """a GGUF v3 file: tensors [(name, shape (ggml order), type, payload bytes)]"""
    head, places, size = gguf.header_bytes(kv, [(n, s, t) for n, s, t, _ in tensors])
    out = np.zeros(size, np.uint8)
    out[:len(head)] = np.frombuffer(head, np.uint8)
    for (at, nb), (_, _, _, payload) in zip(places, tensors):
        out[at:at + nb] = np.frombuffer(payload, np.uint8)
    return out.tobytes()


def case_file(name):
    g = np.random.Generator(np.random.PCG64({"mixed": 61, "one": 62}[name]))
    if name == "mixed":
        ts = []
        for tname, cols, rows in (("blk.0.attn_q.weight", 256, 48), ("blk.0.ffn_up.weight", 512, 40),
                                  ("blk.1.attn_q.weight", 256, 48), ("token_embd.weight", 128, 300)):
            x = g.standard_normal((rows, cols)).astype(np.float32) * np.exp(g.standard_normal((rows, 1)) * 1.5).astype(np.float32) * 0.02
            x[g.integers(0, rows)] = 0                       # a zero row
            ts.append((tname, (cols, rows), Q8_0, q8_blocks(x).tobytes()))
        norm = (1 + 0.1 * g.standard_normal(256)).astype(np.float32)
        ts.insert(2, ("blk.0.attn_norm.weight", (256,), F32, norm.tobytes()))
        kv = {"general.architecture": "llama", "general.name": "m6 case", "llama.block_count": 2}
        return _file(kv, ts)
    cols, rows = 960, 700                                  # 30 blocks a row: segments start mid-row
    x = (g.standard_t(5, (rows, cols)) * 0.015).astype(np.float32)
    x[:, 64:96] = 0                                          # a zero block in every row
    x[g.random((rows, cols)) < 0.001] *= 40
    return _file({"general.name": "m6 one tensor"}, [("blk.3.ffn_down.weight", (cols, rows), Q8_0, q8_blocks(x).tobytes())])


def o1_context(sym, period):
    """the previous symbol, 0 at every period-th position (rans.py:141-146)"""
    ctx = np.zeros(len(sym), np.int32)
    ctx[1:] = sym[:-1]
    ctx[::period] = 0
    return ctx


def rans_case(name):
    """-> (symbols uint8, contexts int32, number of contexts, o1 period or 0)"""
    g = np.random.Generator(np.random.PCG64({"o0": 71, "ctx": 72, "o1": 73, "single": 74}[name]))
    if name == "o0":
        sym = np.minimum(g.geometric(0.15, 5000) - 1, 255).astype(np.uint8)
        return sym, np.zeros(len(sym), np.int32), 1, 0
    if name == "ctx":
        ctx = g.integers(0, 64, 20000).astype(np.int32)
        sym = ((ctx * 3 + np.minimum(g.geometric(0.3, 20000) - 1, 40)) % 256).astype(np.uint8)
        return sym, ctx, 64, 0
    if name == "o1":
        sym = np.zeros(10000, np.uint8)
        for i in range(1, len(sym)):
            sym[i] = (int(sym[i - 1]) + int(g.integers(-3, 4))) % 256 if g.random() < 0.9 else int(g.integers(0, 256))
        return sym, o1_context(sym, 700), 256, 700
    ctx = (g.random(3000) < 0.5).astype(np.int32)
    sym = np.where(ctx == 1, 7, g.integers(0, 256, 3000)).astype(np.uint8)   # context 1: symbol 7 only
    return sym, ctx, 2, 0
