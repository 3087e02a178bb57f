"""Writes seed codec golden vectors (seedpack/seed.py SeedCodec: a base-less quantized GGUF coded by
parts) by running the reference's own code on the CPU: seed.py, gpu2.py / gpu3.py (the Q8_0 codec),
bf16v2.py / gpu_bf16.py (the BF16 codec and its header coder) and qr.py (QR without a seed), through
the reference's --cpu backend (seedpack/cpu.py, seedpack/cpukernels.py). Run in the build container
only:

    python tests/golden/make_seed_golden.py

These modules import numba and zstandard (absent here), so their top-level statements other than
the imports are executed from the source text (read with `ast`), each module in a namespace of its
own holding what its imports would: the --cpu backend as `cp`, the reference's detmath, this
repository's GGUF reader for GGUF.from_bytes (the reference reader's fields: tensors with name, shape,
type, absolute offset and bytes; spans; data_start), and its framing / libzstd bindings for pack /
pack_parts / unpack / zstd_c / zstd_d (codecs_gguf.py:26-83; zstd 1.5.7). Functions that import
other reference modules at run time (gpuquant, for QR without a seed) import them from the
reference package under the --cpu backend. SeedCodec is built with the reference's Q8Parts() and
BF16v2(budget=1_500_000_000) (seed.py:60-64).

Cases (tests/golden/seed_vectors.npz): "<case>/input" the seed file (a GGUF written here with a BPE
tokenizer or without metadata; Q8_0 token_embd and attention tensors, Q4_K / Q6_K tensors of 64 KiB
and more, 2-D F16 (some weights not BF16 values) and BF16 tensors, F32 vectors below and above
64 KiB; quantized blocks from the reference's C quantizers, oracle/_ref), "<case>/chunk" the
reference's SeedCodec.compress output. Each chunk is decoded again by the reference as a check.
"""
import ast
import json
import lzma
import os
import re
import struct
import sys
import tempfile
import types
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, ROOT)

os.environ["SEEDPACK_CPU"] = "1"
os.environ.setdefault("SEEDPACK_CACHE", tempfile.mkdtemp(prefix="seedpack_refcache_"))
sys.path.insert(0, REF)

from oracle import ref as qref  # noqa: E402
from seedpack_amd import framing, gguf, zstd  # noqa: E402
from tests.golden.header_cases import _bpe  # noqa: E402
from tests.golden.q8_cases import group_of, q8_blocks  # noqa: E402

CASES = ["tok", "plain"]


class _GGUF:
    """GGUF.from_bytes of the reference reader, by this repository's reader (the same fields)"""

    @staticmethod
    def from_bytes(data, light=False):
        return gguf.GGUF(np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else data, light)


def _exec_module(name, ns):
    path = os.path.join(REF, "seedpack", name)
    src = open(path).read()
    ns.setdefault("__name__", "seedpack." + name[:-3])
    ns.setdefault("__package__", "seedpack")
    for node in ast.parse(src).body:
        if isinstance(node, (ast.Import, ast.ImportFrom)):
            continue
        exec(compile(ast.Module([node], []), path, "exec"), ns)
    return ns


def load():
    from seedpack import cpu as cp
    from seedpack import detmath
    common = {"np": np, "cp": cp, "cupyx": cp.cupyx, "detmath": detmath, "json": json, "lzma": lzma, "struct": struct,
              "os": os, "re": re, "sys": sys, "ThreadPoolExecutor": ThreadPoolExecutor, "pack": framing.pack,
              "pack_parts": framing.pack_parts, "unpack": framing.unpack, "zstd_c": zstd.zstd_c, "zstd_d": zstd.decompress,
              "group_of": group_of, "GGUF": _GGUF, "BLOCK": gguf.BLOCK, "GGML_F32": 0, "GGML_F16": 1, "GGML_Q8_0": 8,
              "GGML_BF16": 30}
    g2 = _exec_module("gpu2.py", dict(common, __name__="seedpack.gpu2"))
    g3 = _exec_module("gpu3.py", dict(g2, __name__="seedpack.gpu3"))
    fromg2 = {k: g2[k] for k in ("normalize_gpu", "cum_of", "store_tables", "load_tables", "Timer", "GPU2", "h2d", "_trim",
                                 "header_pairs_c", "header_pairs_d", "xz_chunks_c", "xz_chunks_d", "rest_of", "fill_rest",
                                 "parse_layout", "PB")}
    gb = _exec_module("gpu_bf16.py", dict(common, **fromg2, __name__="seedpack.gpu_bf16"))
    b2 = _exec_module("bf16v2.py", dict(common, **fromg2, M24BF16GPU=gb["M24BF16GPU"], __name__="seedpack.bf16v2"))
    qn = _exec_module("qr.py", dict(common, **{k: fromg2[k] for k in ("cum_of", "store_tables", "load_tables", "h2d")},
                                    __name__="seedpack.qr"))
    sd = _exec_module("seed.py", dict(common, fill_rest=fromg2["fill_rest"], _trim=fromg2["_trim"],
                                      qr=types.SimpleNamespace(**qn), __name__="seedpack.seed"))
    return sd, g3, b2


def codec(sd, g3, b2):
    """SeedCodec with the reference's parts (seed.py:60-64), built without its module imports"""
    c = sd["SeedCodec"].__new__(sd["SeedCodec"])
    c.q8 = g3["Q8Parts"]()
    c.r2 = b2["BF16v2"](budget=1_500_000_000)
    return c


def _quant(T, x):
    return qref.quantize(T, x.astype(np.float32)).reshape(-1)


def seed_file(name):
    """a seed GGUF: (bytes, description)"""
    g = np.random.Generator(np.random.PCG64(0x5EED + CASES.index(name)))
    kv = {"general.architecture": "qwen35", "general.name": f"seed case {name}", "general.alignment": 32,
          "qwen35.block_count": 2}
    if name == "tok":
        toks, merges = _bpe(g, 600)
        kv.update({"tokenizer.ggml.model": "gpt2", "tokenizer.ggml.tokens": toks, "tokenizer.ggml.merges": merges,
                   "tokenizer.ggml.token_type": [1] * len(toks)})
    else:
        kv = {}
    def normal(rows, cols, s=0.02):
        cs = np.exp(g.normal(0, 0.4, cols))
        return (g.normal(0, s, (rows, cols)) * cs).astype(np.float32)
    emb = normal(300, 128)
    for r in range(40, 300):
        if g.random() < 0.6:
            a, b = g.integers(0, r, 2)
            emb[r] = 0.7 * emb[a] + 0.3 * emb[b] + 0.3 * emb[r]
    emb[60:62] = emb[5]
    f16 = normal(96, 256).astype(np.float16)
    f16 = (f16.view(np.uint16) & 0xFFF8).view(np.float16)           # mostly BF16 values (low mantissa bits clear)
    f16.reshape(-1)[g.integers(0, f16.size, 50)] += np.float16(0.0001)  # some are not
    bf = (normal(64, 256).view(np.uint32) >> 16).astype(np.uint16)
    tensors = [
        ("token_embd.weight", (128, 300), 8, q8_blocks(emb).tobytes()),
        ("blk.0.attn_norm.weight", (256,), 0, (1 + 0.01 * g.normal(size=256)).astype(np.float32).tobytes()),
        ("blk.0.attn_q.weight", (256, 64), 8, q8_blocks(normal(64, 256)).tobytes()),
        ("blk.0.attn_k.weight", (256, 64), 30, bf.tobytes()),
        ("blk.0.ffn_up.weight", (512, 256), 12, _quant(12, normal(256, 512)).tobytes()),
        ("blk.0.ffn_down.weight", (1024, 80), 14, _quant(14, normal(80, 1024)).tobytes()),
        ("blk.1.ffn_gate.weight", (256, 512), 12, _quant(12, 0.001 * np.round(normal(512, 256) * 1000)).tobytes()),
        ("rope_freqs.weight", (20000,), 0, np.linspace(0, 1, 20000, dtype=np.float32).tobytes()),
        ("output.weight", (256, 96), 1, f16.tobytes()),
    ]
    shapes = [(n, s, t) for n, s, t, _ in tensors]
    head, where, size = gguf.header_bytes(kv, shapes)
    out = np.zeros(size, np.uint8)
    out[:len(head)] = np.frombuffer(head, np.uint8)
    for (_, _, _, payload), (off, nb) in zip(tensors, where):
        assert nb == len(payload), (nb, len(payload))
        out[off:off + nb] = np.frombuffer(payload, np.uint8)
    return out.tobytes()


def main():
    sd, g3, b2 = load()
    out = {}
    for name in CASES:
        data = seed_file(name)
        c = codec(sd, g3, b2)
        chunk = c.compress(data)
        back = codec(sd, g3, b2).decompress(chunk)
        assert np.asarray(back).tobytes() == data, f"{name}: the reference does not round-trip"
        parts = framing.unpack(chunk)
        print(f"{name}: {len(data)} B -> {len(chunk)} B; parts {[(k, len(v)) for k, v in parts.items()]}", flush=True)
        out[f"{name}/input"] = np.frombuffer(data, np.uint8)
        out[f"{name}/chunk"] = np.frombuffer(chunk, np.uint8)
    np.savez_compressed(os.path.join(HERE, "seed_vectors.npz"), **out)


if __name__ == "__main__":
    main()
