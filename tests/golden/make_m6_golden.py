"""Writes M6 golden vectors by running the reference's own seedpack/gpu_codec.py (M6GPU: its CUDA kernel
text compiled for the CPU by the reference's --cpu backend, seedpack/cpu.py and cpukernels.py) on the
synthetic Q8_0 GGUFs of tests/golden/m6_cases.py, and the reference's rans.py coder (_encode, _decode,
_decode_o1, build_freqs, normalize, o1_context) on seeded symbol streams. Run in the build container
only:

    python tests/golden/make_m6_golden.py

gpu_codec.py, codecs_gguf.py, gguf_reader.py and rans.py import numba and zstandard (absent here), so
their top-level statements other than the imports are executed from the source text (read with `ast`)
in namespaces that supply what the imports would: the --cpu backend as `cp`, numba's njit as the plain
function (rans.py's coders and gguf_reader's string skipper are plain loops), and this repository's
libzstd binding for codecs_gguf's zstd_c / zstd_d (zstd 1.5.7; the rest of codecs_gguf -- pack,
split, join, xz, tables -- is the reference's own text). Each M6 chunk is decoded again by the
reference's M6GPU.decompress as a check, each rANS stream by its decoder. Output:
tests/golden/m6_vectors.npz (data only).
"""
import ast
import json
import lzma
import os
import struct
import subprocess
import sys
import tempfile
import types
from collections import defaultdict
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, ROOT)

os.environ["SEEDPACK_CPU"] = "1"
os.environ.setdefault("SEEDPACK_CACHE", tempfile.mkdtemp(prefix="seedpack_refcache_"))
sys.path.insert(0, REF)

from seedpack_amd import zstd  # noqa: E402
from tests.golden.m6_cases import CASES, RANS_CASES, case_file, rans_case  # noqa: E402

NUMBA = types.SimpleNamespace(njit=lambda *a, **k: (lambda f: f))


def _exec_module(path, ns):
    src = open(path).read()
    for node in ast.parse(src).body:
        if isinstance(node, (ast.Import, ast.ImportFrom)):
            continue
        exec(compile(ast.Module([node], []), path, "exec"), ns)
    return ns


def load():
    from seedpack import cpu as cp
    gr = _exec_module(os.path.join(REF, "seedpack", "gguf_reader.py"),
                      {"np": np, "struct": struct, "numba": NUMBA, "dataclass": __import__("dataclasses").dataclass,
                       "__name__": "gguf_reader_ref"})
    rans = _exec_module(os.path.join(REF, "seedpack", "rans.py"), {"np": np, "njit": NUMBA.njit, "__name__": "rans_ref"})
    cg = _exec_module(os.path.join(REF, "seedpack", "codecs_gguf.py"),
                      {"np": np, "json": json, "lzma": lzma, "struct": struct, "subprocess": subprocess,
                       "defaultdict": defaultdict, "rans": types.SimpleNamespace(**rans), "GGUF": gr["GGUF"],
                       "GGML_Q8_0": gr["GGML_Q8_0"], "zstandard": None, "__name__": "codecs_gguf_ref"})
    cg["zstd_c"] = zstd.zstd_c
    cg["zstd_d"] = zstd.decompress
    names = ("split", "join", "pack", "unpack", "zstd_c", "zstd_d", "xz_c", "xz_d", "tables_c", "tables_d", "N_COL", "N_SB")
    gc = _exec_module(os.path.join(REF, "seedpack", "gpu_codec.py"),
                      {"np": np, "json": json, "struct": struct, "ThreadPoolExecutor": ThreadPoolExecutor, "cp": cp,
                       "rans": types.SimpleNamespace(**rans), **{k: cg[k] for k in names}, "__name__": "gpu_codec_ref"})
    return gc, rans


def main():
    gc, rans = load()
    out = {}
    for name in CASES:
        data = case_file(name)
        buf = gc["M6GPU"]().compress(data)
        back = gc["M6GPU"]().decompress(buf)
        assert back == data, f"{name}: the reference does not round-trip"
        out[f"{name}/chunk"] = np.frombuffer(buf, np.uint8)
        print(f"m6 {name}: {len(data)} B -> {len(buf)} B", flush=True)
    for name in RANS_CASES:
        sym, ctx, nctx, period = rans_case(name)
        f = rans["build_freqs"](sym, ctx, nctx)
        enc = rans["encode"](sym, ctx, f)
        if period:
            dec = rans["decode_o1"](enc, len(sym), f, period)
        else:
            dec = rans["decode"](enc, ctx, f)
        assert np.array_equal(dec, sym), f"{name}: the reference's rANS does not round-trip"
        out[f"rans/{name}/freq"] = f
        out[f"rans/{name}/stream"] = np.frombuffer(enc, np.uint8)
        print(f"rans {name}: {len(sym)} symbols, {nctx} contexts -> {len(enc)} B", flush=True)
    np.savez_compressed(os.path.join(HERE, "m6_vectors.npz"), **out)


if __name__ == "__main__":
    main()
