"""Writes Q8_0 codec golden vectors (M22 = gpu3.M22Fast, the codec of gpu3.Q8Parts that SeedCodec
uses for a seed's Q8_0 tensors) by running the reference's own code on the CPU: gpu2.py and gpu3.py
(the classes GPU2, GPU3, M17..M22Fast, their kernels and host steps) through the reference's --cpu
backend (seedpack/cpu.py, seedpack/cpukernels.py) and its detmath module. Run in the build
container only:

    python tests/golden/make_q8_golden.py

gpu2.py / gpu3.py import numba and zstandard (absent here), so their top-level statements other than
the imports are executed from the source text (read with `ast`) in a namespace that supplies what
the imports would: the --cpu backend as `cp`, the reference's detmath, and this repository's framing
and libzstd bindings for pack / unpack / zstd_c / zstd_d (the formats of codecs_gguf.py:26-83; zstd
1.5.7). M22Fast.compress runs with header=False (the caller's way in Q8Parts, gpu3.py:606-627), on
the tensors of tests/golden/q8_cases.py; the Q8Parts case groups tensors by the part budget as
Q8Parts.compress does (gpu3.py:612-617). Each case's coded chunk is decoded again by the
reference's M22Fast.decompress as a check. Output: tests/golden/q8_vectors.npz (data only).
"""
import ast
import json
import lzma
import os
import struct
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, ROOT)

os.environ["SEEDPACK_CPU"] = "1"
os.environ.setdefault("SEEDPACK_CACHE", tempfile.mkdtemp(prefix="seedpack_refcache_"))
sys.path.insert(0, REF)

from seedpack_amd import framing, zstd  # noqa: E402
from tests.golden.q8_cases import CASES, case_file, group_of  # noqa: E402


def _exec_module(path, ns):
    src = open(path).read()
    for node in ast.parse(src).body:
        if isinstance(node, (ast.Import, ast.ImportFrom)):
            continue
        exec(compile(ast.Module([node], []), path, "exec"), ns)


def load():
    from seedpack import cpu as cp
    from seedpack import detmath
    ns = {"np": np, "cp": cp, "detmath": detmath, "json": json, "lzma": lzma, "struct": struct,
          "ThreadPoolExecutor": ThreadPoolExecutor, "pack": framing.pack, "unpack": framing.unpack,
          "zstd_c": zstd.zstd_c, "zstd_d": zstd.decompress, "group_of": group_of, "GGUF": None, "GGML_Q8_0": 8,
          "__name__": "gpu_ref"}
    _exec_module(os.path.join(REF, "seedpack", "gpu2.py"), ns)
    _exec_module(os.path.join(REF, "seedpack", "gpu3.py"), ns)
    return ns


def main():
    ns = load()
    out = {}
    for name, tensors, opts in CASES:
        data, layout, opts = case_file(name)
        if "stat_elems" in opts:
            ns["STAT_ELEMS"] = opts["stat_elems"]
        budget = opts.get("part_bytes", 1 << 30)
        groups, cur, size = [], [], 0
        for i, (_, nb, _, _) in enumerate(layout["t"]):
            if cur and size + nb > budget:
                groups.append(cur)
                cur, size = [], 0
            cur.append(i)
            size += nb
        groups.append(cur)
        check = np.frombuffer(data, np.uint8).copy()
        for k, idx in enumerate(groups):
            codec = ns["M22Fast"]()
            buf = codec.compress(data, tensors=idx, header=False, parsed=(layout, None))
            dec = ns["M22Fast"]().decompress(buf, out=np.zeros(len(data), np.uint8))
            for i in idx:
                o, nb = layout["t"][i][:2]
                assert (dec[o:o + nb] == check[o:o + nb]).all(), f"{name}: the reference does not round-trip"
            out[f"{name}/p{k}"] = np.frombuffer(buf, np.uint8)
            parts = framing.unpack(buf)
            print(f"{name} part {k}: tensors {idx}, {len(buf)} B for {sum(layout['t'][i][1] for i in idx)} B; "
                  f"parts {[(p, len(v)) for p, v in parts.items()]}", flush=True)
        out[f"{name}/groups"] = np.array([len(g) for g in groups], np.int64)
        ns["STAT_ELEMS"] = 32 << 20
    np.savez_compressed(os.path.join(HERE, "q8_vectors.npz"), **out)


if __name__ == "__main__":
    main()
