"""Writes M24 (method m28's BF16 codec) golden vectors by running the reference's own code on the CPU:
its bf_hist / bf_enc / bf_dec kernels (seedpack/gpu_bf16.py KERNELS) through the reference's --cpu
backend, gpu2.normalize_gpu for the tables, and the side-information steps of
M24BF16GPU.compress_dev (gpu_bf16.py:352-371) with the reference's detmath module. Run in the build
container only:

    python tests/golden/make_m24_golden.py

The driver steps (statistics per tensor, histogram, normalisation, encode, gather) are restated
below without the GGUF parsing and header coding; the inputs are the R2 golden files
(tests/golden/r2_cases.py). Output: tests/golden/m24_vectors.npz (data only).
"""
import ast
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.golden import make_r2_golden as r2g  # noqa: E402  (sets up the reference's --cpu backend)
from tests.golden.r2_cases import CASES, case_file  # noqa: E402

REF = r2g.REF


def load():
    from seedpack import cpu as cp
    from seedpack import cpukernels, detmath
    src, tree = r2g._source(os.path.join(REF, "seedpack", "gpu_bf16.py"))
    ns = {"np": np, "cp": cp, "detmath": detmath}
    kernels = None
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "KERNELS" for t in node.targets):
            kernels = ast.literal_eval(node.value.left) % {"SEG": 16384, "SEGQ": 512}
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) in ("TB_DT", "SG_DT", "SEG", "TPT")
                                                for t in node.targets):
            exec(ast.get_source_segment(src, node), ns)
    gsrc, gtree = r2g._source(os.path.join(REF, "seedpack", "gpu2.py"))
    for node in gtree.body:
        if isinstance(node, ast.FunctionDef) and node.name == "normalize_gpu":
            g2 = {"np": np, "cp": cp, "PB": 12}                 # gpu2.py:34
            exec(ast.get_source_segment(gsrc, node), g2)
            ns["normalize_gpu"] = g2["normalize_gpu"]
    mod = cpukernels.RawModule(code=kernels, options=("-std=c++17",))
    ns["kern"] = mod.get_function
    return ns, cp


def side(ns, cp, data, layout):
    """M24BF16GPU.compress_dev's statistics loop (gpu_bf16.py:352-369)"""
    detmath = ns["detmath"]
    rfi_l, cfi_l, sc_l = [], [], []
    host = np.frombuffer(data, np.uint8)
    for off, nbytes, rowlen, _ in layout["t"]:
        u = cp.asarray(host[off:off + nbytes].copy()).view(cp.uint16).reshape(-1, rowlen)
        w = (u.astype(cp.uint32) << 16).view(cp.float32)
        nr = w.shape[0]
        rf = detmath.log2(cp.sqrt(detmath.rows(w, True) / rowlen) + 1e-30)
        wn = w / detmath.exp2(rf).astype(cp.float32)[:, None]
        cf = detmath.log2(cp.sqrt(detmath.cols(wn, True) / nr) + 1e-30)
        rfi = cp.clip(cp.rint(rf * 4), -32768, 32767).astype(cp.int16)
        cfi = cp.clip(cp.rint(cf * 4), -32768, 32767).astype(cp.int16)
        bias = (detmath.cols(wn) / nr) / detmath.exp2(cfi.astype(cp.float64) / 4)
        rfi_l.append(np.asarray(rfi)); cfi_l.append(np.asarray(cfi))
        sc_l.append(np.asarray(cp.clip(cp.floor(bias * 16) + 8, 0, 15).astype(cp.int8)))
    return np.concatenate(rfi_l), np.concatenate(cfi_l), np.concatenate(sc_l)


def tables(ns, layout):
    """M24BF16GPU._tables (gpu_bf16.py:332-342)"""
    tb = np.zeros(len(layout["t"]), ns["TB_DT"]); segs = []
    rowbase = colbase = 0
    for i, (off, nbytes, rowlen, _) in enumerate(layout["t"]):
        n = nbytes // 2
        tb[i] = (off, rowlen, rowbase, colbase, i * ns["TPT"])
        for i0 in range(0, n, ns["SEG"]):
            segs.append((i, min(ns["SEG"], n - i0), i0))
        rowbase += n // rowlen; colbase += rowlen
    return tb, np.array(segs, ns["SG_DT"])


def main():
    ns, cp = load()
    out = {}
    for name, _, _ in CASES:
        data, lay, _ = case_file(name)
        layout = {"size": lay["size"], "t": lay["t"]}
        rfi, cfi, scl = side(ns, cp, data, layout)
        tb, sg = tables(ns, layout)
        dev = np.frombuffer(data, np.uint8).copy()
        args = (dev, tb.view(np.uint8), sg.view(np.uint8), np.int32(len(sg)), rfi, cfi, scl)
        counts = np.zeros((len(tb) * ns["TPT"], 256), np.uint32)
        ns["kern"]("bf_hist")(((len(sg) + 63) // 64,), (64,), args + (counts,))
        freq, used = ns["normalize_gpu"](cp.asarray(counts))
        freq, used = np.asarray(freq), np.asarray(used)
        remap = np.full(counts.shape[0], -1, np.int32); remap[used] = np.arange(len(used), dtype=np.int32)
        cum = np.zeros((len(freq), 257), np.uint32); cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
        cap = 16384 * 2 + 1024
        o = np.zeros(len(sg) * cap, np.uint8); ln = np.zeros(len(sg), np.uint32)
        ns["kern"]("bf_enc")(((len(sg) + 63) // 64,), (64,), args + (remap, freq, cum, o, np.uint64(cap), ln))
        assert not (ln == 0xFFFFFFFF).any()
        stream = b"".join(o[(s + 1) * cap - ln[s]:(s + 1) * cap].tobytes() for s in range(len(sg)))
        # decode back with the reference's bf_dec
        lut = np.zeros((len(freq), 1 << 12), np.uint8)
        for t in range(len(freq)):
            lut[t] = np.repeat(np.arange(256, dtype=np.uint8), freq[t].astype(np.int64))
        offs = np.zeros(len(sg), np.uint64); offs[1:] = np.cumsum(ln.astype(np.uint64))[:-1]
        back = np.zeros(len(data), np.uint8)
        ns["kern"]("bf_dec")(((len(sg) + 63) // 64,), (64,),
                             (np.frombuffer(stream, np.uint8).copy(), offs, back, tb.view(np.uint8), sg.view(np.uint8),
                              np.int32(len(sg)), rfi, cfi, scl, remap, freq, cum, lut))
        for off, nb, _, _ in layout["t"]:
            assert back[off:off + nb].tobytes() == data[off:off + nb], "reference decode does not round-trip"
        out.update({f"{name}/rfi": rfi, f"{name}/cfi": cfi, f"{name}/scl": scl, f"{name}/counts": counts,
                    f"{name}/freq": freq, f"{name}/used": used.astype(np.int32), f"{name}/lens": ln,
                    f"{name}/stream": np.frombuffer(stream, np.uint8)})
        print(f"{name}: {len(sg)} segments, stream {len(stream)} B of {sum(t[1] for t in layout['t'])}", flush=True)
    np.savez_compressed(os.path.join(HERE, "m24_vectors.npz"), **out)


if __name__ == "__main__":
    main()
