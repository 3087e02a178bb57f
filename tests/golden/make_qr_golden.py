"""Writes QR-coder golden vectors by running the reference's own QR kernels (seedpack/qr.py KERNELS)
through the reference's own --cpu backend (seedpack/cpukernels.py: the CUDA text compiled as host
C++ with -ffp-contract=off, launches run on host threads). Run in the build container only:

    python tests/golden/make_qr_golden.py

Nothing here runs on the GPU box or at test time: the output is data (qr_vectors.npz).

The kernel text is read from qr.py with `ast` (qr.py itself imports zstandard and numba, which are
absent); `normalize` (qr.py:904-923) is taken the same way and run on numpy. The host-side steps of
qr.encode/decode (qr.py:957-968 _layout, :1007-1090) are restated below, minus the zstd framing.
Inputs: seeded BF16 tensors (seed type 30), predictions P = the reference quantizer's bytes
(oracle/_ref), files F = P with 1% of blocks perturbed (one byte or nibble changed), as in
BASELINE.json configs[0].
"""
import ast
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, ROOT)

os.environ["SEEDPACK_CPU"] = "1"
# the reference's --cpu backend caches its compiled kernels; a temporary directory keeps them out of
# the repository
os.environ.setdefault("SEEDPACK_CACHE", tempfile.mkdtemp(prefix="seedpack_refcache_"))
sys.path.insert(0, REF)

from oracle import ref as qref  # noqa: E402
from seedpack_amd import synth  # noqa: E402
from tests.golden.qr_cases import CASES, case_seed  # noqa: E402


def _qr_source():
    src = open(os.path.join(REF, "seedpack", "qr.py")).read()
    tree = ast.parse(src)
    out = {}
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "KERNELS" for t in node.targets):
            out["KERNELS"] = ast.literal_eval(node.value)
        if isinstance(node, ast.FunctionDef) and node.name == "normalize":
            out["normalize"] = ast.get_source_segment(src, node)
    return out


class _NP:
    """the two CuPy calls normalize() makes, on numpy"""
    asnumpy = staticmethod(np.asarray)
    asarray = staticmethod(np.asarray)


def load():
    from seedpack import cpukernels
    s = _qr_source()
    ns = {"np": np, "cp": _NP, "PB": 12}
    exec(s["normalize"], ns)
    mod = cpukernels.RawModule(code=s["KERNELS"], options=("-std=c++17", "--fmad=false"))
    return mod, ns["normalize"]


TM_DT = np.dtype([("blk0", "<i8"), ("seed_off", "<i8"), ("seed_type", "<i4"), ("cols", "<i4"), ("imx_off", "<i8")])
SG_DT = np.dtype([("t", "<i4"), ("nb", "<i4"), ("b0", "<i8")])
QK = {2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 20: 32, 42: 64, 10: 256, 11: 256, 12: 256, 13: 256, 14: 256, 23: 256,
      16: 256, 17: 256, 18: 256, 19: 256, 21: 256, 22: 256, 29: 256}
BS = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 20: 18, 42: 18, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 23: 136,
      16: 66, 17: 74, 18: 98, 19: 50, 21: 110, 22: 82, 29: 56}
GRID_TAB = {16: "iq2_data_0", 17: "iq2_data_1", 19: "iq2_data_2", 29: "iq2_data_2", 22: "iq2_data_3",
            18: "iq3_data_0", 21: "iq3_data_1"}


def grid_keys(T):
    """uint16 per grid point: its levels (grid byte - 1) / 2, 2 bits each (IQ3: 3 bits), as the
    reference's qr.grid_keys builds them from its table fixture"""
    if T not in GRID_TAB:
        return np.zeros(1, np.uint16)
    tb = np.load(os.path.join(REF, "seedpack", "ggml", "iqtables.npz"))
    g = tb[GRID_TAB[T] + "_grid"]
    n, bits = (8, 2) if g.dtype == np.uint64 else (4, 3)
    lev = np.stack([((g >> np.array(8 * i, g.dtype)) & np.array(255, g.dtype)).astype(np.int64) for i in range(n)], 1)
    return (((lev - 1) // 2) << (bits * np.arange(n))).sum(1).astype(np.uint16)
NSB_MAX, NTAB2 = 20, 20 + 64 + 2 + 208


def seg_blocks(T):
    return max(16, 16384 // QK[T])


def layout(T, nblocks):
    sb = seg_blocks(T)
    tm = np.zeros(len(nblocks), TM_DT)
    segs, b0 = [], 0
    for i, nb in enumerate(nblocks):
        tm[i]["blk0"] = b0
        for o in range(0, nb, sb):
            segs.append((i, min(sb, nb - o), b0 + o))
        b0 += nb
    return tm, np.array(segs, SG_DT), b0


def perturb(P, bs, g, frac=0.01):
    F = P.copy().reshape(-1, bs)
    nb = len(F)
    idx = g.choice(nb, size=max(1, int(round(nb * frac))), replace=False)
    for b in idx:
        j = int(g.integers(0, bs))
        if g.random() < 0.5:
            F[b, j] ^= np.uint8(1 << int(g.integers(0, 8)))                 # one bit
        else:
            F[b, j] = np.uint8((F[b, j] & 0xF0) | int(g.integers(0, 16)))    # one nibble
    return F.reshape(-1)


def encode(mod, normalize, T, F, P, seed, cols, mv=2, imx=None):
    """qr.py:1007-1061 without the zstd framing -> dict of the coded parts"""
    tm, sg, nb = layout(T, [len(F) // BS[T]])
    tm["seed_off"] = 0
    tm["seed_type"] = 30
    tm["cols"] = cols
    tm["imx_off"] = -1 if imx is None else 0
    gk = grid_keys(T)
    imx = np.zeros(1, np.float32) if imx is None else np.ascontiguousarray(imx, np.float32)
    smem = 0 if T not in GRID_TAB else 64 * 4 * (128 if T in (18, 21) else 64)
    nseg = len(sg)
    counts = np.zeros((NTAB2, 256), np.uint32)
    grid = ((nseg + 63) // 64,)
    tmb, sgb = tm.view(np.uint8), sg.view(np.uint8)
    mod.get_function("qr_hist")(grid, (64,), (np.int32(T), F, P, seed, tmb, sgb, np.int32(nseg), counts, gk, imx,
                                              np.int32(mv)), shared_mem=smem)
    freq, used = normalize(counts)
    remap = np.full(NTAB2, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    cum = np.zeros((len(freq), 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    cap = seg_blocks(T) * (3 * BS[T] if T in GRID_TAB else (QK[T] + NSB_MAX) * 2) + 1024
    out = np.zeros(nseg * cap, np.uint8)
    out_len = np.zeros(nseg, np.uint32)
    mod.get_function("qr_enc")(grid, (64,), (np.int32(T), F, P, seed, tmb, sgb, np.int32(nseg), remap, freq, cum,
                                             out, np.uint64(cap), out_len, gk, imx, np.int32(mv)), shared_mem=smem)
    assert not (out_len == 0xFFFFFFFF).any()
    stream = b"".join(out[(s + 1) * cap - out_len[s]:(s + 1) * cap].tobytes() for s in range(nseg))
    # decode back (qr.py:1064-1090)
    lut = np.zeros((len(freq), 1 << 12), np.uint8)
    mod.get_function("build_lut")((len(freq),), (256,), (cum, np.int32(len(freq)), lut))
    offs = np.zeros(nseg, np.uint64)
    offs[1:] = np.cumsum(out_len.astype(np.uint64))[:-1]
    Fd = np.zeros(nb * BS[T], np.uint8)
    mod.get_function("qr_dec")(grid, (64,), (np.int32(T), np.frombuffer(stream, np.uint8).copy(), offs, P, seed, tmb, sgb,
                                             np.int32(nseg), remap, freq, cum, lut, Fd, gk, imx, np.int32(mv)),
                               shared_mem=smem)
    assert Fd.tobytes() == F.tobytes(), "reference decode does not round-trip"
    return {"counts": counts, "freq": freq, "used": used.astype(np.int32), "lens": out_len,
            "stream": np.frombuffer(stream, np.uint8)}


def main():
    mod, normalize = load()
    out = {}
    for k, (name, T, rows, cols, dist, use_imx, how) in enumerate(CASES):
        g, w, imx = case_seed(k)
        x = synth.bf16_to_f32(w).reshape(rows, cols)
        P = qref.quantize(T, x, imx)
        if how == "perturb":
            F = perturb(P, BS[T], g)
        elif how == "drift":        # the file was made from slightly different weights
            x2 = (x + g.normal(0, 0.002, x.shape)).astype(np.float32)
            F = qref.quantize(T, x2, imx)
        else:                       # the file used the imatrix, the prediction did not
            F = P
            P = qref.quantize(T, x, None)
        res = encode(mod, normalize, T, F, P, w.reshape(-1).view(np.uint8).copy(), cols,
                     imx=imx if T in GRID_TAB else None)
        out[f"{name}/T"] = np.array([T, rows, cols, k], np.int64)
        out[f"{name}/seed_sha"] = np.frombuffer(__import__("hashlib").sha256(w.tobytes()).digest(), np.uint8)
        out[f"{name}/P"] = P
        out[f"{name}/FxP"] = F ^ P
        for kk, v in res.items():
            out[f"{name}/{kk}"] = v
        print(f"{name}: {len(F)} bytes, {int((F != P).sum())} differ, stream {len(res['stream'])} B, "
              f"{len(res['lens'])} segments, {len(res['used'])} tables", flush=True)
    np.savez_compressed(os.path.join(HERE, "qr_vectors.npz"), **out)


if __name__ == "__main__":
    main()
