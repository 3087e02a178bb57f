"""Writes golden vectors for the QR coder's other seeds by running the reference's own QR kernels
(seedpack/qr.py KERNELS) through the reference's --cpu backend, as make_qr_golden.py does. Run in
the build container only:

    python tests/golden/make_qr_seed_golden.py

Output: tests/golden/qr_seed_vectors.npz (data only). Cases:
  * no seed (seed type 98): a tensor coded against template blocks (the rounded mean of each block
    field over the rows, qr.py:1116-1136 -- built here with the reference's block_fields /
    blocks_from_fields kernels) with its per-column RMS as the seed;
  * explicit seeds (99): float32 (value, uncertainty) pairs, some uncertainties zero;
  * quantized seeds (a Q8_0 / Q6_K / Q4_K / IQ4_XS tensor): the prediction is the target type's
    quantization of the seed's dequantized values (the seeds path, seed.py:1-10);
  * the per-weight kernels intervals, grid_h, weq and block_fields on every type they serve.
The column RMS and dequantized values come from the reference's C library (oracle/_ref) and
in-order float64 sums, the quantizations from oracle/_ref.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.golden import make_qr_golden as base  # noqa: E402  (sets up the reference's --cpu backend)
from tests.golden.qr_seed_cases import SELF_CASES, EXPLICIT_CASES, QSEED_CASES, AUX_TYPES, GRID_AUX_TYPES, inputs  # noqa: E402
from oracle import ref as qref  # noqa: E402

BS, QK = base.BS, base.QK
NF = {2: 1, 6: 1, 8: 1, 20: 1, 42: 1, 3: 2, 7: 2, 10: 34, 11: 17, 14: 17, 12: 18, 13: 18, 23: 9,
      16: 9, 18: 9, 19: 9, 21: 9, 17: 17, 22: 17, 29: 17}


def encode(mod, normalize, T, F, P, seed, seed_type, cols, mv=2):
    """make_qr_golden.encode with the seed type as a parameter"""
    tm, sg, nb = base.layout(T, [len(F) // BS[T]])
    tm["seed_off"] = 0
    tm["seed_type"] = seed_type
    tm["cols"] = cols
    tm["imx_off"] = -1
    gk = base.grid_keys(T)
    imx = np.zeros(1, np.float32)
    smem = 0 if T not in base.GRID_TAB else 64 * 4 * (128 if T in (18, 21) else 64)
    nseg = len(sg)
    counts = np.zeros((base.NTAB2, 256), np.uint32)
    grid = ((nseg + 63) // 64,)
    tmb, sgb = tm.view(np.uint8), sg.view(np.uint8)
    mod.get_function("qr_hist")(grid, (64,), (np.int32(T), F, P, seed, tmb, sgb, np.int32(nseg), counts, gk, imx,
                                              np.int32(mv)), shared_mem=smem)
    freq, used = normalize(counts)
    remap = np.full(base.NTAB2, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    cum = np.zeros((len(freq), 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    cap = base.seg_blocks(T) * (3 * BS[T] if T in base.GRID_TAB else (QK[T] + base.NSB_MAX) * 2) + 1024
    out = np.zeros(nseg * cap, np.uint8)
    out_len = np.zeros(nseg, np.uint32)
    mod.get_function("qr_enc")(grid, (64,), (np.int32(T), F, P, seed, tmb, sgb, np.int32(nseg), remap, freq, cum,
                                             out, np.uint64(cap), out_len, gk, imx, np.int32(mv)), shared_mem=smem)
    assert not (out_len == 0xFFFFFFFF).any()
    stream = b"".join(out[(s + 1) * cap - out_len[s]:(s + 1) * cap].tobytes() for s in range(nseg))
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


def block_fields(mod, T, F):
    nblk = len(F) // BS[T]
    out = np.zeros(nblk * NF[T], np.int32)
    mod.get_function("block_fields")(((nblk + 255) // 256,), (256,), (np.int32(T), F, np.int64(nblk), out))
    return out


def template(mod, T, F, rows, cols):
    """the reference's self_side template blocks (qr.py:1126-1134)"""
    nb_row = cols // QK[T]
    fl = block_fields(mod, T, F).reshape(rows, nb_row, NF[T])
    v = np.rint(fl.astype(np.float64).mean(0)).astype(np.int32)
    tpl = np.zeros(nb_row * BS[T], np.uint8)
    mod.get_function("blocks_from_fields")(((nb_row + 31) // 32,), (32,), (np.int32(T), v, np.int32(nb_row), tpl))
    return tpl


def colrms(T, F, rows, cols):
    x = qref.dequantize(T, F.tobytes(), rows * cols).reshape(rows, cols).astype(np.float64)
    z = np.zeros((1, cols))
    s = np.add.accumulate(np.concatenate([z, x * x], 0), axis=0)[-1]
    return np.sqrt((s / rows).astype(np.float32)).astype(np.float16)


def main():
    mod, normalize = base.load()
    out = {}
    for k, (name, T, rows, cols) in enumerate(SELF_CASES):
        x, imx = inputs("self", k, rows, cols)
        F = qref.quantize(T, x, imx)
        tpl = template(mod, T, F, rows, cols)
        rms = colrms(T, F, rows, cols)
        P = np.tile(tpl, rows)
        res = encode(mod, normalize, T, F, P, rms.astype(np.float32).view(np.uint8).copy(), 98, cols)
        out.update({f"self_{name}/F": F, f"self_{name}/tpl": tpl, f"self_{name}/rms": rms.view(np.uint16)})
        out.update({f"self_{name}/{kk}": v for kk, v in res.items()})
        print(f"self {name}: stream {len(res['stream'])} B of {len(F)}", flush=True)
    for k, (name, T, rows, cols) in enumerate(EXPLICIT_CASES):
        x, imx = inputs("explicit", k, rows, cols)
        g = np.random.Generator(np.random.PCG64(0xE5 + k))
        F = qref.quantize(T, x, imx)
        xs = (x + g.normal(0, 0.003, x.shape)).astype(np.float32)
        P = qref.quantize(T, xs, imx)
        h = np.abs(g.normal(0, 0.004, x.shape)).astype(np.float32)
        h[g.random(x.shape) < 0.1] = 0
        seed = np.stack([xs.reshape(-1), h.reshape(-1)], 1).astype(np.float32).reshape(-1)
        res = encode(mod, normalize, T, F, P, seed.view(np.uint8).copy(), 99, cols)
        out.update({f"explicit_{name}/F": F, f"explicit_{name}/P": P, f"explicit_{name}/seed": seed})
        out.update({f"explicit_{name}/{kk}": v for kk, v in res.items()})
        print(f"explicit {name}: stream {len(res['stream'])} B", flush=True)
    for k, (name, T, S, rows, cols) in enumerate(QSEED_CASES):
        x, imx = inputs("qseed", k, rows, cols)
        Sb = qref.quantize(S, x, imx)                       # the seed file's tensor
        xd = qref.dequantize(S, Sb.tobytes(), rows * cols).reshape(rows, cols)
        P = qref.quantize(T, xd, imx)                       # the prediction from the seed
        g = np.random.Generator(np.random.PCG64(0x5EED + k))
        F = base.perturb(qref.quantize(T, x, imx), BS[T], g, 0.02)
        res = encode(mod, normalize, T, F, P, Sb.copy(), S, cols)
        out.update({f"qseed_{name}/F": F, f"qseed_{name}/P": P, f"qseed_{name}/seed": Sb})
        out.update({f"qseed_{name}/{kk}": v for kk, v in res.items()})
        print(f"qseed {name}: stream {len(res['stream'])} B", flush=True)
    for T in AUX_TYPES:
        x, imx = inputs("aux", T, 8, 512)
        F = qref.quantize(T, x, imx)
        F[::7] ^= 0x55                                      # odd codes and scales too
        nw = 8 * 512
        lo, hi = np.zeros(nw, np.float32), np.zeros(nw, np.float32)
        mod.get_function("intervals")(((nw + 255) // 256,), (256,), (np.int32(T), F, np.int64(nw), lo, hi))
        P = F.copy()
        P[::5] ^= 0x0F
        weq = np.zeros(nw, np.uint8)
        mod.get_function("weq")(((nw + 255) // 256,), (256,), (np.int32(T), F, P, np.int64(nw), weq))
        out.update({f"aux_{T}/F": F, f"aux_{T}/P": P, f"aux_{T}/lo": lo, f"aux_{T}/hi": hi, f"aux_{T}/weq": weq,
                    f"aux_{T}/fields": block_fields(mod, T, F)})
    for T in GRID_AUX_TYPES:
        x, imx = inputs("aux", T, 4, 512)
        F = qref.quantize(T, x, imx)
        nw = 4 * 512
        h = np.zeros(nw, np.float32)
        mod.get_function("grid_h")(((nw + 255) // 256,), (256,), (np.int32(T), F, np.int64(nw), h))
        out.update({f"grid_{T}/F": F, f"grid_{T}/h": h})
    np.savez_compressed(os.path.join(HERE, "qr_seed_vectors.npz"), **out)


if __name__ == "__main__":
    main()
