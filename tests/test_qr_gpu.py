"""HIP QR coder vs the reference's own QR kernels (golden vectors) and round trips (MI355X)."""
import os
import sys

import numpy as np
import pytest

from oracle import qr as oqr
from seedpack_amd import device as dev
from seedpack_amd import qr, synth
from seedpack_amd.gpuquant import GPUQuant
from tests.golden.qr_cases import CASES, GRID
from tests.test_oracle_qr import case_grid, case_inputs

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def vectors():
    return np.load(os.path.join(ROOT, "tests", "golden", "qr_vectors.npz"))


def _imx(name):
    """(device imatrix, its offset) of a grid case; (None, -1) otherwise"""
    imx, _ = case_grid(name)
    return (None, -1) if imx is None else (dev.DeviceArray.from_host(imx), 0)


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_hip_qr_encode_matches_reference(vectors, name):
    T, cols, F, P, seed = case_inputs(vectors, name)
    say("case qr encode", name)
    sd = dev.DeviceArray.from_host(seed)
    imx, off = _imx(name)
    res = qr.encode_parts(T, [(F, P, 0, 30, cols, off)], sd, imx)
    assert np.array_equal(res["counts"], vectors[f"{name}/counts"]), "histogram"
    assert np.array_equal(res["used"], vectors[f"{name}/used"])
    assert np.array_equal(res["freq"], vectors[f"{name}/freq"])
    assert np.array_equal(res["lens"], vectors[f"{name}/lens"]), "segment lengths"
    assert res["stream"].tobytes() == vectors[f"{name}/stream"].tobytes(), "stream bytes"


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_hip_qr_decodes_reference_stream(vectors, name):
    T, cols, F, P, seed = case_inputs(vectors, name)
    say("case qr decode", name)
    sd = dev.DeviceArray.from_host(seed)
    imx, off = _imx(name)
    out = qr.decode_parts(T, vectors[f"{name}/freq"], vectors[f"{name}/used"], vectors[f"{name}/lens"],
                          vectors[f"{name}/stream"].tobytes(), [(P, 0, 30, cols, off)], sd, imx)
    got = out.to_host()[:len(F)]
    bad = np.flatnonzero(got != F)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


@pytest.mark.parametrize("T", [8, 2])
def test_hip_qr_cfg1_full_size(T):
    """configuration 1: the 3072x1024 tensor, Q8_0 / Q4_0 without imatrix, file = prediction with 1%
    of blocks perturbed; the stream equals the oracle's and decodes back to the file"""
    w, _ = synth.tensor(1, 0)
    g = np.random.Generator(np.random.PCG64(1234 + T))
    say("case qr cfg1", T)
    P = GPUQuant().quantize_tensors(T, [(w.reshape(-1), w.shape[1])], [None])[0]
    Fb = P.copy().reshape(-1, qr.BS[T])
    idx = g.choice(len(Fb), size=len(Fb) // 100, replace=False)
    Fb[idx, g.integers(0, qr.BS[T], len(idx))] ^= np.uint8(0x10)
    F = Fb.reshape(-1)
    sd = dev.DeviceArray.from_host(w.reshape(-1).view(np.uint8))
    res = qr.encode_parts(T, [(F, P, 0, 30, w.shape[1], -1)], sd)
    want = oqr.encode(T, F.tobytes(), P.tobytes(), w.reshape(-1).view(np.uint8).tobytes(), 30, w.shape[1])
    assert res["stream"].tobytes() == want["stream"].tobytes()
    assert np.array_equal(res["lens"], want["lens"])
    buf = qr.encode(T, [(F, P, 0, 30, w.shape[1], -1)], sd)
    back = qr.decode(T, buf, [(P, 0, 30, w.shape[1], -1)], sd).to_host()[:len(F)]
    assert back.tobytes() == F.tobytes()


def test_hip_qr_multi_tensor_batch_round_trip(vectors):
    """two tensors in one batch (segments never span tensors; seed offsets per tensor)"""
    names = ["q4_k_drift", "q4_k_var"]
    ins = [case_inputs(vectors, n) for n in names]
    seeds = [i[4] for i in ins]
    off = [0, (len(seeds[0]) + 255) // 256 * 256]
    seed = np.zeros(off[1] + len(seeds[1]), np.uint8)
    seed[:len(seeds[0])] = seeds[0]
    seed[off[1]:] = seeds[1]
    sd = dev.DeviceArray.from_host(seed)
    items = [(F, P, o, 30, cols, -1) for (T, cols, F, P, _), o in zip(ins, off)]
    buf = qr.encode(12, items, sd)
    out = qr.decode(12, buf, [(P, o, 30, cols, -1) for (T, cols, F, P, _), o in zip(ins, off)], sd).to_host()
    want = np.concatenate([i[2] for i in ins])
    assert out[:len(want)].tobytes() == want.tobytes()


@pytest.mark.parametrize("T", sorted(GRID))
def test_hip_qr_grid_cfg3_rows(T):
    """configuration-3 rows (256 x 12288 Student-t, imatrix) of every grid type: prediction = the HIP
    quantizer's bytes, file = 2% of its blocks perturbed; the stream equals the oracle's and decodes
    back to the file; a second file from drifted weights round-trips too"""
    w, imx = synth.tensor(3, 0, rows=256)
    say("case qr grid cfg3", T)
    gq = GPUQuant()
    P = gq.quantize_tensors(T, [(w.reshape(-1), w.shape[1])], [imx])[0]
    g = np.random.Generator(np.random.PCG64(4321 + T))
    Fb = P.copy().reshape(-1, qr.BS[T])
    idx = g.choice(len(Fb), size=len(Fb) // 50, replace=False)
    Fb[idx, g.integers(0, qr.BS[T], len(idx))] ^= np.uint8(0x21)
    F = Fb.reshape(-1)
    sd = dev.DeviceArray.from_host(w.reshape(-1).view(np.uint8))
    dimx = dev.DeviceArray.from_host(imx)
    item = (F, P, 0, 30, w.shape[1], 0)
    res = qr.encode_parts(T, [item], sd, dimx)
    want = oqr.encode(T, F.tobytes(), P.tobytes(), w.reshape(-1).view(np.uint8).tobytes(), 30, w.shape[1],
                      imx=imx, gk=qr.grid_keys(T))
    assert np.array_equal(res["counts"], want["counts"]), "histogram"
    assert np.array_equal(res["lens"], want["lens"])
    assert res["stream"].tobytes() == want["stream"].tobytes()
    buf = qr.encode(T, [item], sd, dimx)
    back = qr.decode(T, buf, [(P, 0, 30, w.shape[1], 0)], sd, dimx).to_host()[:len(F)]
    assert back.tobytes() == F.tobytes()
    # drift: most blocks differ
    x = synth.bf16_to_f32(w).reshape(w.shape)
    x2 = (x + g.normal(0, 0.002, x.shape)).astype(np.float32)
    F2 = gq.quantize_tensors(T, [(x2.reshape(-1), w.shape[1])], [imx])[0]
    buf = qr.encode(T, [(F2, P, 0, 30, w.shape[1], 0)], sd, dimx)
    back = qr.decode(T, buf, [(P, 0, 30, w.shape[1], 0)], sd, dimx).to_host()[:len(F2)]
    assert back.tobytes() == F2.tobytes()


def test_hip_lut32_folds_freq_and_cum_into_the_symbol_table():
    """the QR decoders' LUT32 entry of every slot names the symbol of the byte LUT, that symbol's
    frequency - 1 and the slot's offset in its range, on tables with zero-frequency symbols, one
    symbol holding every slot and runs of frequency-1 symbols"""
    from seedpack_amd._lib import check, lib
    g = np.random.Generator(np.random.PCG64(5))
    freq = np.zeros((5, 256), np.int64)
    freq[0, 3] = 4096
    freq[1, :100] = 1; freq[1, 200] = 4096 - 100
    freq[2, ::2] = 32
    freq[3] = 16
    p = g.dirichlet(np.full(256, 0.1)); f = np.floor(p * (4096 - 256)).astype(np.int64) + 1
    f[np.argmax(f)] += 4096 - f.sum(); freq[4] = f
    assert (freq.sum(1) == 4096).all()
    cum = np.zeros((5, 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq, 1)
    cum_d = dev.DeviceArray.from_host(cum)
    l8, l32 = dev.DeviceArray((5, 4096), np.uint8), dev.DeviceArray((5, 4096), np.uint32)
    check(lib().spa_rans_build_lut(cum_d.ptr, 5, l8.ptr, None))
    check(lib().spa_rans_build_lut32(cum_d.ptr, 5, l32.ptr, None))
    a, e = l8.to_host().astype(np.int64), l32.to_host().astype(np.int64)
    slots = np.arange(4096)
    for t in range(5):
        sym = e[t] & 255
        assert np.array_equal(sym, a[t]), t
        assert np.array_equal(((e[t] >> 8) & 4095) + 1, freq[t][sym]), t
        assert np.array_equal(e[t] >> 20, slots - cum[t][sym]), t
