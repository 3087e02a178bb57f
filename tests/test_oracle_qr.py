"""The QR oracle against the reference's own QR kernels (golden vectors from its --cpu backend)."""
import hashlib
import os

import numpy as np
import pytest

from oracle import qr as oqr
from tests.golden.qr_cases import CASES, GRID, case_seed

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def vectors():
    return np.load(os.path.join(ROOT, "tests", "golden", "qr_vectors.npz"))


def case_inputs(vectors, name):
    T, rows, cols, k = (int(v) for v in vectors[f"{name}/T"])
    _, w, _ = case_seed(k)
    assert hashlib.sha256(w.tobytes()).digest() == vectors[f"{name}/seed_sha"].tobytes()
    P = vectors[f"{name}/P"]
    F = P ^ vectors[f"{name}/FxP"]
    return T, cols, F, P, w.reshape(-1).view(np.uint8)


def case_grid(name):
    """(imatrix, grid keys) the grid-type cases are coded with; (None, None) for the others"""
    k = [c[0] for c in CASES].index(name)
    if CASES[k][1] not in GRID:
        return None, None
    from seedpack_amd.qr import grid_keys
    return case_seed(k)[2], grid_keys(CASES[k][1])


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_oracle_qr_matches_reference_kernels(vectors, name):
    T, cols, F, P, seed = case_inputs(vectors, name)
    imx, gk = case_grid(name)
    res = oqr.encode(T, F.tobytes(), P.tobytes(), seed.tobytes(), 30, cols, imx=imx, gk=gk)
    assert np.array_equal(res["counts"], vectors[f"{name}/counts"]), "histogram"
    assert np.array_equal(res["used"], vectors[f"{name}/used"]), "used tables"
    assert np.array_equal(res["freq"], vectors[f"{name}/freq"]), "normalised frequencies"
    assert np.array_equal(res["lens"], vectors[f"{name}/lens"]), "segment lengths"
    assert res["stream"].tobytes() == vectors[f"{name}/stream"].tobytes(), "stream bytes"


def test_normalize_invariants():
    g = np.random.default_rng(3)
    c = np.zeros((5, 256), np.uint32)
    c[0, 0] = 10 ** 7; c[0, 1:200] = 1                      # one dominant symbol, many rare ones
    c[1, :] = g.integers(0, 50, 256)
    c[3, 7] = 1
    f, used = oqr.normalize(c)
    assert list(used) == [0, 1, 3]
    assert (f.astype(np.int64).sum(1) == 4096).all()
    assert ((c[used] > 0) <= (f > 0)).all()
    assert f[2, 7] == 4096


def test_rans_round_trip_textbook():
    """encode with the oracle coder, decode with an independent textbook byte-wise rANS decoder"""
    g = np.random.default_rng(9)
    counts = np.zeros((oqr.NTAB2, 256), np.uint32)
    seq = [(int(t), int(s)) for t, s in zip(g.integers(0, 3, 5000), np.minimum(255, g.geometric(0.3, 5000)))]
    for t, s in seq:
        counts[t, s] += 1
    freq, used = oqr.normalize(counts)
    remap = np.full(oqr.NTAB2, -1, np.int32); remap[used] = np.arange(len(used))
    cum = oqr.cum_of(freq)
    data = oqr.rans_encode(seq, remap, freq, cum)
    x = int.from_bytes(data[:4], "big"); p = 4
    for t, s in seq:
        tt = remap[t]; slot = x & 4095
        v = int(np.searchsorted(cum[tt], slot, side="right") - 1)
        assert v == s
        x = int(freq[tt, v]) * (x >> 12) + slot - int(cum[tt, v])
        while x < oqr.RANS_L:
            x = (x << 8) | data[p]; p += 1
        assert oqr.RANS_L <= x < oqr.RANS_L << 8
    assert p == len(data) and x == oqr.RANS_L


def test_encoder_reciprocal_step_equals_division():
    """the device encoder's division-free step (qr.hip enc_rcp / Enc::put_fc): for every frequency
    1..4096 and states 1 .. ((RANS_L >> PB) << 8) * f - 1 (the bound renormalisation leaves), with 32-bit
    wrap-around, it equals (x // f) * 2^PB + x % f + c"""
    M, L = 1 << 12, 1 << 23
    g = np.random.default_rng(11)

    def rcp(f):
        if f < 2:
            return 0xFFFFFFFF
        sh = (f - 1).bit_length()
        return ((1 << (31 + sh)) + f - 1) // f

    def step(x, f, c):
        sh = 0 if f < 2 else 31 - (32 - (f - 1).bit_length())
        q = ((x * rcp(f)) >> 32) >> sh
        return (x + c + (M - 1 if f < 2 else 0) + q * (M - f)) & 0xFFFFFFFF

    for f in range(1, M + 1):
        xm = ((L >> 12) << 8) * f                # the state after renormalisation is below this
        xs = [1, 2, f, f + 1, xm - 1, xm - 2, xm - f, xm - f - 1] + [int(v) for v in g.integers(1, xm, 24)]
        xs += [k * f + r for k in (1, xm // f - 1) for r in (0, f - 1)]
        c = int(g.integers(0, M - f + 1))
        for x in xs:
            if 1 <= x < xm:
                assert step(x, f, c) == ((x // f) << 12) + x % f + c, (f, x)
