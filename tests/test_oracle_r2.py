"""The R2 oracle against the reference's own R2 code (golden vectors from its --cpu backend), and
detmath's log2 / exp2 against the C library."""
import math
import os

import numpy as np
import pytest

from oracle import r2 as or2
from tests.golden.r2_cases import CASES, case_file

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def vectors():
    return np.load(os.path.join(ROOT, "tests", "golden", "r2_vectors.npz"))


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_oracle_r2_matches_reference(vectors, name):
    data, layout, gb = case_file(name)
    res = or2.compress(data, layout, gb)
    for k in ("rfi", "cfi", "scl", "nrows_c", "dups", "rowmap", "counts", "freq", "used", "lens"):
        assert np.array_equal(res[k], vectors[f"{name}/{k}"]), k
    assert res["stream"].tobytes() == vectors[f"{name}/stream"].tobytes()


def _ulps(a, b):
    ia, ib = np.float64(a).view(np.int64), np.float64(b).view(np.int64)
    return abs(int(ia) - int(ib))


def test_detmath_log2_exp2_against_libm():
    g = np.random.default_rng(1)
    xs = np.concatenate([g.lognormal(0, 30, 4000), [1e-310, 5e-324, 1.0, 2.0, 0.5, 1e300, np.sqrt(2.0)]])
    got = or2.dm_log2(xs)
    for x, y in zip(xs, got):
        assert _ulps(y, math.log2(x)) <= 2 or abs(y - math.log2(x)) < 1e-15, (x, y, math.log2(x))
    for e in range(-1070, 1020, 7):
        assert or2.dm_log2(2.0 ** e)[0] == e                   # exact at powers of two
    ys = np.concatenate([g.uniform(-1000, 1000, 4000), [0.0, -0.5, 0.5, 1023.5, -1074.0]])
    got = or2.dm_exp2(ys)
    for y, v in zip(ys, got):
        ref = 2.0 ** y
        assert ref == 0 or _ulps(v, ref) <= 2, (y, v, ref)
    for e in range(-1022, 1023, 5):
        assert or2.dm_exp2(float(e))[0] == 2.0 ** e
    assert np.isnan(or2.dm_log2(-1.0)[0]) and or2.dm_log2(0.0)[0] == -np.inf and or2.dm_exp2(2000.0)[0] == np.inf
    assert or2.dm_exp2(-2000.0)[0] == 0.0


def test_rint_half_even():
    assert list(or2.dm_rint([0.5, 1.5, 2.5, -0.5, -1.5, 2.4999999999999996])) == [0.0, 2.0, 2.0, -0.0, -2.0, 2.0]


def test_normalize_invariants():
    g = np.random.default_rng(4)
    c = np.zeros((6, 256), np.uint32)
    c[0, 0] = 10 ** 6; c[0, 1:40] = 1                               # one dominant symbol, rare ones
    # (a row needing more than 64 corrections makes the reference's own assertion fail, gpu2.py:478)
    c[1] = g.integers(0, 1000, 256)
    c[3, 9] = 5
    c[4, :3] = [1, 1, 1]
    f, used = or2.normalize(c)
    assert list(used) == [0, 1, 3, 4]
    assert (f.astype(np.int64).sum(1) == 1 << 15).all()
    assert ((c[used] > 0) <= (f > 0)).all()
