"""Deterministic arithmetic (spa_dm_*), the importance fit (spa_imx_conditions + seedpack_amd.imxfit)
and the sibling estimate (spa_est_*) on the MI355X, bit-exact against the oracle (oracle/detmath.py,
oracle/imxfit.py, oracle/r2.py) on the same inputs."""
import sys

import numpy as np
import pytest

from oracle import detmath as odm
from oracle import ref
from seedpack_amd import detmath, estimate, imxfit
from seedpack_amd import device as dev
from seedpack_amd.gpuquant import GPUQuant

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.mark.parametrize("nr,nc", [(1, 1), (5, 63), (64, 64), (130, 200), (3, 1000)])
def test_rows_and_cols(nr, nc):
    say("case detmath rows/cols", nr, nc)
    g = np.random.default_rng(nr * 1000 + nc)
    x = (g.standard_normal((nr, nc)) * np.exp(3 * g.standard_normal((nr, 1)))).astype(np.float32)
    for sq in (False, True):
        assert np.array_equal(detmath.rows(x, sq).to_host(), odm.rows_sum(x, sq))
        assert np.array_equal(detmath.rows(x.astype(np.float64), sq).to_host(),
                              odm._inorder(x.astype(np.float64) ** 2 if sq else x.astype(np.float64), -1))
        assert np.array_equal(detmath.cols(x, sq).to_host(), odm.cols(x, sq))
        mask = g.random(nr) < 0.6
        assert np.array_equal(detmath.cols(x, sq, mask).to_host(), odm.cols(x, sq, mask))
    assert detmath.total(x, True) == float(odm.rows_sum(x.reshape(1, -1), True)[0])


@pytest.mark.parametrize("n,k,d", [(1, 1, 1), (3, 4, 70), (2, 32, 1000), (40, 32, 64), (5, 17, 129)])
def test_gram_and_bdot(n, k, d):
    say("case detmath gram/bdot", n, k, d)
    g = np.random.default_rng(n * 7 + k * 13 + d)
    X = g.standard_normal((n, k, d)).astype(np.float32)
    y = g.standard_normal((n, d)).astype(np.float32)
    assert np.array_equal(detmath.gram(X).to_host(), odm.gram(X))
    assert np.array_equal(detmath.bdot(X, y).to_host(), odm.bdot(X, y))


def test_cancelling_terms_stay_in_order():
    X = np.array([[[2.0 ** 27] + [1.0] * 64 + [-(2.0 ** 27)]]], np.float32)
    y = np.array([[2.0 ** 27] + [1.0] * 64 + [2.0 ** 27]], np.float32)
    assert detmath.bdot(X, y).to_host()[0, 0] == 0.0


@pytest.mark.parametrize("k", [1, 2, 3, 9, 16])
def test_solve(k):
    say("case detmath solve", k)
    g = np.random.default_rng(k)
    n = 50
    A = (g.standard_normal((n, k, k)) + 2 * np.eye(k)).astype(np.float32)
    A[0, 0, :] = 0                                        # first system: the first pivot needs an exchange
    A[0, 0, k - 1] = 1 if k > 1 else 3
    b = g.standard_normal((n, k)).astype(np.float32)
    assert np.array_equal(detmath.solve(A, b).to_host(), odm.solve(A, b))


def test_log2_exp2():
    x = np.array([1.0, 2.0, 0.5, 3.0, 1e-310, 5e-324, 0.0, -1.0, np.inf, np.nan, 1.4142135623730951, 1e300,
                  0.7071067811865476, 123.456], np.float64)
    x = np.concatenate([x, np.random.default_rng(5).random(1000) * 1e3])
    got = detmath.log2(x).to_host()
    want = odm.dm_log2(x)
    assert np.array_equal(got, want, equal_nan=True)
    y = np.concatenate([np.array([0.0, 1.0, -1.0, 0.5, 1023.9, 1024.0, -1074.5, -1075.5, np.nan, -np.inf, np.inf]),
                        np.random.default_rng(6).standard_normal(1000) * 40])
    assert np.array_equal(detmath.exp2(y).to_host(), odm.dm_exp2(y), equal_nan=True)


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("T", [2, 3, 6, 7])
def test_importance_fit_equals_oracle(T):
    from oracle import imxfit as oi
    say("case imxfit", T)
    g = np.random.default_rng(20 + T)
    R, cols = 600, 512
    X = (g.standard_normal((R, cols)) * 0.02).astype(np.float32)
    X[g.random((R, cols)) < 0.001] *= 25
    X[7] = 0                                               # a zero row: zero scales
    e = np.exp(g.standard_normal(cols)).astype(np.float32)
    F = np.asarray(ref.quantize(T, X, e)).reshape(R, -1)
    gq = GPUQuant()
    G = imxfit.ls_gram(gq, T, X[:400], F[:400])
    Go = oi.ls_gram(T, X[:400], F[:400])
    assert np.array_equal(G, Go)
    q = imxfit.ls_solve(G, e)
    assert np.array_equal(q, oi.ls_solve(Go, e))
    eq = imxfit.equal_blocks(gq, T, X[400:], F[400:], q)
    assert eq == oi.equal_blocks(T, X[400:], F[400:], q) and eq > 0.5


def _fit_cases():
    from tests.golden.fit_cases import CASES
    return [c[0] for c in CASES]


@pytest.mark.parametrize("name", _fit_cases())
def test_importance_fit_equals_the_reference_fit(name):
    """the device fit against tests/golden/fit_vectors.npz (the reference's own imxfit.py run under its
    --cpu backend): the quantizer's blocks, the Gram sums over the tensors sharing the importance, the
    fitted vector and the check share, all equal"""
    from tests.golden.fit_cases import CASES, COLS, R_FIT, case_inputs, digest
    say("case imxfit golden", name)
    z = np.load("tests/golden/fit_vectors.npz")
    _, T, ntens, _ = next(c for c in CASES if c[0] == name)
    xs, e = case_inputs(name)
    assert bytes(z[f"{name}/inputs_sha256"]).hex() == digest(xs, e), "numpy's generator changed: inputs differ"
    gq = GPUQuant()
    G = np.zeros((COLS // 32, 32, 32), np.float64)
    for k in range(ntens):
        F = z[f"{name}/blocks{k}"]
        X = dev.DeviceArray.from_host(xs[k])
        assert gq.quantize_batch(T, [X], [e])[0].to_host().tobytes() == F.tobytes()
        G += imxfit.ls_gram(gq, T, xs[k][:R_FIT], F[:R_FIT])
    assert np.array_equal(G, z[f"{name}/G"])
    q = imxfit.ls_solve(G, e)
    assert np.array_equal(q, z[f"{name}/fit"])
    share = [imxfit.equal_blocks(gq, T, xs[k][R_FIT:], z[f"{name}/blocks{k}"][R_FIT:], q) for k in range(ntens)]
    assert share == list(z[f"{name}/share"])


def test_sibling_estimate():
    g = np.random.default_rng(9)
    n = 5000
    x = g.standard_normal(n).astype(np.float32)
    lo = (x - g.random(n).astype(np.float32) * 0.1).astype(np.float32)
    hi = (x + g.random(n).astype(np.float32) * 0.1).astype(np.float32)
    lo[:50] = -np.inf
    hi[25:75] = np.inf
    d = {k: dev.DeviceArray.from_host(v) for k, v in (("x", x), ("lo", lo), ("hi", hi))}
    h = estimate.half_step(d["x"], d["lo"], d["hi"]).to_host()
    fl, fu = np.isfinite(lo), np.isfinite(hi)
    want_h = np.where(fl & fu, np.float32(0.5) * (hi - lo), np.where(fu, hi - x, np.where(fl, x - lo, np.float32(-1))))
    assert np.array_equal(h, want_h.astype(np.float32))
    est = estimate.Est(n)
    ws = np.zeros(n, np.float32)
    wx = np.zeros(n, np.float32)
    xs = [x, (x + 0.01).astype(np.float32)]
    for k, xv in enumerate(xs):
        hv = h if k == 0 else np.abs(h[::-1]).astype(np.float32)
        est.add(dev.DeviceArray.from_host(xv), dev.DeviceArray.from_host(hv))
        w = np.float32(1) / np.fmax(hv * hv, np.float32(1e-30))
        ws = np.where(hv < 0, ws, ws + w).astype(np.float32)
        wx = np.where(hv < 0, wx, wx + xv * w).astype(np.float32)
    s = est.seed().to_host().reshape(-1, 2)
    with np.errstate(divide="ignore", invalid="ignore"):
        want = np.where(ws > 0, wx / ws, xs[0]).astype(np.float32)
        wanth = np.where(ws > 0, np.float32(1) / np.sqrt(ws), np.float32(0)).astype(np.float32)
    assert np.array_equal(s[:, 0], want) and np.array_equal(s[:, 1], wanth)
