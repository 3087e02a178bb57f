"""The oracle's deterministic arithmetic (oracle/detmath.py) and importance fit (oracle/imxfit.py),
pinned by what the mathematics fixes and by the reference's own C quantizers (oracle/_ref)."""
import numpy as np
import pytest

from oracle import detmath as odm
from oracle import ref

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")


def _loop_sum(t):
    s = 0.0
    for v in t:
        s = s + float(v)
    return s


def test_inorder_sums_are_term_by_term():
    g = np.random.default_rng(1)
    X = g.standard_normal((3, 4, 50)).astype(np.float32)
    G = odm.gram(X)
    for c in range(3):
        for a in range(4):
            for b in range(4):
                want = _loop_sum(np.float64(X[c, a]) * np.float64(X[c, b]))
                assert G[c, a, b] == np.float32(want)
    assert np.array_equal(G, G.transpose(0, 2, 1))
    np.testing.assert_allclose(G, np.einsum("nkd,njd->nkj", X.astype(np.float64), X.astype(np.float64)), rtol=1e-6)
    y = g.standard_normal((3, 50)).astype(np.float32)
    B = odm.bdot(X, y)
    assert B[1, 2] == np.float32(_loop_sum(np.float64(X[1, 2]) * np.float64(y[1])))


def test_inorder_differs_from_pairwise_on_cancelling_terms():
    # products 2^54, 1 (64 times), -2^54: in order each 1 is lost to rounding (0); numpy's pairwise
    # summation keeps most of them
    X = np.array([[[2.0 ** 27] + [1.0] * 64 + [-(2.0 ** 27)]]], np.float32)
    y = np.array([[2.0 ** 27] + [1.0] * 64 + [2.0 ** 27]], np.float32)
    assert odm.bdot(X, y)[0, 0] == 0.0
    assert np.sum(X[0, 0].astype(np.float64) * y[0].astype(np.float64)) > 0


def test_masked_column_sums():
    g = np.random.default_rng(2)
    x = g.standard_normal((40, 7)).astype(np.float32)
    mask = g.random(40) < 0.5
    s = odm.cols(x, True, mask)
    for c in range(7):
        assert s[c] == _loop_sum(np.float64(x[mask, c]) ** 2)


def test_solve():
    g = np.random.default_rng(3)
    k, n = 9, 20
    A = (g.standard_normal((n, k, k)) + 4 * np.eye(k)).astype(np.float32)
    b = g.standard_normal((n, k)).astype(np.float32)
    x = odm.solve(A, b)
    np.testing.assert_allclose(x, np.linalg.solve(A.astype(np.float64), b.astype(np.float64)[..., None])[..., 0],
                               rtol=1e-4, atol=1e-5)
    # integer systems: exact; a zero first pivot needs the row exchange, which a planted mistake skips
    A2 = np.array([[[0, 2, 1], [1, 1, 0], [3, 0, 1]]], np.float32)
    xs = np.array([[2, -1, 3]], np.float32)
    b2 = np.einsum("nij,nj->ni", A2, xs).astype(np.float32)
    assert np.array_equal(odm.solve(A2, b2), xs)
    bad = odm.solve(A2, b2, pivot=False)
    assert not np.array_equal(bad, xs)
    # k = 1 and k = 16
    assert odm.solve(np.array([[[4.0]]], np.float32), np.array([[2.0]], np.float32))[0, 0] == 0.5
    A16 = (g.standard_normal((2, 16, 16)) + 8 * np.eye(16)).astype(np.float32)
    b16 = g.standard_normal((2, 16)).astype(np.float32)
    np.testing.assert_allclose(odm.solve(A16, b16), np.linalg.solve(A16.astype(np.float64), b16.astype(np.float64)[..., None])[..., 0],
                               rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("T", [2, 3, 6, 7])
def test_importance_fit_recovers_the_quantizers_importance(T):
    from oracle import imxfit as oi
    g = np.random.default_rng(10 + T)
    R, cols = 768, 256
    X = (g.standard_normal((R, cols)) * 0.02).astype(np.float32)
    e = np.exp(g.standard_normal(cols)).astype(np.float32)
    F = np.asarray(ref.quantize(T, X, e)).reshape(R, -1)
    q = oi.ls_solve(oi.ls_gram(T, X[:512], F[:512]), e)
    qp = oi.ls_solve(oi.ls_gram(T, X[:512], F[:512], plant="no_sigma"), e)
    fit = oi.equal_blocks(T, X[512:], F[512:], q)
    planted = oi.equal_blocks(T, X[512:], F[512:], qp)
    unit = oi.equal_blocks(T, X[512:], F[512:], np.ones(cols, np.float32))
    assert np.corrcoef(np.log(q), np.log(e))[0, 1] > 0.99
    assert fit > 0.55 and fit > planted + 0.2 and unit < 0.1, (fit, planted, unit)
    assert oi.equal_blocks(T, X[512:], F[512:], e) == 1.0


def _fit_cases():
    from tests.golden.fit_cases import CASES
    return [c[0] for c in CASES]


@pytest.mark.parametrize("name", _fit_cases())
def test_importance_fit_equals_the_reference_fit(name):
    """the restatement against tests/golden/fit_vectors.npz, written by the reference's own imxfit.py
    (ls_gram, ls_solve, equal_blocks) under its --cpu backend: Gram sums over the tensors that share
    the importance, fitted vector and check share all equal"""
    from oracle import imxfit as oi
    from tests.golden.fit_cases import CASES, COLS, R_FIT, case_inputs, digest
    z = np.load("tests/golden/fit_vectors.npz")
    _, T, ntens, _ = next(c for c in CASES if c[0] == name)
    xs, e = case_inputs(name)
    assert bytes(z[f"{name}/inputs_sha256"]).hex() == digest(xs, e), "numpy's generator changed: inputs differ"
    G = np.zeros((COLS // 32, 32, 32), np.float64)
    for k in range(ntens):
        F = z[f"{name}/blocks{k}"]
        assert np.frombuffer(ref.quantize(T, xs[k], e), np.uint8).tobytes() == F.tobytes()
        G += oi.ls_gram(T, xs[k][:R_FIT], F[:R_FIT])
    assert np.array_equal(G, z[f"{name}/G"])
    q = oi.ls_solve(G, e)
    assert np.array_equal(q, z[f"{name}/fit"])
    share = [oi.equal_blocks(T, xs[k][R_FIT:], z[f"{name}/blocks{k}"][R_FIT:], q) for k in range(ntens)]
    assert share == list(z[f"{name}/share"])
