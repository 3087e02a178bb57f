"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

CPU restatement of the reference's deterministic arithmetic (seedpack/detmath.py, cited as
detmath.py:LINES) beyond the row / column sums and log2 / exp2 that oracle/r2.py already holds:
batched Gram matrices and matrix-vector products with float64 sums in index order (dm_gram / dm_bdot,
detmath.py:109-126), masked column sums (dm_cols, :95-106), and small systems by Gaussian elimination
with partial pivoting in float64 (dm_solve, :128-153), step for step.

Pinned by tests/test_oracle_fit.py: the in-order sums against a Python loop and, within rounding,
against numpy's float64 einsum; an input whose terms cancel makes pairwise summation (a plausible
mistake) differ; solve against numpy.linalg.solve on well-conditioned systems and exactly on systems
with integer solutions, a system whose first pivot is zero, and a planted mistake (no pivoting) that
must fail there.
"""
import numpy as np

from oracle.r2 import cols_sum, dm_exp2, dm_log2, rows_sum  # noqa: F401  (re-exported)

F64 = np.float64


def _inorder(t, axis):
    """float64 sum of t along axis, term by term from index 0 (0 + t0 + t1 + ...)"""
    t = np.moveaxis(np.asarray(t, F64), axis, -1)
    z = np.zeros(t.shape[:-1] + (1,), F64)
    return np.add.accumulate(np.concatenate([z, t], -1), axis=-1)[..., -1]


def cols(x, square=False, mask=None):
    """detmath.cols (detmath.py:95-106): rows with mask False left out"""
    x = np.asarray(x, np.float32)
    if mask is not None:
        x = x[np.asarray(mask, bool)]
    if x.shape[0] == 0:
        return np.zeros(x.shape[1], F64)
    return cols_sum(x, square)


def gram(X):
    """detmath.gram (detmath.py:109-117): X (n, k, d) float32 -> (n, k, k) float32"""
    X = np.asarray(X, np.float32).astype(F64)
    return _inorder(X[:, :, None, :] * X[:, None, :, :], -1).astype(np.float32)


def bdot(X, y):
    """detmath.bdot (detmath.py:118-126): X (n, k, d), y (n, d) -> (n, k) float32"""
    X = np.asarray(X, np.float32).astype(F64)
    y = np.asarray(y, np.float32).astype(F64)
    return _inorder(X * y[:, None, :], -1).astype(np.float32)


def solve(A, b, pivot=True):
    """detmath.solve (detmath.py:128-153): A (n, k, k), b (n, k) float32 -> x (n, k) float32"""
    A = np.asarray(A, np.float32)
    b = np.asarray(b, np.float32)
    n, k = b.shape
    out = np.empty((n, k), np.float32)
    for c in range(n):
        M = [[float(A[c, i, j]) for j in range(k)] + [float(b[c, i])] for i in range(k)]
        for col in range(k):
            piv = col
            if pivot:
                for i in range(col + 1, k):
                    if abs(M[i][col]) > abs(M[piv][col]):
                        piv = i
            if piv != col:
                M[col], M[piv] = M[piv], M[col]
            p = M[col][col]
            for i in range(col + 1, k):
                f = M[i][col] / p if p != 0.0 else (np.inf if M[i][col] != 0.0 else np.nan)
                for j in range(col, k + 1):
                    M[i][j] = M[i][j] - f * M[col][j]
        for i in range(k - 1, -1, -1):
            s = M[i][k]
            for j in range(i + 1, k):
                s = s - M[i][j] * M[j][k]
            M[i][k] = s / M[i][i] if M[i][i] != 0.0 else np.nan
        out[c] = [M[i][k] for i in range(k)]
    return out
