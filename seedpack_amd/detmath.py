"""Deterministic arithmetic on the device (the reference's seedpack/detmath.py): float64 sums in
index order, batched Gram matrices and matrix-vector products, small systems by Gaussian
elimination, log2 / exp2 from basic operations -- the same bits as the reference's GPU and --cpu
builds, so the decisions taken from them (scale bins, fitted importance, row parents) do not depend
on the device. Arguments are DeviceArrays or host arrays (uploaded); results are DeviceArrays.
"""
import numpy as np

from . import device as dev
from ._lib import check, lib


def _dev(a, dtype, stream):
    if isinstance(a, dev.DeviceArray):
        if a.dtype != np.dtype(dtype):
            raise TypeError(f"{a.dtype} array where {np.dtype(dtype)} is expected")
        return a
    return dev.DeviceArray.from_host(np.ascontiguousarray(a, dtype), stream)


def rows(x, square=False, stream=None):
    """float64 sums (of squares) along the rows of a 2-D float32 / float64 array (detmath.py:185-192)"""
    f64 = (x.dtype == np.float64)
    x = _dev(x, np.float64 if f64 else np.float32, stream)
    nr, nc = x.shape
    out = dev.DeviceArray(nr, np.float64)
    check(lib().spa_dm_rows(x.ptr, int(f64), nr, nc, int(square), out.ptr, stream))
    return out


def cols(x, square=False, mask=None, stream=None):
    """float64 sums (of squares) down the columns of a 2-D float32 array, rows with mask False left out
    (detmath.py:195-202)"""
    x = _dev(x, np.float32, stream)
    nr, nc = x.shape
    m = None if mask is None else _dev(np.asarray(mask).astype(np.uint8) if not isinstance(mask, dev.DeviceArray) else mask,
                                        np.uint8, stream)
    out = dev.DeviceArray(nc, np.float64)
    check(lib().spa_dm_cols(x.ptr, nr, nc, int(square), None if m is None else m.ptr, out.ptr, stream))
    return out


def total(x, square=False, stream=None):
    """float64 sum (of squares) of all elements in index order (detmath.py:205-207)"""
    x = x if isinstance(x, dev.DeviceArray) else np.asarray(x)
    flat = x.view(0, (1, x.size), x.dtype) if isinstance(x, dev.DeviceArray) else x.reshape(1, -1)
    return float(rows(flat, square, stream).to_host(stream=stream)[0])


def gram(X, stream=None):
    """X (n, k, d) float32 -> X X^T per batch element (n, k, k) float32 (detmath.py:210-216)"""
    X = _dev(X, np.float32, stream)
    n, k, d = X.shape
    out = dev.DeviceArray((n, k, k), np.float32)
    check(lib().spa_dm_gram(X.ptr, n, k, d, out.ptr, stream))
    return out


def bdot(X, y, stream=None):
    """X (n, k, d), y (n, d) float32 -> X y per batch element (n, k) float32 (detmath.py:219-225)"""
    X, y = _dev(X, np.float32, stream), _dev(y, np.float32, stream)
    n, k, d = X.shape
    out = dev.DeviceArray((n, k), np.float32)
    check(lib().spa_dm_bdot(X.ptr, y.ptr, n, k, d, out.ptr, stream))
    return out


def solve(A, b, stream=None):
    """batched small systems A (n, k, k) x = b (n, k), k <= 16 -> x (n, k) float32 (detmath.py:228-235)"""
    A, b = _dev(A, np.float32, stream), _dev(b, np.float32, stream)
    n, k = b.shape
    x = dev.DeviceArray((n, k), np.float32)
    check(lib().spa_dm_solve(A.ptr, b.ptr, n, k, x.ptr, stream))
    return x


def log2(x, stream=None):
    """float64 log2 elementwise (detmath.py:171-175)"""
    x = _dev(x, np.float64, stream)
    y = dev.DeviceArray(x.shape, np.float64)
    check(lib().spa_dm_log2(x.ptr, x.size, y.ptr, stream))
    return y


def exp2(x, stream=None):
    """float64 2 ** x elementwise (detmath.py:178-182)"""
    x = _dev(x, np.float64, stream)
    y = dev.DeviceArray(x.shape, np.float64)
    check(lib().spa_dm_exp2(x.ptr, x.size, y.ptr, stream))
    return y
