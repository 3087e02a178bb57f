"""Recovering the importance matrix a legacy quant (Q4_0, Q4_1, Q5_0, Q5_1) was made with, from the
quant itself (the reference's seedpack/imxfit.py): the block scale of these quantizers is a weighted
least-squares fit, so every block's residual x - v is weighted-orthogonal to its codes (and to 1 when
a minimum is kept). Those conditions, summed over rows as per-block-of-columns Gram matrices
(ls_gram, on the device with detmath's in-order sums), have the importance of the block's columns as
their smallest eigenvector (ls_solve, numpy on the host as in the reference); equal_blocks checks a
fit on other rows by quantizing them again.
"""
import numpy as np

from . import detmath
from . import device as dev
from ._lib import check, lib
from .requant import QFUN

LS_TYPES = {2, 3, 6, 7}


def ls_gram(gq, T, X, F, stream=None):
    """conditions of rows X (float32, rows x cols; device or host) quantized as F (their blocks of type
    T, device or host uint8) -> float64 (blocks of columns, 32, 32) numpy, to be summed over tensors
    with the same input (imxfit.py:30-58)"""
    if T not in LS_TYPES:
        raise ValueError(f"type {T} is not a least-squares legacy type")
    _, qk, bs = QFUN[T]
    X = X if isinstance(X, dev.DeviceArray) else dev.DeviceArray.from_host(np.ascontiguousarray(X, np.float32), stream)
    R, cols = X.shape
    nb = cols // qk
    F = F if isinstance(F, dev.DeviceArray) else dev.DeviceArray.from_host(np.ascontiguousarray(F, np.uint8).reshape(-1), stream)
    if F.nbytes != R * nb * bs:
        raise ValueError(f"{F.nbytes} bytes of blocks for {R} rows of {cols} weights")
    V = gq.dequantize(T, F, cols)
    rowsq = detmath.rows(X, True, stream)
    two = T in (3, 7)
    e1 = dev.DeviceArray((nb, qk, R), np.float32)
    e2 = dev.DeviceArray((nb, qk, R), np.float32) if two else None
    check(lib().spa_imx_conditions(T, X.ptr, F.ptr, V.ptr, rowsq.ptr, R, cols, e1.ptr, None if e2 is None else e2.ptr,
                                   stream))
    G = np.zeros((nb, qk, qk), np.float64)
    for e in ([e1, e2] if two else [e1]):
        G += detmath.gram(e, stream).to_host(stream=stream).astype(np.float64)
    return G


def ls_solve(G, e0):
    """importance (float32) from summed conditions G, each block of columns scaled to the sum of e0's
    there (imxfit.py:61-71)"""
    nb, qk = G.shape[0], G.shape[1]
    _, V = np.linalg.eigh(np.asarray(G))
    q = V[:, :, 0]
    q = q * np.sign(q.sum(1, keepdims=True))
    q = np.maximum(q, 1e-6 * np.abs(q).max(1, keepdims=True))
    e0 = np.asarray(e0, np.float64).reshape(nb, qk)
    q = q / q.sum(1, keepdims=True) * e0.sum(1, keepdims=True)
    return q.reshape(-1).astype(np.float32)


def equal_blocks(gq, T, X, F, e):
    """share of the blocks of rows X (float32, rows x cols) that importance e reproduces; F: the
    file's blocks of those rows (imxfit.py:74-79)"""
    _, qk, bs = QFUN[T]
    X = X if isinstance(X, dev.DeviceArray) else dev.DeviceArray.from_host(np.ascontiguousarray(X, np.float32), gq.stream)
    Y = gq.quantize_batch(T, [X], [np.asarray(e, np.float32)])[0].to_host(stream=gq.stream)
    Fh = F.to_host(stream=gq.stream) if isinstance(F, dev.DeviceArray) else np.asarray(F, np.uint8)
    return float((Y.reshape(-1, bs) == Fh.reshape(-1, bs)).all(-1).mean())
