"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

CPU restatement of the reference's importance fit (seedpack/imxfit.py, cited as imxfit.py:LINES):
ls_gram's per-weight conditions c (x - v) l (and c (x - v) [m != 0] for the types with a minimum),
c = sqrt(rowsq / cols + x^2), normalised per block and summed into per-block-of-columns Gram matrices
with detmath's in-order float64 sums (imxfit.py:30-58); ls_solve is the reference's own numpy code
(imxfit.py:61-71); equal_blocks re-quantizes through the reference's C quantizers (oracle/_ref).
Every float32 operation is one numpy operation in the reference's order.

Pinned by tests/test_oracle_fit.py: bit for bit against tests/golden/fit_vectors.npz, which the
reference's own imxfit.py wrote under its --cpu backend (tests/golden/make_fit_golden.py: Gram sums
over tensors sharing an importance, the fitted vector, the share of check blocks reproduced, for Q4_0,
Q4_1, Q5_0, Q5_1 with zero rows, zero blocks and outliers); and by properties: quantized with a known
importance by the reference's own C quantizers, the fit recovers an importance that reproduces the
quant's blocks on rows it was not fit on (a planted mistake -- the weights c without their sigma^2
term -- must do measurably worse), and the per-block normalisation and Gram sums follow
oracle/detmath.py.
"""
import numpy as np

from oracle import detmath as odm
from oracle import ref

QK, BS = 32, {2: 18, 3: 20, 6: 22, 7: 24}


def conditions(T, X, F, plant=None):
    """the normalised conditions [e1 (, e2)] of rows X (R, cols) float32 quantized as F (uint8 blocks),
    each (nb, 32, R) float32"""
    X = np.ascontiguousarray(X, np.float32)
    R, cols = X.shape
    nb = cols // QK
    F = np.ascontiguousarray(F, np.uint8).reshape(R, nb, BS[T])
    v = ref.dequantize(T, F.tobytes(), R * cols).reshape(R, nb, QK)
    d = F[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    two = T in (3, 7)
    m = F[:, :, 2:4].copy().view(np.float16).astype(np.float32) if two else np.zeros_like(d)
    l = np.rint((v - m) / np.where(d == 0, np.float32(1), d))
    xb = X.reshape(R, nb, QK)
    a = (odm.rows_sum(X, True) / cols).astype(np.float32)[:, None, None]
    c = np.sqrt(xb * xb) if plant == "no_sigma" else np.sqrt(a + xb * xb)
    res = xb - v
    out = []
    for e in ([c * res * l, c * res * (m != 0)] if two else [c * res * l]):
        e = e.astype(np.float32)
        nrm = np.sqrt(odm.rows_sum(e.reshape(-1, QK), True)).astype(np.float32).reshape(R, nb, 1)
        nrm = np.where(np.isnan(nrm), nrm, np.maximum(nrm, np.float32(1e-30)))
        out.append((e / nrm).astype(np.float32).transpose(1, 2, 0).copy())
    return out


def ls_gram(T, X, F, plant=None):
    G = np.zeros((X.shape[1] // QK, QK, QK), np.float64)
    for e in conditions(T, X, F, plant):
        G += odm.gram(e).astype(np.float64)
    return G


def ls_solve(G, e0):
    """imxfit.py:61-71 as the reference writes it (numpy on the host)"""
    nb, qk = G.shape[0], G.shape[1]
    _, V = np.linalg.eigh(G)
    q = V[:, :, 0]
    q = q * np.sign(q.sum(1, keepdims=True))
    q = np.maximum(q, 1e-6 * np.abs(q).max(1, keepdims=True))
    e0 = np.asarray(e0, np.float64).reshape(nb, qk)
    q = q / q.sum(1, keepdims=True) * e0.sum(1, keepdims=True)
    return q.reshape(-1).astype(np.float32)


def equal_blocks(T, X, F, e):
    Y = ref.quantize(T, np.ascontiguousarray(X, np.float32), np.asarray(e, np.float32))
    return float((np.frombuffer(Y, np.uint8).reshape(-1, BS[T]) == np.asarray(F, np.uint8).reshape(-1, BS[T])).all(-1).mean())
