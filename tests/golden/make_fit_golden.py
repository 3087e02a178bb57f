"""Writes importance-fit golden vectors by running the reference's own seedpack/imxfit.py (ls_gram,
ls_solve, equal_blocks) through its --cpu backend (seedpack/cpu.py, seedpack/cpukernels.py) and its
detmath module. Run in the build container only:

    python tests/golden/make_fit_golden.py

imxfit.py imports only detmath, xp and requant.QFUN, all importable with SEEDPACK_CPU=1, so the module
is imported as it stands. Its `gq` argument (the GPUQuant object of the reference's GPU path) is served
by the reference's own C quantizers and dequantizers, compiled from ggml-quants.c into oracle/_ref
(`make -C oracle`): GPUQuant is bit-exact with them by construction (gpuquant.py:1-11).

Cases (one per least-squares legacy type): BF16 weights, N(0, 0.02) with 0.2% outliers at x25, one
zero row, one row with a zero block; a log-normal importance; one tensor, or two tensors that share
the importance (gate and up: their Gram matrices are summed, imxfit.py:1-14). The first R_FIT rows of
each tensor are fitted, the last R_CHECK rows check the fit. Output: tests/golden/fit_vectors.npz with,
per case, the BF16 weights, the importance, the reference C quantizer's blocks, the summed Gram
matrices G, the fitted importance and the share of check blocks it reproduces (data only).
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, ROOT)

os.environ["SEEDPACK_CPU"] = "1"
os.environ.setdefault("SEEDPACK_CACHE", tempfile.mkdtemp(prefix="seedpack_refcache_"))
sys.path.insert(0, REF)

from oracle import ref  # noqa: E402
from tests.golden.fit_cases import CASES, COLS, R_FIT, case_inputs, digest  # noqa: E402


class RefQuant:
    """GPUQuant's dequantize / quantize_batch as the reference's C library computes them"""

    def __init__(self, cp):
        self.cp = cp

    def dequantize(self, T, F, cols):
        F = np.ascontiguousarray(np.asarray(F), np.uint8).reshape(-1)
        n = F.size // ref.BS[T] * ref.QK[T]
        return self.cp.asarray(np.asarray(ref.dequantize(T, F.tobytes(), n), np.float32))

    def quantize_batch(self, T, Xs, imxs):
        return [self.cp.asarray(np.frombuffer(ref.quantize(T, np.asarray(X, np.float32), imx), np.uint8).copy())
                for X, imx in zip(Xs, imxs)]


def main():
    if not ref.available():
        raise SystemExit("oracle/_ref is not built: make -C oracle")
    from seedpack import cpu as cp
    from seedpack import imxfit
    gq = RefQuant(cp)
    out = {}
    for name, T, ntens, seed in CASES:
        xs, e = case_inputs(name)
        G = np.zeros((COLS // 32, 32, 32), np.float64)
        blocks = []
        for k in range(ntens):
            X = xs[k]
            F = np.frombuffer(ref.quantize(T, X, e), np.uint8).reshape(X.shape[0], -1).copy()
            blocks.append(F)
            G += np.asarray(imxfit.ls_gram(gq, T, cp.asarray(X[:R_FIT]), cp.asarray(F[:R_FIT])))
        q = imxfit.ls_solve(cp.asarray(G), e)
        share = [imxfit.equal_blocks(gq, T, cp.asarray(xs[k][R_FIT:]), cp.asarray(blocks[k][R_FIT:]), q)
                 for k in range(ntens)]
        for k in range(ntens):
            out[f"{name}/blocks{k}"] = blocks[k]
        out[f"{name}/inputs_sha256"] = np.frombuffer(bytes.fromhex(digest(xs, e)), np.uint8)
        out[f"{name}/G"] = G
        out[f"{name}/fit"] = np.asarray(q, np.float32)
        out[f"{name}/share"] = np.array(share, np.float64)
        print(f"{name}: type {T}, {ntens} tensor(s), fitted share of check blocks {share}", flush=True)
    np.savez_compressed(os.path.join(HERE, "fit_vectors.npz"), **out)


if __name__ == "__main__":
    main()
