"""Inputs of the importance-fit golden cases (tests/golden/make_fit_golden.py writes the expected
outputs): seeded BF16 weights and importances. The SHA-256 of each case's weight and importance
bytes is stored with the outputs, so a change of numpy's generator shows as a failed input check."""
import hashlib

import numpy as np

COLS = 256                     # 8 blocks of 32 columns
R_FIT, R_CHECK = 160, 64       # rows fitted, rows that check the fit

# (name, ggml type, tensors sharing the importance, seed)
CASES = [("q4_0", 2, 1, 101), ("q4_1", 3, 2, 102), ("q5_0", 6, 1, 103), ("q5_1", 7, 2, 104)]


def _bf16_round(x):
    u = np.asarray(x, np.float32).view(np.uint32)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return u.view(np.float32)


def case_inputs(name):
    """-> ([float32 (R_FIT + R_CHECK, COLS) weights holding BF16 values per tensor], float32 importance)"""
    _, T, ntens, seed = next(c for c in CASES if c[0] == name)
    g = np.random.Generator(np.random.PCG64(seed))
    e = np.exp(g.standard_normal(COLS)).astype(np.float32)
    xs = []
    for k in range(ntens):
        x = g.standard_normal((R_FIT + R_CHECK, COLS)) * 0.02
        x[g.random(x.shape) < 0.002] *= 25
        x[3] = 0                                  # a zero row: zero scales
        x[5, 64:96] = 0                           # a zero block
        xs.append(_bf16_round(x))
    return xs, e


def digest(xs, e):
    h = hashlib.sha256()
    for x in xs:
        h.update(np.ascontiguousarray(x, np.float32).tobytes())
    h.update(np.ascontiguousarray(e, np.float32).tobytes())
    return h.hexdigest()
