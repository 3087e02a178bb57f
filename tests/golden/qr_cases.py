"""QR golden cases: shapes, distributions and the seeded BF16 seeds (shared by the generator
make_qr_golden.py and the tests, which regenerate the seeds instead of storing them)."""
import numpy as np

from seedpack_amd import synth

CASES = [  # (name, ggml type, rows, cols, distribution, imatrix, how the file differs from the prediction)
    ("q8_0", 8, 48, 1024, "cfg1", False, "perturb"), ("q4_0", 2, 48, 1024, "cfg1", False, "perturb"),
    ("q8_0_drift", 8, 20, 1024, "cfg1", False, "drift"), ("q4_0_drift", 2, 20, 1024, "cfg1", False, "drift"),
    ("q4_1", 3, 16, 1024, "cfg1", True, "drift"), ("q5_0", 6, 16, 1024, "cfg1", True, "drift"),
    ("q5_1", 7, 16, 1024, "cfg1", True, "drift"), ("q2_0", 42, 16, 1024, "cfg1", False, "drift"),
    ("q2_k", 10, 20, 1024, "cfg2", True, "perturb"), ("q3_k", 11, 20, 1024, "cfg2", True, "perturb"),
    ("q4_k", 12, 20, 1024, "cfg2", True, "perturb"), ("q5_k", 13, 20, 1024, "cfg2", True, "perturb"),
    ("q6_k", 14, 20, 1024, "cfg2", True, "perturb"),
    ("q2_k_var", 10, 12, 1024, "cfg2", True, "variant"), ("q3_k_var", 11, 12, 1024, "cfg2", True, "variant"),
    ("q4_k_var", 12, 12, 1024, "cfg2", True, "variant"), ("q5_k_var", 13, 12, 1024, "cfg2", True, "variant"),
    ("q6_k_var", 14, 12, 1024, "cfg2", True, "variant"),
    ("q4_k_drift", 12, 8, 3072, "cfg2", True, "drift"), ("q6_k_drift", 14, 8, 3072, "cfg2", False, "drift"),
    ("q8_0_tail", 8, 3, 4096, "cfg1", False, "drift"),
]


def case_seed(k):
    """the BF16 seed tensor and imatrix of case k (regenerated identically by the tests)"""
    name, T, rows, cols, dist, use_imx, how = CASES[k]
    g = np.random.Generator(np.random.PCG64(0x9E5 + k))
    if dist == "cfg1":
        w = synth.normal_bf16(g, (rows, cols), 0.02, outlier_frac=0.001)
    else:
        w = synth.normal_bf16(g, (rows, cols), 0.02)
    imx = g.lognormal(0, 1, cols).astype(np.float32) if use_imx else None
    return g, w, imx


