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
    # grid types (the E8 / D4 lattice codes): Student-t seeds as configuration 3, with the imatrix
    ("iq2_xxs", 16, 64, 1024, "cfg3", True, "perturb"), ("iq2_xs", 17, 64, 1024, "cfg3", True, "perturb"),
    ("iq2_s", 22, 64, 1024, "cfg3", True, "perturb"), ("iq3_xxs", 18, 64, 1024, "cfg3", True, "perturb"),
    ("iq3_s", 21, 64, 1024, "cfg3", True, "perturb"), ("iq1_s", 19, 64, 1024, "cfg3", True, "perturb"),
    ("iq1_m", 29, 64, 1024, "cfg3", True, "perturb"),
    ("iq2_xxs_drift", 16, 4, 1024, "cfg3", True, "drift"), ("iq2_xs_drift", 17, 4, 1024, "cfg3", True, "drift"),
    ("iq2_s_drift", 22, 4, 1024, "cfg3", True, "drift"), ("iq3_xxs_drift", 18, 4, 1024, "cfg3", True, "drift"),
    ("iq3_s_drift", 21, 4, 1024, "cfg3", True, "drift"), ("iq1_s_drift", 19, 4, 1024, "cfg3", True, "drift"),
    ("iq1_m_drift", 29, 4, 1024, "cfg3", True, "drift"),
    ("iq2_s_var", 22, 4, 1024, "cfg3", True, "variant"), ("iq3_s_var", 21, 4, 1024, "cfg3", True, "variant"),
    ("iq1_m_var", 29, 4, 1024, "cfg3", True, "variant"), ("iq3_xxs_var", 18, 4, 1024, "cfg3", True, "variant"),
]
GRID = {16, 17, 18, 19, 21, 22, 29}


def case_seed(k):
    """the BF16 seed tensor and imatrix of case k (regenerated identically by the tests)"""
    name, T, rows, cols, dist, use_imx, how = CASES[k]
    g = np.random.Generator(np.random.PCG64(0x9E5 + k))
    if dist == "cfg1":
        w = synth.normal_bf16(g, (rows, cols), 0.02, outlier_frac=0.001)
    elif dist == "cfg3":
        w = synth.student_t_bf16(g, (rows, cols))
    else:
        w = synth.normal_bf16(g, (rows, cols), 0.02)
    imx = g.lognormal(0, 1, cols).astype(np.float32) if use_imx else None
    return g, w, imx


