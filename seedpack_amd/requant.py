"""Quant type table of the path (seedpack/requant.py:21-29 in the reference).

QFUN maps a ggml type id to (quantize function name, block elements, block bytes). The names and
numbers are the llama.cpp/GGUF format constants and must stay identical.
"""
QFUN = {2: ("quantize_q4_0", 32, 18), 3: ("quantize_q4_1", 32, 20), 6: ("quantize_q5_0", 32, 22),
        7: ("quantize_q5_1", 32, 24), 8: ("quantize_q8_0", 32, 34), 10: ("quantize_q2_K", 256, 84),
        11: ("quantize_q3_K", 256, 110), 12: ("quantize_q4_K", 256, 144), 13: ("quantize_q5_K", 256, 176),
        14: ("quantize_q6_K", 256, 210), 16: ("quantize_iq2_xxs", 256, 66), 17: ("quantize_iq2_xs", 256, 74),
        18: ("quantize_iq3_xxs", 256, 98), 19: ("quantize_iq1_s", 256, 50), 20: ("quantize_iq4_nl", 32, 18),
        21: ("quantize_iq3_s", 256, 110), 22: ("quantize_iq2_s", 256, 82), 23: ("quantize_iq4_xs", 256, 136),
        29: ("quantize_iq1_m", 256, 56), 42: ("quantize_q2_0", 64, 18)}

NAMES = {t: f[len("quantize_"):].upper() for t, (f, _, _) in QFUN.items()}
BY_NAME = {v: k for k, v in NAMES.items()}

# types whose quantizer asserts an imatrix (ggml-quants.c:3303, :3481, :4528)
NEED_IMATRIX = {16, 17, 19}

# quantizer variants per type (seedpack/gpuquant.py:182-185): IQ1_M also has the pre-f95b0d9539 search
VARIANTS = {29: 2}


def row_size(ttype, n_per_row):
    _, qk, bs = QFUN[ttype]
    assert n_per_row % qk == 0, (ttype, n_per_row)
    return n_per_row // qk * bs
