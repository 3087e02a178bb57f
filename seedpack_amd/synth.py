"""Seeded synthetic inputs of the benchmark configurations (BF16 weights + imatrix).

Values are drawn in float64 with numpy's PCG64 at seed 0x5EED0000 + 16*config + tensor, cast to
float32 and rounded to BF16 with round-to-nearest-even, (u + 0x7FFF + ((u >> 16) & 1)) >> 16 -- the
rounding the reference applies to float tensors (seedpack/repo2.py:46-48). An imatrix is one
LogNormal(0, 1) float32 per input column.
"""
import numpy as np

SEED0 = 0x5EED0000


def rng(config, tensor=0):
    return np.random.Generator(np.random.PCG64(SEED0 + 16 * config + tensor))


def bf16_bits(x):
    """float32 -> bf16 bits (uint16), round to nearest even"""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(g, shape, std, outlier_frac=0.0, outlier_std=0.5):
    x = g.normal(0.0, std, size=shape)
    if outlier_frac:
        n = x.size
        k = int(round(n * outlier_frac))
        idx = g.choice(n, size=k, replace=False)
        x.reshape(-1)[idx] = g.normal(0.0, outlier_std, size=k)
    return bf16_bits(x.astype(np.float32))


def student_t_bf16(g, shape, df=5, std=0.015):
    x = g.standard_t(df, size=shape) * (std / np.sqrt(df / (df - 2.0)))
    return bf16_bits(x.astype(np.float32))


def imatrix(g, ncols):
    return g.lognormal(0.0, 1.0, size=ncols).astype(np.float32)


# config -> tensors (name, rows, cols); cols = n_per_row, rows back to back (row-major)
SHAPES = {
    1: [("blk.0.ffn_up", 3072, 1024)],
    2: [("token_embd", 151936, 1024), ("blk.0.ffn_down", 1024, 3072)],
    3: [("blk.0.ffn_up", 4096, 12288), ("blk.0.ffn_down", 12288, 4096)],
}

TYPES = {
    1: [8, 2],                          # Q8_0, Q4_0 (no imatrix)
    2: [10, 11, 12, 13, 14],            # Q2_K .. Q6_K
    3: [23, 18, 17, 16, 19, 29],        # IQ4_XS, IQ3_XXS, IQ2_XS, IQ2_XXS, IQ1_S, IQ1_M
}


def tensor(config, index, rows=None):
    """(bf16 bits (rows, cols), imatrix or None) of tensor `index` of a config; `rows` takes the
    first rows only (same generator stream)"""
    name, r, c = SHAPES[config][index]
    g = rng(config, index)
    r = r if rows is None else min(rows, r)
    if config == 1:
        w = normal_bf16(g, (r, c), 0.02, outlier_frac=0.001)
        return w, None
    if config == 2:
        w = normal_bf16(g, (r, c), 0.02)
    else:
        w = student_t_bf16(g, (r, c))
    return w, imatrix(g, c)
