"""The C restatement of the lattice i-quants (oracle/iq_grid.c) against the reference fixture's table
digests, brute force, the golden vectors, the reference's own C build, and planted mistakes."""
import hashlib
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import iq_grid, ref
from seedpack_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAMES = ["iq2_data_0", "iq2_data_1", "iq2_data_2", "iq2_data_3", "iq3_data_0", "iq3_data_1"]
GRID = [16, 17, 22, 18, 21, 19, 29]
NEED_IMX = {16, 17, 19}


@pytest.mark.parametrize("li", range(6))
def test_tables_equal_reference_fixture(li):
    man = json.load(open(os.path.join(ROOT, "tests", "golden", "iqtables_sha256.json")))
    pt, kmap, nb = iq_grid.table(li)
    g = pt.view(np.uint64 if li < 4 else np.uint32)
    assert hashlib.sha256(g.tobytes()).hexdigest() == man[NAMES[li] + "_grid"]["sha256"]
    assert hashlib.sha256(kmap.tobytes()).hexdigest() == man[NAMES[li] + "_map"]["sha256"]
    assert nb.size == man[NAMES[li] + "_nb"]["n"]
    assert hashlib.sha256(nb.tobytes()).hexdigest() == man[NAMES[li] + "_nb"]["sha256"]


@pytest.mark.parametrize("li,dim,bits,nwant", [(2, 8, 2, 3), (5, 4, 3, 3)])
def test_neighbour_lists_by_brute_force(li, dim, bits, nwant):
    """every list holds the points at the nwant smallest distinct squared distances, by (distance, point)"""
    pt, kmap, nb = iq_grid.table(li)
    pts = pt.reshape(-1, dim).astype(np.int64)
    g = np.random.Generator(np.random.PCG64(li))
    off = np.flatnonzero(kmap < 0)
    for u in g.choice(off, 40, replace=False):
        pos = 2 * ((u >> (bits * np.arange(dim))) & ((1 << bits) - 1)) + 1
        d2 = ((pts - pos) ** 2).sum(1)
        o = -kmap[u] - 1
        want = [j for d in np.unique(d2)[:nwant] for j in np.flatnonzero(d2 == d)]
        assert list(nb[o + 1:o + 1 + nb[o]]) == want


def test_half_conversion_matches_numpy():
    g = np.random.Generator(np.random.PCG64(3))
    v = np.concatenate([g.standard_normal(3000).astype(np.float32) * np.float32(10.0) ** g.integers(-9, 6, 3000),
                        np.array([0.0, -0.0, 65504, 65519.99, 65520, 6.1035156e-05, 5.96e-08, 2.9802322e-08,
                                  2.9802326e-08, 1e-30, np.inf, -np.inf], np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    got = np.array([iq_grid.half_bits(a) for a in v], np.uint16)
    assert np.array_equal(got, want)
    assert iq_grid.half_bits(float("nan")) == 0x7E00


def _golden_cases(golden, t):
    for name in ("normal", "student", "edge"):
        b = golden[f"in_{name}"]
        x = synth.bf16_to_f32(b).reshape(b.shape)
        for variant in range(2 if t == 29 else 1):
            for use in ("none", "imx"):
                key = f"q_{name}_{t}_{variant}_{use}"
                if key in golden:
                    yield key, x, (golden["imatrix"] if use == "imx" else None), variant, golden[key]


@pytest.mark.parametrize("t", GRID)
def test_restatement_matches_golden(golden_small, t):
    n = 0
    for key, x, imx, variant, want in _golden_cases(golden_small, t):
        got = iq_grid.quantize(t, x, imx, variant)
        assert got.tobytes() == want.tobytes(), key
        n += 1
    assert n >= 3


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("t", GRID)
def test_restatement_matches_reference_build(t):
    g = np.random.Generator(np.random.PCG64(4321 + t))
    rows = [synth.bf16_to_f32(synth.student_t_bf16(g, (24, 1024))).reshape(24, 1024),
            synth.bf16_to_f32(synth.normal_bf16(g, (24, 1024), 0.02, outlier_frac=0.01)).reshape(24, 1024)]
    x = np.concatenate(rows)
    x[3, :300] = 0                       # whole zero sub-blocks and a zero super-block part
    x[5, 256:512] = 1e-9                 # below every type's skip threshold but IQ3_S's
    x[7, :32] = np.float32(0.0078125)    # equal values: sort ties, flat groups
    imx = g.lognormal(0, 1, 1024).astype(np.float32)
    for w in (None, imx):
        if w is None and t in NEED_IMX:
            continue
        for variant in range(2 if t == 29 else 1):
            want = ref.quantize(t, x, w, variant=variant) if variant else ref.quantize(t, x, w)
            assert iq_grid.quantize(t, x, w, variant).tobytes() == want.tobytes(), (w is None, variant)


def test_missing_imatrix_is_an_error():
    x = np.ones((1, 256), np.float32)
    for t in NEED_IMX:
        with pytest.raises(ValueError):
            iq_grid.quantize(t, x, None)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
@pytest.mark.parametrize("plant,t", [(1, 17), (2, 21), (3, 16)])
def test_planted_mistake_fails_golden(golden_small, tmp_path, plant, t):
    """1: IQ2_XS without the sign-parity fix; 2: IQ3_S refitting only its off-grid groups; 3: IQ2_XXS
    starting from max/5 instead of make_qp_quants -- each must change a golden vector"""
    so = str(tmp_path / f"plant{plant}.so")
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fPIC", "-shared", f"-DOG_PLANT={plant}", "-o", so,
                    os.path.join(ROOT, "oracle", "iq_grid.c"), "-lm"], check=True)
    wrong = iq_grid.Planted(so)
    differs = 0
    for key, x, imx, variant, want in _golden_cases(golden_small, t):
        assert iq_grid.quantize(t, x, imx, variant).tobytes() == want.tobytes(), key
        differs += wrong.quantize(t, x, imx, variant).tobytes() != want.tobytes()
    assert differs > 0
