"""HIP quantizers vs the golden vectors, the oracle and the reference digests (runs on the MI355X)."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

from oracle import quants
from seedpack_amd import device as dev
from seedpack_amd import synth
from seedpack_amd.gpuquant import GPUQuant, quantize_into
from seedpack_amd.requant import QFUN, row_size

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_TYPES = [8, 2, 3, 6, 7, 42, 10, 11, 12, 13, 14, 20, 23, 16, 17, 18, 19, 21, 22, 29]
NEED_IMX = {16, 17, 19}


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gq():
    return GPUQuant()


def hip(gq, t, bits, imx, variant=0):
    return gq.quantize_tensors(t, [(bits.reshape(-1), bits.shape[-1])], [imx], variant)[0]


@pytest.mark.parametrize("t", HIP_TYPES)
def test_hip_matches_golden_small(golden_small, gq, t):
    n = 0
    for name in ("normal", "student", "edge"):
        b = golden_small[f"in_{name}"]
        for variant in range(2 if t == 29 else 1):
            for use in ("none", "imx"):
                key = f"q_{name}_{t}_{variant}_{use}"
                if key not in golden_small:
                    continue
                say("case", key)
                got = hip(gq, t, b, golden_small["imatrix"] if use == "imx" else None, variant)
                want = golden_small[key]
                bad = np.flatnonzero(got != want)
                assert bad.size == 0, f"{key}: {bad.size} bytes differ, first at {bad[:8]}"
                n += 1
    assert n >= 3


@pytest.mark.parametrize("t", HIP_TYPES)
def test_hip_matches_oracle_seeded(gq, t):
    g = np.random.Generator(np.random.PCG64(0xA11CE + t))
    b = synth.normal_bf16(g, (96, 2048), 0.02, outlier_frac=0.002)
    imx = g.lognormal(0, 1, 2048).astype(np.float32)
    x = synth.bf16_to_f32(b).reshape(b.shape)
    for w in (None, imx):
        if w is None and t in NEED_IMX:
            continue
        for variant in range(2 if t == 29 else 1):
            say("case seeded", t, "imx" if w is not None else "none", "variant", variant)
            got = hip(gq, t, b, w, variant)
            want = quants.quantize(t, x, w, variant)
            bad = np.flatnonzero(got != want)
            assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


def _manifest():
    p = os.path.join(ROOT, "tests", "golden", "quant_sha256.json")
    return json.load(open(p)) if os.path.exists(p) else {}


@pytest.mark.parametrize("key", sorted(_manifest()))
def test_hip_full_size_matches_reference_digest(gq, key):
    ent = _manifest()[key]
    cfg, ti, t, variant = key.split("_")
    cfg, ti, t, variant = int(cfg[3:]), int(ti[1:]), int(t), int(variant)
    if t not in HIP_TYPES:
        pytest.skip(f"type {t} not built")
    say("case full", key)
    w, imx = synth.tensor(cfg, ti)
    got = hip(gq, t, w, imx, variant)
    assert got.size == ent["nbytes"]
    assert hashlib.sha256(got.tobytes()).hexdigest() == ent["sha256"]


@pytest.mark.parametrize("t", [8, 2, 12, 14])
def test_source_kinds_agree(gq, t):
    """bf16 bits, f32 and f16 copies of the same values give the same bytes"""
    g = np.random.Generator(np.random.PCG64(77))
    b = synth.normal_bf16(g, (16, 1024), 0.02)
    x = synth.bf16_to_f32(b).reshape(b.shape)
    imx = g.lognormal(0, 1, 1024).astype(np.float32)
    ref_bytes = hip(gq, t, b, imx)
    assert hip(gq, t, x, imx).tobytes() == ref_bytes.tobytes()
    xh = x.astype(np.float16)
    if np.array_equal(xh.astype(np.float32), x):
        assert hip(gq, t, xh, imx).tobytes() == ref_bytes.tobytes()


@pytest.mark.parametrize("t", [8, 2, 10, 12])
def test_row_split_invariance(gq, t):
    """rows are quantized independently: any split of the rows gives the same bytes"""
    g = np.random.Generator(np.random.PCG64(5))
    b = synth.normal_bf16(g, (37, 512), 0.02)
    imx = g.lognormal(0, 1, 512).astype(np.float32)
    whole = hip(gq, t, b, imx)
    rb = row_size(t, 512)
    for k in (1, 13, 36):
        a = hip(gq, t, b[:k], imx)
        c = hip(gq, t, b[k:], imx)
        assert np.concatenate([a, c]).tobytes() == whole.tobytes()
        assert a.size == k * rb


def test_zero_rows_is_a_no_op():
    src = dev.DeviceArray(512, np.uint16).zero()
    dst = dev.DeviceArray(16, np.uint8)
    quantize_into(12, dev.DeviceArray(0, np.uint16), 256, dst)
    dev.synchronize()
    del src


@pytest.mark.parametrize("t", [2, 3, 6, 7])
def test_legacy_imatrix_rows_with_half_tile(gq, t):
    """the BF16 row pre-pass of the imatrix legacy quantizers: rows of n_per_row % 64 == 32 (a half
    tile at the end) and a row count that leaves a partial workgroup, against the oracle; the F32 copy
    (the per-lane pre-pass) gives the same bytes"""
    g = np.random.Generator(np.random.PCG64(0xB0 + t))
    b = synth.normal_bf16(g, (70, 1056), 0.02, outlier_frac=0.002)
    imx = g.lognormal(0, 1, 1056).astype(np.float32)
    x = synth.bf16_to_f32(b).reshape(b.shape)
    say("case legacy half tile", t)
    got = hip(gq, t, b, imx)
    want = quants.quantize(t, x, imx)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"
    assert hip(gq, t, x, imx).tobytes() == got.tobytes()


@pytest.mark.parametrize("t", [2, 3, 6, 7])
def test_legacy_imatrix_with_and_without_scratch(gq, t):
    """the imatrix Q4_0/Q4_1/Q5_0/Q5_1 with the row mean squares from the first launch (scratch) and
    computed inside the quantizer (no scratch): the same bytes, equal to the oracle's, on row lengths
    that leave a partial 128-column tile (32, 96, 160, 4128) and row counts that leave a partial
    32-row group, for BF16, F16 and F32 sources"""
    from seedpack_amd._lib import check, lib
    g = np.random.Generator(np.random.PCG64(0xC0 + t))
    for rows, npr in ((1, 32), (31, 96), (33, 160), (70, 4128), (5, 12288)):
        b = synth.normal_bf16(g, (rows, npr), 0.02, outlier_frac=0.002)
        x = synth.bf16_to_f32(b).reshape(b.shape)
        imx = dev.DeviceArray.from_host(g.lognormal(0, 1, npr).astype(np.float32))
        want = quants.quantize(t, x, imx.to_host()) if rows * npr <= 70 * 4128 else None
        say("case legacy scratch", t, rows, npr)
        for kind, a in ((0, b), (1, x.astype(np.float16)), (2, x)):
            if kind == 1 and not np.array_equal(a.astype(np.float32), x):
                continue
            src = dev.DeviceArray.from_host(np.ascontiguousarray(a).reshape(-1))
            nbw = lib().spa_quantize_work_bytes(t, rows, npr, 1)
            assert nbw == (rows * 4 + 255) // 256 * 256
            work = dev.DeviceArray(nbw, np.uint8)
            outs = []
            for w in (work.ptr, None):
                dst = dev.DeviceArray(rows * row_size(t, npr), np.uint8)
                check(lib().spa_quantize(t, 0, src.ptr, kind, rows, npr, imx.ptr, dst.ptr, w, None))
                outs.append(dst.to_host())
            assert outs[0].tobytes() == outs[1].tobytes(), (t, rows, npr, kind)
            if want is not None:
                assert outs[0].tobytes() == want.tobytes(), (t, rows, npr, kind)


class _Lazy:
    """a quantized tensor as a quantizer input, dequantized into the launch's buffer (the reference's
    _Dequant, repo3.py:545-557)"""

    def __init__(self, gq, t, raw, npr):
        self.gq, self.t, self.raw, self.npr = gq, t, raw, npr
        self.size = raw.size // row_size(t, npr) * npr
        self.calls = 0

    def into(self, out):
        self.calls += 1
        self.gq.dequantize(self.t, self.raw, self.npr, out=out)


@pytest.mark.parametrize("t", [12, 14, 16])
def test_lazy_sources_and_launch_groups(gq, t):
    """sources written by into(out) (a seed's dequantized tensors) and groups of several tensors per
    device hand-over give the bytes of the same weights quantized one by one as float32 arrays; results
    arrive in order through on_result too"""
    say("case lazy sources", t)
    g = np.random.Generator(np.random.PCG64(40 + t))
    shapes = [(16, 256), (3, 512), (40, 256), (1, 1024), (9, 256)]
    seeds = [quants.quantize(14, (g.standard_normal(s) * 0.02).astype(np.float32), None) for s in shapes]
    lazies = [_Lazy(gq, 14, np.asarray(q, np.uint8), s[1]) for q, s in zip(seeds, shapes)]
    imx = [g.lognormal(0, 1, s[1]).astype(np.float32) for s in shapes]
    f32 = [gq.dequantize(14, np.asarray(q, np.uint8), s[1]).to_host().reshape(s) for q, s in zip(seeds, shapes)]
    want = [quants.quantize(t, x, w) for x, w in zip(f32, imx)]
    for mw in (1 << 28, 5000, 256):
        got = gq.quantize_tensors(t, [(z, s[1]) for z, s in zip(lazies, shapes)], imx, max_weights=mw)
        assert [a.tobytes() for a in got] == [np.asarray(w).tobytes() for w in want]
        seen = []
        gq.quantize_tensors(t, [(x.reshape(-1), s[1]) for x, s in zip(f32, shapes)], imx, max_weights=mw,
                            on_result=lambda k, y: seen.append((k, y.tobytes())))
        assert [k for k, _ in seen] == list(range(len(shapes)))
        assert [y for _, y in seen] == [np.asarray(w).tobytes() for w in want]
    assert all(z.calls == 3 for z in lazies)


def test_blocking_waits_give_the_same_bytes(gq):
    """with the library's waits blocking on an event (as the packer runs), host copies and stream
    waits hand over the same results as the spinning waits"""
    say("case blocking waits")
    g = np.random.Generator(np.random.PCG64(77))
    x = (g.standard_normal((64, 512)) * 0.02).astype(np.float32)
    imx = g.lognormal(0, 1, 512).astype(np.float32)
    want = np.asarray(quants.quantize(12, x, imx)).tobytes()
    prev = dev.set_blocking_waits(True)
    try:
        for _ in range(3):
            assert hip(gq, 12, x, imx).tobytes() == want
            back = dev.DeviceArray.from_host(x.reshape(-1)).to_host()
            assert back.tobytes() == x.tobytes()
    finally:
        dev.set_blocking_waits(prev)
    assert dev.set_blocking_waits(prev) is False
    assert hip(gq, 12, x, imx).tobytes() == want
