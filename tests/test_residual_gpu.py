"""The device residual stage (spa_xor / spa_xor3 / spa_diff_count / spa_count_every / spa_float_pred and the
per-tensor variant choice) on the MI355X, against numpy on the host."""
import sys

import numpy as np
import pytest

from seedpack_amd import device as dev
from seedpack_amd import residual as r
from seedpack_amd import synth
from seedpack_amd.gpuquant import GPUQuant

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.mark.parametrize("n,off", [(0, 0), (1, 0), (17, 0), (4096, 0), (4096, 3), (1 << 20, 0), ((1 << 20) + 5, 1)])
def test_xor_and_counts(n, off):
    say("case residual kernels", n, off)
    g = np.random.Generator(np.random.PCG64(n + off))
    a, b, c = (g.integers(0, 256, n + off, dtype=np.uint8) for _ in range(3))
    b[: (n + off) // 2] = a[: (n + off) // 2]                             # half the bytes equal
    da, db, dc = (dev.DeviceArray.from_host(x) for x in (a, b, c))
    va, vb, vc = (x.view(off, (n,), np.uint8) for x in (da, db, dc))
    want = a[off:] ^ b[off:]
    assert r.diff_count(va, vb) == int(np.count_nonzero(want))
    assert r.diff_count(va) == int(np.count_nonzero(a[off:]))
    dst = dev.DeviceArray(n + off, np.uint8).view(off, (n,), np.uint8)
    assert r.xor_into(dst, va, vb) == int(np.count_nonzero(want))
    assert np.array_equal(dst.to_host(), want)
    w3 = want ^ c[off:]
    assert r.xor3_into(dst, va, vb, vc) == int(np.count_nonzero(w3))
    assert np.array_equal(dst.to_host(), w3)
    assert r.xor_into(va, va, vb) == int(np.count_nonzero(want))         # in place
    assert np.array_equal(va.to_host(), want)
    # the residual frame's level sample: every 61st byte (np.count_nonzero(v[::61]))
    from seedpack_amd._lib import check, lib
    cnt = dev.DeviceArray(1, np.uint64)
    for stride in (1, 61, 4096):
        check(lib().spa_count_every(va.ptr, n, stride, cnt.ptr, None))
        assert int(cnt.to_host()[0]) == int(np.count_nonzero(want[::stride])), stride     # va holds want now


def test_float_predictions():
    g = np.random.Generator(np.random.PCG64(8))
    x = np.concatenate([g.normal(0, 1, 5000), [0.0, -0.0, 65504.0, 65520.0, 1e5, -1e5, 6e-8, 1e-9, np.inf, -np.inf]])
    b = synth.bf16_bits(x.astype(np.float32))
    xf = synth.bf16_to_f32(b)
    src = dev.DeviceArray.from_host(b)
    assert r.float_prediction(src, r.F32).to_host().view(np.float32).tobytes() == xf.tobytes()
    assert r.float_prediction(src, r.F16).to_host().view(np.uint16).tobytes() == xf.astype(np.float16).view(np.uint16).tobytes()
    u = xf.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert r.float_prediction(src, r.BF16).to_host().view(np.uint16).tobytes() == want.tobytes()
    # F32 weights to BF16: the rounding formula on values that are not BF16 already
    x32 = g.normal(0, 1, 4096).astype(np.float32)
    u = x32.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    got = r.float_prediction(dev.DeviceArray.from_host(x32), r.BF16).to_host().view(np.uint16)
    assert got.tobytes() == want.tobytes()


def test_float_prediction_f16_every_bit_pattern():
    """F16 prediction of every BF16 and every F16 bit pattern (NaNs included) equals numpy's astype, the
    call of the reference's --cpu path (repo3.py:685); F32 NaNs with payloads only in the low 13 bits
    become 0x7C01 | sign"""
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    with np.errstate(all="ignore"):
        want = (b.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)
    got = r.float_prediction(dev.DeviceArray.from_host(b), r.F16).to_host().view(np.uint16)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(b[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    h = b.view(np.float16)
    got = r.float_prediction(dev.DeviceArray.from_host(h), r.F16).to_host().view(np.uint16)
    assert got.tobytes() == h.astype(np.float32).astype(np.float16).view(np.uint16).tobytes()
    f = np.array([0x7F800001, 0xFF800FFF, 0x7FC00000, 0x7FBFFFFF, 0xFFFFFFFF, 0x7F802000], np.uint32).view(np.float32)
    with np.errstate(all="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    got = r.float_prediction(dev.DeviceArray.from_host(f), r.F16).to_host().view(np.uint16)
    assert got.tobytes() == want.tobytes() and list(want[:2]) == [0x7C01, 0xFC01], [hex(v) for v in got]


def _case(t_type, rows=64, cols=1024, seed=3):
    g = np.random.Generator(np.random.PCG64(seed + t_type))
    w = synth.student_t_bf16(g, (rows, cols)) if t_type in (16, 17, 18, 19, 21, 22, 29) else synth.normal_bf16(g, (rows, cols), 0.02)
    imx = g.lognormal(0, 1, cols).astype(np.float32)
    return g, w, imx


def _tensor(t_type, file_bytes, w, imx, cols):
    region = dev.DeviceArray.from_host(file_bytes)
    base = dev.DeviceArray.from_host(w.reshape(-1))
    return r.Tensor("t", t_type, cols, region, base, imatrix=imx), region


def test_exact_prediction_leaves_zero_residual():
    gq = GPUQuant()
    _, w, imx = _case(12)
    f = gq.quantize_tensors(12, [(w.reshape(-1), 1024)], [imx])[0]
    t, region = _tensor(12, f, w, imx, 1024)
    out = r.residual_tensor(t, gq)
    assert out["kind"] == "rq" and out["variant"] == 0 and not out["nonzero"] and not out["qr"]
    assert not region.to_host().any()


def test_perturbed_goes_to_qr_with_file_bytes_kept():
    gq = GPUQuant()
    g, w, imx = _case(12)
    p = gq.quantize_tensors(12, [(w.reshape(-1), 1024)], [imx])[0]
    f = p.copy()
    idx = g.choice(f.size, 40, replace=False)
    f[idx] ^= 0x11
    t, region = _tensor(12, f, w, imx, 1024)
    out = r.residual_tensor(t, gq)
    assert out["qr"] and out["kind"] == "qr" and out["diff_bytes"] == 40
    assert region.to_host().tobytes() == f.tobytes()
    assert out["prediction"].to_host().tobytes() == p.tobytes()
    # without the QR coder: the XOR residual in place
    t, region = _tensor(12, f, w, imx, 1024)
    out = r.residual_tensor(t, gq, use_qr=False)
    assert out["kind"] == "rq" and out["nonzero"] and not out["qr"]
    assert region.to_host().tobytes() == (f ^ p).tobytes()


def test_iq1_m_older_variant_is_found():
    """the two IQ1_M searches rarely disagree: configuration 3's first 64 rows hold one such block"""
    gq = GPUQuant()
    w, imx = synth.tensor(3, 0, rows=64)
    cols = w.shape[1]
    f = gq.quantize_tensors(29, [(w.reshape(-1), cols)], [imx], variant=1)[0]
    assert f.tobytes() != gq.quantize_tensors(29, [(w.reshape(-1), cols)], [imx])[0].tobytes()
    t, region = _tensor(29, f, w, imx, cols)
    out = r.residual_tensor(t, gq)
    assert out["variant"] == 1 and not out["nonzero"] and not region.to_host().any()
    # through the XOR route: file ^ p0 ^ p1 = 0 after the retry
    t, region = _tensor(29, f, w, imx, cols)
    out = r.residual_tensor(t, gq, use_qr=False)
    assert out["variant"] == 1 and not out["nonzero"] and not region.to_host().any()


def test_no_imatrix_tries_unit_weights_then_unweighted():
    gq = GPUQuant()
    _, w, _ = _case(14)
    f = gq.quantize_tensors(14, [(w.reshape(-1), 1024)], [None])[0]     # the file made without imatrix
    t, region = _tensor(14, f, w, None, 1024)
    out = r.residual_tensor(t, gq)
    assert out["variant"] == 0 and not out["nonzero"] and not region.to_host().any()
    ones = gq.quantize_tensors(14, [(w.reshape(-1), 1024)], [np.ones(1024, np.float32)])[0]
    t, region = _tensor(14, ones, w, None, 1024)                           # made with unit weights
    out = r.residual_tensor(t, gq)
    assert out["variant"] == r.UNIT_W and not out["nonzero"]


def test_float_tensor_xor():
    gq = GPUQuant()
    _, w, _ = _case(1)
    x = synth.bf16_to_f32(w).reshape(-1)
    f = x.astype(np.float16).view(np.uint8).copy()
    f[7] ^= 1
    t = r.Tensor("n", r.F16, 1024, dev.DeviceArray.from_host(f), dev.DeviceArray.from_host(w.reshape(-1)))
    out = r.residual_tensor(t, gq)
    assert out["kind"] == "xor" and out["nonzero"]
    res = t.region.to_host()
    assert np.flatnonzero(res).tolist() == [7] and res[7] == 1


def test_window_matches_per_tensor():
    """residual_window (counts read back once) makes residual_tensor's decisions on a mixed window:
    exact, perturbed (QR and XOR routes), the IQ1_M variant retry, no imatrix, a float tensor"""
    say("case residual window")
    gq = GPUQuant()
    g, w12, imx12 = _case(12)
    p12 = gq.quantize_tensors(12, [(w12.reshape(-1), 1024)], [imx12])[0]
    f12 = p12.copy()
    f12[g.choice(f12.size, 40, replace=False)] ^= 0x11
    w29, imx29 = synth.tensor(3, 0, rows=64)
    c29 = w29.shape[1]
    f29 = gq.quantize_tensors(29, [(w29.reshape(-1), c29)], [imx29], variant=1)[0]
    _, w14, _ = _case(14)
    f14 = gq.quantize_tensors(14, [(w14.reshape(-1), 1024)], [np.ones(1024, np.float32)])[0]
    _, w1, _ = _case(1)
    f1 = synth.bf16_to_f32(w1).reshape(-1).astype(np.float16).view(np.uint8).copy()
    f1[7] ^= 1
    specs = [(12, p12, w12, imx12, 1024), (12, f12, w12, imx12, 1024), (29, f29, w29, imx29, c29),
             (14, f14, w14, None, 1024), (r.F16, f1, w1, None, 1024)]
    for use_qr in (True, False):
        one = [_tensor(t, f, w, m, c) for (t, f, w, m, c) in specs]
        many = [_tensor(t, f, w, m, c) for (t, f, w, m, c) in specs]
        a = [r.residual_tensor(t, gq, use_qr=use_qr) for (t, _) in one]
        b = r.residual_window([t for (t, _) in many], gq, use_qr=use_qr)
        for (x, (_, ra)), (y, (_, rb)) in zip(zip(a, one), zip(b, many)):
            for key in ("kind", "variant", "nonzero", "qr", "diff_bytes"):
                assert x.get(key) == y.get(key), (key, x.get(key), y.get(key))
            assert ra.to_host().tobytes() == rb.to_host().tobytes()
            if x["qr"]:
                assert x["prediction"].to_host().tobytes() == y["prediction"].to_host().tobytes()

