"""The QR coder with seeds other than a BF16 base, on the MI355X, against the reference's own QR
kernels (tests/golden/qr_seed_vectors.npz, written by make_qr_seed_golden.py through the reference's
--cpu backend): no seed (the column RMS, seed type 98), explicit (value, uncertainty) seeds (99) and
quantized seeds; the per-weight kernels intervals / grid_h / weight_equal / block_fields; and the
seed-less codec qr.self_encode / self_decode."""
import os
import sys

import numpy as np
import pytest

from seedpack_amd import device as dev
from seedpack_amd import qr
from seedpack_amd._lib import check, lib
from tests.golden.qr_seed_cases import AUX_TYPES, EXPLICIT_CASES, GRID_AUX_TYPES, QSEED_CASES, SELF_CASES, inputs

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(ROOT, "tests", "golden", "qr_seed_vectors.npz"))


def _check(T, F, P, seed, seed_type, cols, g, key):
    items = [(dev.DeviceArray.from_host(F), dev.DeviceArray.from_host(P), 0, seed_type, cols)]
    sd = dev.DeviceArray.from_host(np.ascontiguousarray(seed).view(np.uint8))
    p = qr.encode_parts(T, items, sd)
    assert np.array_equal(p["counts"], g[f"{key}/counts"]), "counts"
    assert np.array_equal(p["used"], g[f"{key}/used"]) and np.array_equal(p["freq"], g[f"{key}/freq"]), "tables"
    assert np.array_equal(p["lens"], g[f"{key}/lens"]), "segment lengths"
    assert np.array_equal(p["stream"], g[f"{key}/stream"]), "stream"
    back = qr.decode_parts(T, p["freq"], p["used"], p["lens"], p["stream"].tobytes(),
                           [(dev.DeviceArray.from_host(P), 0, seed_type, cols)], sd)
    assert np.array_equal(back.to_host()[:len(F)], F), "decode"


@pytest.mark.parametrize("k", range(len(SELF_CASES)))
def test_no_seed_equals_reference(gold, k):
    name, T, rows, cols = SELF_CASES[k]
    say("case qr no seed", name)
    key = f"self_{name}"
    F = gold[f"{key}/F"]
    rms, tpl, r = qr.self_side(T, dev.DeviceArray.from_host(F), cols)
    assert r == rows
    assert np.array_equal(rms.view(np.uint16), gold[f"{key}/rms"]), "column RMS"
    assert np.array_equal(tpl, gold[f"{key}/tpl"]), "template blocks"
    _check(T, F, np.tile(tpl, rows), rms.astype(np.float32), qr.COLRMS, cols, gold, key)


@pytest.mark.parametrize("k", range(len(EXPLICIT_CASES)))
def test_explicit_seed_equals_reference(gold, k):
    name, T, rows, cols = EXPLICIT_CASES[k]
    say("case qr explicit seed", name)
    key = f"explicit_{name}"
    _check(T, gold[f"{key}/F"], gold[f"{key}/P"], gold[f"{key}/seed"], qr.EXPLICIT, cols, gold, key)


@pytest.mark.parametrize("k", range(len(QSEED_CASES)))
def test_quantized_seed_equals_reference(gold, k):
    name, T, S, rows, cols = QSEED_CASES[k]
    say("case qr quantized seed", name)
    key = f"qseed_{name}"
    _check(T, gold[f"{key}/F"], gold[f"{key}/P"], gold[f"{key}/seed"], S, cols, gold, key)


def test_per_weight_kernels_equal_reference(gold):
    for T in AUX_TYPES:
        F, P = gold[f"aux_{T}/F"], gold[f"aux_{T}/P"]
        nw = 8 * 512
        lo, hi = qr.intervals(T, F, nw)
        # (bit patterns: a damaged fp16 scale makes NaN bounds)
        assert np.array_equal(lo.to_host().view(np.uint32), gold[f"aux_{T}/lo"].view(np.uint32)), T
        assert np.array_equal(hi.to_host().view(np.uint32), gold[f"aux_{T}/hi"].view(np.uint32)), T
        weq = qr.weight_equal(T, dev.DeviceArray.from_host(F), dev.DeviceArray.from_host(P), nw)
        assert np.array_equal(weq.to_host(), gold[f"aux_{T}/weq"]), T
        fl = dev.DeviceArray(len(gold[f"aux_{T}/fields"]), np.int32)
        Fd = dev.DeviceArray.from_host(F)
        check(lib().spa_qr_block_fields(T, Fd.ptr, len(F) // qr.BS[T], fl.ptr, None))
        assert np.array_equal(fl.to_host(), gold[f"aux_{T}/fields"]), T
        assert lib().spa_qr_nfields(T) == qr.NFIELDS[T]
    for T in GRID_AUX_TYPES:
        F = gold[f"grid_{T}/F"]
        h = qr.grid_half_steps(T, dev.DeviceArray.from_host(F), 4 * 512)
        assert np.array_equal(h.to_host().view(np.uint32), gold[f"grid_{T}/h"].view(np.uint32)), T


def test_self_encode_round_trip():
    """several tensors of one type in one call (batches cut as the reference cuts them), decoded back"""
    from oracle import ref
    say("case qr self codec")
    tens = []
    for k, (rows, cols) in enumerate([(16, 1024), (8, 512), (40, 2048)]):
        x, imx = inputs("self", 100 + k, rows, cols)
        tens.append((ref.quantize(12, x, imx), cols))
    buf = qr.self_encode(12, tens)
    back = qr.self_decode(12, buf)
    assert len(back) == 3
    for (b, _), d in zip(tens, back):
        assert np.array_equal(d.to_host(), b)
