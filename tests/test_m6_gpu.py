"""M6 (csrc/m6.hip + seedpack_amd/m6.py) and the context-mixed rANS (spa_crans_* + seedpack_amd/crans.py)
on the MI355X, byte for byte against the reference's own code (tests/golden/m6_vectors.npz, written by
tests/golden/make_m6_golden.py: gpu_codec.M6GPU through its --cpu backend, rans.py's coder)."""
import sys

import numpy as np
import pytest

from seedpack_amd import crans, m6
from tests.golden.m6_cases import CASES, RANS_CASES, case_file, rans_case

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gold():
    return np.load("tests/golden/m6_vectors.npz")


@pytest.mark.parametrize("name", CASES)
def test_m6_equals_reference(gold, name):
    say("case m6", name)
    data = case_file(name)
    got = m6.M6().compress(data)
    assert got == gold[f"{name}/chunk"].tobytes()
    assert m6.M6().decompress(gold[f"{name}/chunk"].tobytes()) == data


def test_m6_multi_segment_round_trip():
    say("case m6 round trip, 3 files")
    for name in CASES:
        data = case_file(name)
        assert m6.M6().decompress(m6.M6().compress(data)) == data


@pytest.mark.parametrize("name", RANS_CASES)
def test_crans_equals_reference(gold, name):
    say("case crans", name)
    sym, ctx, nctx, period = rans_case(name)
    f = crans.build_freqs(sym, ctx, nctx)
    assert np.array_equal(f, gold[f"rans/{name}/freq"])
    enc = crans.encode(sym, ctx, f)
    assert enc == gold[f"rans/{name}/stream"].tobytes()
    dec = crans.decode_o1(enc, len(sym), f, period) if period else crans.decode(enc, ctx, f)
    assert np.array_equal(dec, sym)


def test_crans_batch_equals_single(gold):
    say("case crans batch")
    items, dec_items, want = [], [], []
    for name in RANS_CASES:
        sym, ctx, nctx, period = rans_case(name)
        f = gold[f"rans/{name}/freq"]
        items.append((sym, ctx, f))
        dec_items.append((gold[f"rans/{name}/stream"].tobytes(), None if period else ctx, f, len(sym), period))
        want.append(sym)
    enc = crans.encode_many(items)
    assert [e == gold[f"rans/{n}/stream"].tobytes() for e, n in zip(enc, RANS_CASES)] == [True] * len(RANS_CASES)
    for got, w in zip(crans.decode_many(dec_items), want):
        assert np.array_equal(got, w)
    # an empty stream codes to the initial state's four bytes
    e = crans.encode(np.zeros(0, np.uint8), np.zeros(0, np.int32), np.full((1, 256), 64, np.uint16))
    assert e == (1 << 23).to_bytes(4, "big")
