"""The M6 and context-rANS oracles (oracle/m6.py, oracle/rans.py) against the reference's own code run in
the build container (tests/golden/m6_vectors.npz, tests/golden/make_m6_golden.py), with planted mistakes;
and the product's host helpers of both codecs (split/join, table normalisation, the chunk's table and
xz framing) against the oracles, on the CPU."""
import json

import numpy as np
import pytest

from oracle import m6 as om6
from oracle import rans as orans
from seedpack_amd import crans, framing, m6, zstd
from tests.golden.m6_cases import CASES, RANS_CASES, case_file, o1_context, rans_case


@pytest.fixture(scope="module")
def gold():
    return np.load("tests/golden/m6_vectors.npz")


def _blocks(data, layout):
    d = np.frombuffer(data, np.uint8)
    return np.concatenate([d[o:o + nb] for o, nb, _, _ in layout["t"]]).reshape(-1, 34)


@pytest.mark.parametrize("name", CASES)
def test_oracle_m6_equals_reference(gold, name):
    parts = framing.unpack(memoryview(gold[f"{name}/chunk"].tobytes()))
    assert list(parts) == ["layout", "rest", "meta", "colmap", "used", "tables", "seglen", "stream"]
    layout = json.loads(zstd.decompress(parts["layout"]))
    data = case_file(name)
    r = om6.encode(_blocks(data, layout), layout)
    assert json.loads(zstd.decompress(parts["meta"])) == {"groups": r["groups"], "med": r["med"]}
    assert zstd.decompress(parts["colmap"]) == r["colmap"].tobytes()
    used = np.frombuffer(zstd.decompress(parts["used"]), np.uint32)
    assert np.array_equal(used, np.flatnonzero(r["counts"].sum(1)))
    raw = zstd.decompress(parts["tables"])
    assert raw[:12] == np.array([1, len(used), 256], np.uint32).tobytes()
    assert np.array_equal(np.frombuffer(raw, np.uint16, offset=12).reshape(-1, 256), r["freq"][used])
    assert np.array_equal(np.frombuffer(zstd.decompress(parts["seglen"]), np.uint16), r["lens"])
    assert bytes(parts["stream"]) == r["stream"]


def test_oracle_m6_planted_context_reset_fails(gold):
    # the hi context not reset at a segment's first block: the reference's stream is missed
    parts = framing.unpack(memoryview(gold["one/chunk"].tobytes()))
    layout = json.loads(zstd.decompress(parts["layout"]))
    r = om6.encode(_blocks(case_file("one"), layout), layout, plant=True)
    assert bytes(parts["stream"]) != r["stream"]


@pytest.mark.parametrize("name", RANS_CASES)
def test_oracle_rans_equals_reference(gold, name):
    sym, ctx, nctx, period = rans_case(name)
    f = orans.build_freqs(sym, ctx, nctx)
    assert np.array_equal(f, gold[f"rans/{name}/freq"])
    assert f.sum(1)[np.bincount(ctx, minlength=nctx) > 0].tolist() == [orans.PROB_SCALE] * int((np.bincount(ctx, minlength=nctx) > 0).sum())
    enc = orans.encode(sym, ctx, f)
    assert enc == gold[f"rans/{name}/stream"].tobytes()
    assert np.array_equal(orans.decode(enc, ctx, f, n=len(sym), period=period), sym)


def test_oracle_rans_planted_o1_reset_fails(gold):
    sym, _, nctx, period = rans_case("o1")
    ctx = orans.o1_context(sym, period, plant=True)
    f = orans.build_freqs(sym, ctx, nctx)
    assert orans.encode(sym, ctx, f) != gold["rans/o1/stream"].tobytes()


def test_o1_contexts_agree():
    sym, ctx, _, period = rans_case("o1")
    assert np.array_equal(orans.o1_context(sym, period), ctx)
    assert np.array_equal(crans.o1_context(sym, period), ctx)
    assert np.array_equal(o1_context(sym, period), ctx)


def test_product_table_normalisation_equals_oracle():
    g = np.random.default_rng(3)
    for _ in range(20):
        c = g.integers(0, 50, (5, 256)) * (g.random((5, 256)) < 0.3)
        c[1] = 0
        c[2, :3] = [1, 1, 100000]                                  # drift taken from the largest
        assert np.array_equal(m6.normalize(c), om6.normalize(c))
        assert np.array_equal(crans.normalize(c), orans.normalize(c))
        f = m6.normalize(c)
        assert (f.sum(1)[c.sum(1) > 0] == 1 << m6.PB).all() and (f[c > 0] >= 1).all() and (f[c == 0] == 0).all()


@pytest.mark.parametrize("name", CASES)
def test_product_split_join_and_framing(name):
    data = case_file(name)
    layout, rest, blocks = m6.split(data)
    assert m6.join(layout, rest, blocks) == data
    offs = [t[0] for t in layout["t"]]
    assert offs == sorted(offs) and all(t[1] % 34 == 0 for t in layout["t"])      # the Q8_0 tensors by offset
    assert len(rest) + blocks.size == len(data)
    assert m6.xz_d(m6.xz_c(rest)) == rest
    tabs = [np.arange(512, dtype=np.uint16).reshape(2, 256), np.ones((3, 256), np.uint16)]
    back = m6.tables_d(m6.tables_c(tabs))
    assert all(np.array_equal(a, b) for a, b in zip(tabs, back))
