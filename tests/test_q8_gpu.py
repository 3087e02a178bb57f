"""M22, the Q8_0 codec of Q8Parts and of seeds (seedpack_amd/q8.py), on the MI355X: every coded part
(side information, planner output, tables, lengths and the three phases' streams) equals the
reference's own (tests/golden/q8_vectors.npz, written by make_q8_golden.py, which runs the reference's
gpu2.py / gpu3.py through its --cpu backend), part by part, and the reference's chunks decode back to
the exact tensor bytes. The int8 similarity product of the row planner is checked against numpy's
exact integer product, and its top-4 choice against a brute-force ranking."""
import os
import sys

import numpy as np
import pytest

from seedpack_amd import device as dev
from seedpack_amd import framing, q8, zstd
from seedpack_amd._lib import check, lib
from tests.golden.q8_cases import CASES, case_file

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ZSTD_PARTS = ("layout", "side", "cfi", "lens", "scls", "Clens", "Cside", "Cpar", "Ccoef", "Cfbin", "Cmu", "Ccadj")


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(ROOT, "tests", "golden", "q8_vectors.npz"))


def _groups(layout, budget):
    return q8.Q8Parts(budget).groups(layout)


def _compare(mine, want, label):
    a, b = framing.unpack(mine), framing.unpack(want)
    assert list(a) == list(b), f"{label}: part names {list(a)} vs {list(b)}"
    for k in b:
        x, y = bytes(a[k]), bytes(b[k])
        if k in ZSTD_PARTS:
            x, y = zstd.decompress(x), zstd.decompress(y)
        if k in ("tables", "Ctables"):
            x, y = zstd.decompress(x), zstd.decompress(y)
        if x != y:
            n = min(len(x), len(y))
            first = next((i for i in range(n) if x[i] != y[i]), n)
            raise AssertionError(f"{label}: part {k} differs ({len(x)} vs {len(y)} bytes, first difference at {first})")
    assert mine == want, f"{label}: chunk bytes (framing or zstd levels)"


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_q8_equals_reference(gold, name):
    data, layout, opts = case_file(name)
    groups = _groups(layout, opts.get("part_bytes", 1 << 30))
    assert len(groups) == len(gold[f"{name}/groups"])
    codec = q8.M22(stat_elems=opts.get("stat_elems", q8.STAT_ELEMS))
    for k, idx in enumerate(groups):
        say("case q8", name, "part", k, "tensors", idx)
        mine = codec.compress(data, tensors=idx, header=False, parsed=(layout, None))
        _compare(mine, gold[f"{name}/p{k}"].tobytes(), f"{name} part {k}")


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_q8_decodes_reference_chunks(gold, name):
    data, layout, opts = case_file(name)
    groups = _groups(layout, opts.get("part_bytes", 1 << 30))
    host = np.frombuffer(data, np.uint8)
    for k, idx in enumerate(groups):
        say("case q8 decode", name, "part", k)
        out = q8.M22().decompress(gold[f"{name}/p{k}"].tobytes(), out=np.zeros(len(data), np.uint8))
        for i in idx:
            o, nb = layout["t"][i][:2]
            assert np.array_equal(out[o:o + nb], host[o:o + nb]), f"{name} part {k}: tensor {i}"


def test_sim8_exact_and_neighbours_brute_force():
    say("case sim8 / neighbours")
    g = np.random.Generator(np.random.PCG64(5))
    n, C = 300, 96
    base = g.integers(-127, 128, (40, C))
    Wq = np.clip(base[g.integers(0, 40, n)] + g.integers(-30, 31, (n, C)), -127, 127).astype(np.int8)
    Wq[17] = Wq[3]                          # ties: equal similarities go to the lower row
    Wq[250] = 0
    A = dev.DeviceArray.from_host(Wq)
    S = dev.DeviceArray((n, n), np.int32)
    check(lib().spa_q8_sim8(A.ptr, n, A.ptr, n, C, S.ptr, None))
    ref = Wq.astype(np.int64) @ Wq.astype(np.int64).T
    assert np.array_equal(S.to_host(), ref)
    rb = 77                                 # a partial tile of candidates
    S2 = dev.DeviceArray((n, rb), np.int32)
    check(lib().spa_q8_sim8(A.ptr, n, A.ptr, rb, C, S2.ptr, None))
    assert np.array_equal(S2.to_host(), ref[:, :rb])
    wave = (np.arange(n) * 16) // n
    wstart = np.searchsorted(wave, wave, side="left").astype(np.int32)
    valid = np.ones(n, np.uint8)
    valid[[5, 9, 40]] = 0
    cand = dev.DeviceArray((n, 4), np.int32)
    wstart_d, valid_d = dev.DeviceArray.from_host(wstart), dev.DeviceArray.from_host(valid)   # alive through the call
    check(lib().spa_q8_neighbours(A.ptr, n, C, wstart_d.ptr, valid_d.ptr, cand.ptr, None))
    got = cand.to_host()
    for r in range(n):
        cols = [c for c in range(wstart[r]) if valid[c]]
        order = sorted(cols, key=lambda c: (-ref[r, c], c))[:4]
        want = order + [-1] * (4 - len(order))
        assert list(got[r]) == want, f"row {r}"


def test_q8parts_round_trip_with_rest():
    """a whole file through Q8Parts with its bytes around the tensors (X form: no tokenizer)"""
    say("case q8parts round trip")
    data, layout, _ = case_file("parts")
    host = np.frombuffer(data, np.uint8)

    class _G:                                 # the layout's tensors as a parsed header would list them
        tensors = []
    from seedpack_amd.gguf import Tensor
    names = ["blk.0.attn_v.weight", "token_embd.weight", "blk.0.ffn_gate.weight", "blk.1.attn_v.weight"]
    _G.tensors = [Tensor(nm, (rl, nb // 34 * 32 // rl), q8.Q8_0, o, nb) for nm, (o, nb, rl, _) in zip(names, layout["t"])]
    _G.spans, _G.data_start = {}, 0
    parts = q8.Q8Parts(80000)
    buf = parts.compress(data, g=_G)
    assert parts.parts == 3
    assert np.array_equal(q8.Q8Parts().decompress(buf), host)
