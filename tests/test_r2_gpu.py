"""HIP R2 BF16 base codec vs the reference's own R2 code (golden vectors), the oracle, and round trips
(MI355X)."""
import ctypes
import os
import sys

import numpy as np
import pytest

from oracle import r2 as or2
from seedpack_amd import device as dev
from seedpack_amd import r2, synth
from seedpack_amd._lib import check, lib
from tests.golden.r2_cases import CASES, case_file

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def vectors():
    return np.load(os.path.join(ROOT, "tests", "golden", "r2_vectors.npz"))


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_hip_r2_matches_reference(vectors, name):
    say("case r2", name)
    data, layout, gb = case_file(name)
    codec = r2.BF16v2(group_bytes=gb)
    parts = codec.compress(data, layout)
    a = parts["arrays"]
    for k in ("rfi", "cfi", "scl", "nrows_c", "dups", "rowmap", "counts", "freq", "used", "lens"):
        assert np.array_equal(a[k], vectors[f"{name}/{k}"]), k
    assert parts["stream"] == vectors[f"{name}/stream"].tobytes()
    out = codec.decompress(parts)
    host = np.frombuffer(data, np.uint8)
    for off, nb, _, _ in layout["t"]:
        assert out[off:off + nb].tobytes() == host[off:off + nb].tobytes()


def test_hip_r2_row_statistics_bit_exact():
    """the float64 log2 row RMS (sums, division, sqrt, detmath log2) equals the oracle's bit for bit"""
    g = np.random.Generator(np.random.PCG64(11))
    x = g.normal(0, 1, (256, 1000)) * np.exp(g.uniform(-40, 10, (256, 1)))
    x[3] = 0.0
    x[4, :7] = 1e-40
    u = synth.bf16_bits(x.astype(np.float32))
    d = dev.DeviceArray.from_host(u.reshape(-1))
    nr, rl = u.shape
    rfi, cfi, scl = dev.DeviceArray(nr, np.int16), dev.DeviceArray(rl, np.int16), dev.DeviceArray(rl, np.int8)
    work, rf = dev.DeviceArray(nr, np.float32), dev.DeviceArray(nr, np.float64)
    check(lib().spa_r2_stats(d.ptr, nr, rl, rfi.ptr, cfi.ptr, scl.ptr, None, work.ptr, rf.ptr, None))
    want_rf = or2.dm_log2(np.sqrt(or2.rows_sum(or2.bf16_f32(u), True) / rl) + 1e-30)
    assert rf.to_host().tobytes() == want_rf.tobytes()
    want = or2.stats(u, rl)
    assert np.array_equal(rfi.to_host(), want[0]) and np.array_equal(cfi.to_host(), want[1])
    assert np.array_equal(scl.to_host(), want[2])


def test_hip_r2_larger_file_round_trip_and_tables():
    """an 8M-weight file (two roles, duplicate rows): side information and counts equal the oracle's,
    the tables its normalisation, and the stream decodes back"""
    g = np.random.Generator(np.random.PCG64(21))
    w1 = synth.normal_bf16(g, (1024, 4096), 0.02)
    w2 = synth.student_t_bf16(g, (2048, 2048))
    w2[100:140] = w2[7]
    data = b"\x01" * 64 + w1.tobytes() + b"\x02" * 32 + w2.tobytes()
    layout = r2.layout_of([("blk.0.ffn_up.weight", 64, w1.nbytes, 4096),
                           ("blk.0.ffn_down.weight", 96 + w1.nbytes, w2.nbytes, 2048)], len(data))
    codec = r2.BF16v2(group_bytes=16 << 20)
    parts = codec.compress(data, layout)
    a = parts["arrays"]
    o1, o2 = or2.stats(w1, 4096), or2.stats(w2, 2048)
    assert np.array_equal(a["rfi"], np.concatenate([o1[0], o2[0]]))
    assert np.array_equal(a["cfi"], np.concatenate([o1[1], o2[1]]))
    assert np.array_equal(a["scl"], np.concatenate([o1[2], o2[2]]))
    keep, pairs = or2.dups(w2, 2048)
    assert a["dups"].tolist() == [[1, r, s] for r, s in pairs]
    counts = np.zeros_like(a["counts"])
    for i, (w, rl, k_, o) in enumerate([(w1, 4096, None, o1), (w2, 2048, keep, o2)]):
        t, s = or2.symbols(w, rl, k_, o[0], o[1], o[2], layout["role"][i] * or2.TPT)
        np.add.at(counts, (t, s), 1)
    assert np.array_equal(a["counts"], counts)
    f, u = or2.normalize(counts)
    assert np.array_equal(a["freq"], f) and np.array_equal(a["used"], u)
    out = codec.decompress(parts)
    host = np.frombuffer(data, np.uint8)
    for off, nb, _, _ in layout["t"]:
        assert out[off:off + nb].tobytes() == host[off:off + nb].tobytes()
