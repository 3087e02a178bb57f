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
    assert bytes(parts["stream"]) == vectors[f"{name}/stream"].tobytes()
    out = codec.decompress(parts)
    host = np.frombuffer(data, np.uint8)
    for off, nb, _, _ in layout["t"]:
        assert out[off:off + nb].tobytes() == host[off:off + nb].tobytes()


@pytest.mark.parametrize("shape", [(256, 1000), (200, 999), (130, 4096), (300, 131072)])
def test_hip_r2_row_statistics_bit_exact(shape):
    """the float64 log2 row RMS (sums, division, sqrt, detmath log2) equals the oracle's bit for bit,
    and so do rfi, cfi and scl: rows read as vectors with a partial last tile (1000), rows not 16-byte
    aligned (999), rows past the last full workgroup (130), and columns summed over three chunks of
    rows (131072: 128-row chunks)"""
    say("case r2 stats", shape)
    g = np.random.Generator(np.random.PCG64(11))
    x = g.normal(0, 1, shape) * np.exp(g.uniform(-40, 10, (shape[0], 1)))
    x[3] = 0.0
    x[4, :7] = 1e-40
    u = synth.bf16_bits(x.astype(np.float32))
    d = dev.DeviceArray.from_host(u.reshape(-1))
    nr, rl = u.shape
    rfi, cfi, scl = dev.DeviceArray(nr, np.int16), dev.DeviceArray(rl, np.int16), dev.DeviceArray(rl, np.int8)
    wb = lib().spa_r2_stats_work_bytes(nr, rl)
    work, rf, h = dev.DeviceArray(wb, np.uint8), dev.DeviceArray(nr, np.float64), dev.DeviceArray(nr, np.uint64)
    check(lib().spa_r2_stats(d.ptr, nr, rl, rfi.ptr, cfi.ptr, scl.ptr, h.ptr, work.ptr, wb, rf.ptr, None))
    want_rf = or2.dm_log2(np.sqrt(or2.rows_sum(or2.bf16_f32(u), True) / rl) + 1e-30)
    assert rf.to_host().tobytes() == want_rf.tobytes()
    assert np.array_equal(h.to_host(), or2.row_hash(u, rl))
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


@pytest.mark.parametrize("pad", [None, 0, 448, -5, 9999])
def test_hip_r2_hist_any_window(pad):
    """the histogram's LDS window of exponent contexts (TB.pad) changes no count: a tensor whose rows
    span ~12 octaves (contexts far outside any 64-wide window) counted with the window at the median,
    at either end and clamped, against the oracle's symbols"""
    say("case r2 hist pad", pad)
    g = np.random.Generator(np.random.PCG64(31))
    x = g.normal(0, 1, (700, 1536)) * np.exp2(g.uniform(-14, -2, (700, 1)))
    w = synth.bf16_bits(x.astype(np.float32))
    layout = r2.layout_of([("blk.0.attn_q.weight", 0, w.nbytes, 1536)], w.nbytes)
    rfi, cfi, scl = or2.stats(w, 1536)
    tb, sg = r2.plan(layout, [0], {0: 700}, {}, rfi, cfi)
    if pad is not None:
        tb["pad"] = pad
    d = dev.DeviceArray.from_host(w.reshape(-1))
    side = [dev.DeviceArray.from_host(np.ascontiguousarray(v)) for v in (rfi, cfi, scl)]
    tb_d, sg_d = dev.DeviceArray.from_host(tb.view(np.uint8)), dev.DeviceArray.from_host(sg.view(np.uint8))
    rm = dev.DeviceArray.from_host(np.zeros(1, np.int32))
    counts = dev.DeviceArray((r2.TPT, 256), np.uint32).zero()
    check(lib().spa_r2_hist(d.ptr, tb_d.ptr, sg_d.ptr, len(sg), side[0].ptr, side[1].ptr, side[2].ptr, rm.ptr, counts.ptr, None))
    got = counts.to_host()
    want = np.zeros_like(got)
    t, s = or2.symbols(w, 1536, None, rfi, cfi, scl, 0)
    np.add.at(want, (t, s), 1)
    pe = np.flatnonzero(want[:512].sum(1))
    assert pe.max() - pe.min() > 64
    assert np.array_equal(got, want)


def test_hip_r2_device_resident_matches_host():
    """compress of the file already in HBM (duplicate rows fetched from the device) gives the same
    parts as compress of host bytes, and decompress(device=True) leaves the tensors in HBM"""
    say("case r2 device-resident roles")
    data, layout, gb = case_file("embd_dups")
    codec = r2.BF16v2(group_bytes=gb)
    want = codec.compress(data, layout)
    d = dev.DeviceArray.from_host(np.frombuffer(data, np.uint8))
    got = codec.compress(d, layout)
    for k in ("meta", "side", "tables", "lens", "stream"):
        assert bytes(got[k]) == bytes(want[k]), k
    back = codec.decompress(got, device=True).to_host()
    host = np.frombuffer(data, np.uint8)
    for off, nb, _, _ in layout["t"]:
        assert back[off:off + nb].tobytes() == host[off:off + nb].tobytes()


def test_hip_synth_normal_bf16():
    """the device generator of benchmark inputs: deterministic per seed, N(0, std)-shaped"""
    say("case synth normal bf16")
    n = 1 << 20
    a, b = dev.DeviceArray(n, np.uint16), dev.DeviceArray(n, np.uint16)
    check(lib().spa_synth_normal_bf16(a.ptr, n, 7, 0.02, None))
    check(lib().spa_synth_normal_bf16(b.ptr, n, 7, 0.02, None))
    x, y = a.to_host(), b.to_host()
    assert np.array_equal(x, y)
    f = synth.bf16_to_f32(x)
    assert abs(f.mean()) < 1e-4 and abs(f.std() - 0.02) < 2e-4
    assert len(np.unique(x)) > 1000


def test_hip_r2_dec_tables_give_lut_symbols():
    """the compact decode tables (symbol at every 128th slot, cumulative frequencies) name the same
    symbol for every one of the 2^15 slots as the full lookup table, on tables with zero-frequency
    symbols, one symbol holding every slot, and long runs of frequency-1 symbols"""
    say("case r2 decode tables")
    g = np.random.Generator(np.random.PCG64(41))
    freq = np.zeros((6, 256), np.int64)
    freq[0, 7] = 1 << 15
    freq[1] = 128
    freq[2, :200] = 1; freq[2, 255] = (1 << 15) - 200
    freq[3, ::3] = g.integers(1, 400, 86); freq[3, 0] += (1 << 15) - freq[3].sum()
    p = g.dirichlet(np.full(256, 0.05)); f = np.floor(p * ((1 << 15) - 256)).astype(np.int64) + 1
    f[np.argmax(f)] += (1 << 15) - f.sum(); freq[4] = f
    freq[5, 100:228] = 256
    assert (freq.sum(1) == 1 << 15).all()
    cum = r2.cum_of(freq.astype(np.uint16))
    cum_d = dev.DeviceArray.from_host(cum)
    nb = lib().spa_r2_dec_table_bytes()
    remap = np.array([5, 4, 3, 2, 1, 0, -1], np.int32)          # contexts -> tables; the last has none
    remap_d = dev.DeviceArray.from_host(remap)
    dt = dev.DeviceArray((7, nb), np.uint8)
    lut = dev.DeviceArray((6, 1 << 15), np.uint8)
    check(lib().spa_r2_build_dec_tables(cum_d.ptr, remap_d.ptr, 7, dt.ptr, None))
    check(lib().spa_rans_build_lut_pb(cum_d.ptr, 6, 15, lut.ptr, None))
    dth, luth = dt.to_host(), lut.to_host()
    slots = np.arange(1 << 15)

    def decode_all(tab):
        """every slot's (symbol, cum, freq) from the compact table: a two-symbol bucket's s0 or s1 by
        the bound c1; in a bucket of more symbols its first symbol, or the last of its other symbols
        whose cum <= slot"""
        eu = tab[:2048].view(np.uint64)[slots >> 7]
        multi = (eu >> np.uint64(63)).astype(bool)
        e = (eu & np.uint64((1 << 63) - 1)).astype(np.int64)
        # buckets of at most two symbols
        s0, s1, b0, b1, b2 = e & 255, (e >> 8) & 255, (e >> 16) & 0x7FFF, (e >> 31) & 0xFFFF, (e >> 47) & 0xFFFF
        up = slots >= b1
        two = (np.where(up, s1, s0), np.where(up, b1, b0), np.where(up, b2 - b1, b1 - b0))
        # the others
        ps = tab[2048:3072].view(np.uint32).astype(np.int64)
        first, span, c0, f = e & 255, (e >> 8) & 255, (e >> 16) & 0xFFFF, (e >> 32) & 0xFFFF
        sym = first.copy()
        for k in range(1, 256):                   # every candidate of the bucket, in order
            cand = first + k
            take = (k <= span) & ((ps[np.minimum(cand, 255)] & 0xFFFF) <= slots)
            sym = np.where(take, cand, sym)
        u = ps[np.minimum(sym, 255)]             # (a two-symbol bucket's fields read this way: unused)
        moved = sym != first
        more = (sym, np.where(moved, u & 0xFFFF, c0), np.where(moved, u >> 16, f))
        return tuple(np.where(multi, m, t) for m, t in zip(more, two))

    sym, c0, f = decode_all(dth[6])                       # no table: one symbol with every slot
    assert not sym.any() and not c0.any() and (f == 1 << 15).all()
    for t in range(6):
        sym, c0, f = decode_all(dth[5 - t])
        assert np.array_equal(sym, luth[t].astype(np.int64)), t
        assert np.array_equal(c0, cum[t][sym]) and np.array_equal(f, freq[t][sym])
        assert np.array_equal(np.repeat(np.arange(256), freq[t]), luth[t])


def test_hip_r2_packed_chunk_and_random_access():
    """compress_parts' packed chunk decodes to the whole file (the rest part included); R2Tensors
    decodes chosen tensors alone (from reads of their stream ranges) and writes the file in order
    through windows of tensors"""
    say("case r2 packed + R2Tensors roles")
    data, layout, gb = case_file("roles")
    codec = r2.BF16v2(group_bytes=gb)
    chunk = b"".join(bytes(p) for p in codec.compress_parts(data, layout))
    out = codec.decompress(chunk)
    assert out.tobytes() == data
    parts = r2.unpack(memoryview(chunk))
    stream = np.frombuffer(parts["stream"], np.uint8)
    reads = []

    def read(off, n, dst):
        reads.append((off, n))
        dst[:] = stream[off:off + n]

    rt = r2.R2Tensors(lambda name: bytes(parts[name]), read)
    host = np.frombuffer(data, np.uint8)
    for idxs in ([2], [0, 3], [1, 2, 3]):
        d, outs = rt.decode(idxs)
        h = d.to_host()
        for i, o in zip(idxs, outs):
            off, nb, _, _ = layout["t"][i]
            assert h[o:o + nb].tobytes() == host[off:off + nb].tobytes()
    assert sum(n for _, n in reads[:1]) == rt.coded_bytes(2)
    pieces = []
    rt.write_to(lambda b: pieces.append(bytes(b)), window=40 << 10)
    assert b"".join(pieces) == data


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_hip_r2_grouped_equals_one_pass(name):
    """a file in host memory coded in groups of tensors (the path of a base bigger than HBM: a third
    of the coded bytes on the device at a time, each group read twice) gives the parts of the
    one-pass coding, and they decode back"""
    say("case r2 grouped", name)
    data, layout, gb = case_file(name)
    whole = r2.BF16v2(group_bytes=gb).compress(data, layout)
    span = max(off + nb for off, nb, _, _ in layout["t"]) - layout["t"][0][0]
    codec = r2.BF16v2(group_bytes=gb, stream_bytes=max(1, span // 3))
    parts = codec.compress(data, layout)
    for k in ("meta", "side", "tables", "lens"):
        assert bytes(parts[k]) == bytes(whole[k]), k
    got = b"".join(bytes(p) for p in parts["stream"]) if isinstance(parts["stream"], list) else bytes(parts["stream"])
    want = b"".join(bytes(p) for p in whole["stream"]) if isinstance(whole["stream"], list) else bytes(whole["stream"])
    assert got == want
    out = codec.decompress(whole)
    host = np.frombuffer(data, np.uint8)
    for off, nb, _, _ in layout["t"]:
        assert out[off:off + nb].tobytes() == host[off:off + nb].tobytes()
