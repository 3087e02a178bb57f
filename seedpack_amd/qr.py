"""Host side of the QR residual coder over the HIP C ABI (the reference's seedpack/qr.py interface).

encode(T, items, seed_dev, imx_dev=None, mv=None) -> bytes and decode(T, buf, items, seed_dev,
imx_dev=None) -> device array keep qr.py:1007-1090's argument meaning and the coded batch format:
pack({"t": zstd(u32 n, u32 used deltas, u16 freq[n][256]), "l": zstd(u32 segment lengths),
"s": stream, "v": model}). The symbol model, the rANS coding, the gather and the decode lookup tables
run as HIP kernels; the table normalisation runs on the host, as in the reference (it is a loop over
a few hundred rows).

items (encode): (file bytes, predicted bytes, seed byte offset, seed type[, weights per row,
imatrix offset]); (decode): the same without the file bytes. Bytes are numpy uint8 arrays or
DeviceArrays; seeds are device arrays (BF16 = type 30, F32 = 0, F16 = 1).
"""
import ctypes
import json
import struct
import threading
import time

import numpy as np

from . import device as dev
from . import zstd
from .framing import pack, unpack  # noqa: F401  (the reference's codecs_gguf.pack/unpack)
from ._lib import check, lib

SELF_TYPES = {2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 20, 23, 42}     # also coded without a seed, and seeds
GRID_TYPES = {16, 17, 18, 19, 21, 22, 29}
QR_TYPES = SELF_TYPES | GRID_TYPES
SEED_TYPES = SELF_TYPES | {0, 1, 30}
COLRMS = 98                                  # no seed: the seed buffer holds the per-column RMS (float32)
EXPLICIT = 99                                # the seed buffer holds float32 (value, uncertainty) per weight
NFIELDS = {2: 1, 6: 1, 8: 1, 20: 1, 42: 1, 3: 2, 7: 2, 10: 34, 11: 17, 14: 17, 12: 18, 13: 18, 23: 9,
           16: 9, 18: 9, 19: 9, 21: 9, 17: 17, 22: 17, 29: 17}
BS = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 20: 18, 23: 136, 42: 18,
      16: 66, 17: 74, 18: 98, 19: 50, 21: 110, 22: 82, 29: 56}
QK = {t: (32 if t in (2, 3, 6, 7, 8, 20) else 64 if t == 42 else 256) for t in QR_TYPES}
NSB_MAX = 20
NTAB2 = NSB_MAX + 64 + 2 + 208
MODEL = 2
PB = 12
BATCH = 384 << 20                                   # bytes per coding batch (qr.py:56)

TM_DT = np.dtype([("blk0", "<i8"), ("seed_off", "<i8"), ("seed_type", "<i4"), ("cols", "<i4"), ("imx_off", "<i8")])
SG_DT = np.dtype([("t", "<i4"), ("nb", "<i4"), ("b0", "<i8")])


# the library's IQ table holding each grid type's lattice (iq_table_index in the C library)
GRID_TABLE = {16: 0, 17: 1, 19: 2, 29: 2, 22: 3, 18: 4, 21: 5}
_GK = {}


def grid_keys(T):
    """numpy uint16 per grid point of grid type T: its coordinate levels (value - 1) / 2, 2 bits each
    (IQ3: 3 bits) -- what the grid model looks distances up by (qr.py:935-948). Built from the
    library's own lattice tables."""
    if T not in _GK:
        g, n = ctypes.c_void_p(), ctypes.c_int()
        check(lib().spa_iq_table_host(GRID_TABLE[T], ctypes.byref(g), ctypes.byref(n), None, None, None, None))
        grid = np.ctypeslib.as_array(ctypes.cast(g, ctypes.POINTER(ctypes.c_uint8)), (n.value,))
        d, bits = (4, 3) if T in (18, 21) else (8, 2)
        lev = (grid.reshape(-1, d).astype(np.int64) - 1) // 2
        _GK[T] = (lev << (bits * np.arange(d))).sum(1).astype(np.uint16)
    return _GK[T]


def seg_blocks(T):
    """blocks per rANS segment: max(16, 16384 // QK) (part of the stream format)"""
    return max(16, 16384 // QK[T])


def layout(T, nblocks):
    """tensors' block counts -> (TM records without the seed fields, SG records, total blocks)"""
    sb = seg_blocks(T)
    tm = np.zeros(len(nblocks), TM_DT)
    starts, b0 = [], 0
    for i, nb in enumerate(nblocks):
        tm[i]["blk0"] = b0
        starts += [(i, min(sb, nb - o), b0 + o) for o in range(0, nb, sb)]
        b0 += nb
    return tm, np.array(starts, SG_DT) if starts else np.zeros(0, SG_DT), b0


def batches(T, sizes):
    """tensor indices split into coding batches of about BATCH bytes (the same split on both sides)"""
    out, cur, n = [], [], 0
    for i, s in enumerate(sizes):
        if cur and n + s > BATCH:
            out.append(cur)
            cur, n = [], 0
        cur.append(i)
        n += s
    if cur:
        out.append(cur)
    return out


def normalize(counts, scale=1 << PB):
    """(rows, 256) counts -> (u16 frequencies of the used rows, used row ids); each row sums to
    `scale`, every seen symbol keeps a frequency >= 1. The rounding error is settled on the largest
    entry, one step at a time, as qr.py:904-923 does."""
    c = np.asarray(counts, np.int64)
    tot = c.sum(1)
    used = np.flatnonzero(tot)
    rows = c[used]
    f = np.where(rows > 0, np.maximum(1, rows * scale // tot[used, None]), 0)
    # one step settles a row whose error is a surplus, or a deficit its largest entry can give up while
    # staying >= 1 (nearly every row); the others take the steps one at a time
    diffs = scale - f.sum(1)
    r = np.arange(len(f))
    j = np.argmax(f, axis=1) if len(f) else np.zeros(0, np.int64)
    one = (diffs > 0) | ((diffs < 0) & (f[r, j] - 1 >= -diffs))
    f[r[one], j[one]] += diffs[one]
    for k in np.flatnonzero(~one & (diffs != 0)):
        fr = f[k]
        diff = scale - int(fr.sum())
        while diff:
            j = int(np.argmax(fr))
            step = diff if diff > 0 else -min(-diff, int(fr[j]) - 1)
            if step == 0:                       # the largest is 1: take from the first entry > 1
                j = int(np.argmax(fr > 1))
                step = -1
            fr[j] += step
            diff -= step
    return f.astype(np.uint16), used.astype(np.int32)


def cum_of(freq):
    cum = np.zeros((freq.shape[0], 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    return cum


def store_tables(freq, used):
    """table chunk: u32 row count, u32 deltas of the used row ids, u16 frequencies (gpu2.py:489-492)"""
    u = np.asarray(used, np.int64)
    du = np.diff(u, prepend=0).astype(np.uint32)
    return zstd.compress(struct.pack("<I", len(u)) + du.tobytes() + np.asarray(freq, np.uint16).tobytes(), 19)


def load_tables(buf):
    raw = zstd.decompress(buf)
    (n,) = struct.unpack_from("<I", raw)
    used = np.cumsum(np.frombuffer(raw, np.uint32, n, 4).astype(np.int64))
    freq = np.frombuffer(raw, np.uint16, n * 256, 4 + 4 * n).reshape(n, 256)
    return freq, used


_WS = threading.local()


def _workspace(name, nbytes):
    """a device buffer of at least nbytes kept for this thread and device between encode_parts calls
    (each call has finished its device work when it returns: the stream is read back). Allocating and
    freeing several hundred MB per batch instead stalled for seconds now and then when much of the
    device memory was in use."""
    cache = getattr(_WS, "bufs", None)
    if cache is None:
        cache = _WS.bufs = {}
    key = (dev.current_device(), name)
    a = cache.get(key)
    if a is None or a.nbytes < nbytes:
        cache.pop(key, None)
        a = None
        a = cache[key] = dev.DeviceArray(max(1, nbytes + nbytes // 4), np.uint8)
    return a.view(0, (max(1, nbytes),), np.uint8)


def _put(name, a, stream=None):
    """a host array copied into the named workspace buffer (typed view)"""
    a = np.ascontiguousarray(a)
    w = _workspace(name, a.nbytes)
    if a.nbytes:
        check(lib().spa_memcpy_h2d(w.ptr, a.ctypes.data, a.nbytes, stream))
    return w.view(0, a.shape, a.dtype) if a.nbytes else w


def _gather(arrs, stream=None, workspace=None):
    """host or device uint8 arrays -> one device array, each copied to its place (into the named
    workspace buffer when given)"""
    if len(arrs) == 1 and isinstance(arrs[0], dev.DeviceArray):
        return arrs[0]
    n = sum(a.nbytes if isinstance(a, dev.DeviceArray) else len(a) for a in arrs)
    out = _workspace(workspace, n) if workspace else dev.DeviceArray(max(n, 1), np.uint8)
    o = 0
    for a in arrs:
        if isinstance(a, dev.DeviceArray):
            check(lib().spa_memcpy_d2d(out.ptr + o, a.ptr, a.nbytes, stream))
            o += a.nbytes
        else:
            a = np.ascontiguousarray(a, np.uint8)
            check(lib().spa_memcpy_h2d(out.ptr + o, a.ctypes.data, a.nbytes, stream))
            o += a.nbytes
    return out


def _nbytes(a):
    return a.nbytes if isinstance(a, dev.DeviceArray) else len(a)


def _descriptors(T, nbs, meta):
    tm, sg, nb = layout(T, nbs)
    tm["seed_off"] = [m[0] for m in meta]
    tm["seed_type"] = [m[1] for m in meta]
    tm["cols"] = [m[2] if len(m) > 2 else 0 for m in meta]
    tm["imx_off"] = [m[3] if len(m) > 3 else -1 for m in meta]
    return tm, sg, nb


def _check_type(T):
    if T not in QR_TYPES:
        raise ValueError(f"type {T} is not a QR type")


_GK_DEV = {}
_GK_LOCK = threading.Lock()


def _gk_ptr(T):
    """device grid keys of grid type T (uploaded once per device, under a lock: coder threads share
    them, and an entry once published is never replaced), or None for the other types"""
    if T not in GRID_TYPES:
        return None
    key = (T, dev.current_device())
    with _GK_LOCK:
        a = _GK_DEV.get(key)
        if a is None:
            a = _GK_DEV[key] = dev.DeviceArray.from_host(grid_keys(T))
    return a.ptr


def encode_parts(T, items, seed_dev, imx_dev=None, mv=None, stream=None):
    """the coded batch before framing: dict(counts, freq, used, lens, stream, mv)"""
    _check_type(T)
    mv = MODEL if mv is None else mv
    bs = BS[T]
    clock = [time.perf_counter()]

    def lap():
        clock.append(time.perf_counter())
    tm, sg, nb = _descriptors(T, [_nbytes(it[0]) // bs for it in items], [it[2:] for it in items])
    F = _gather([it[0] for it in items], stream, "F")
    P = _gather([it[1] for it in items], stream, "P")
    nseg = len(sg)
    # every device buffer of the call is a workspace kept for the thread: no frees, which would wait
    # for the whole device (work other threads queued on other streams included)
    tm_d = _put("tm", tm.view(np.uint8), stream)
    sg_d = _put("sg", sg.view(np.uint8) if nseg else np.zeros(16, np.uint8), stream)
    counts = _workspace("counts", NTAB2 * 256 * 4).view(0, (NTAB2, 256), np.uint32).zero(stream)
    imx = None if imx_dev is None else imx_dev.ptr
    gk = _gk_ptr(T)
    lap()
    work = _workspace("work", lib().spa_qr_work_bytes(T, nseg))
    check(lib().spa_qr_hist(T, F.ptr, P.ptr, seed_dev.ptr, tm_d.ptr, sg_d.ptr, nseg, counts.ptr, gk, imx, mv, work.ptr,
                            stream))
    counts_h = counts.to_host(stream=stream)
    lap()
    freq, used = normalize(counts_h)
    remap = np.full(NTAB2, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    cum = cum_of(freq)
    remap_d, freq_d, cum_d = (_put(n, a, stream) for n, a in (("remap", remap), ("freq", freq), ("cum", cum)))
    cap = seg_blocks(T) * (3 * BS[T] if T in GRID_TYPES else (QK[T] + NSB_MAX) * 2) + 1024
    lap()
    tries = 0
    for _ in range(3):
        tries += 1
        out = _workspace("out", nseg * cap)
        out_len = _workspace("out_len", 4 * max(1, nseg)).view(0, (max(1, nseg),), np.uint32).zero(stream)
        check(lib().spa_qr_encode(T, F.ptr, P.ptr, seed_dev.ptr, tm_d.ptr, sg_d.ptr, nseg, remap_d.ptr, freq_d.ptr,
                                  cum_d.ptr, out.ptr, cap, out_len.ptr, gk, imx, mv, work.ptr, stream))
        lens = out_len.to_host(stream=stream)[:nseg]
        if not (lens == 0xFFFFFFFF).any():
            break
        cap *= 2                                 # an overflowing segment: retry with twice the room
    else:
        raise RuntimeError("QR segment overflow")
    lap()
    offs = np.zeros(nseg + 1, np.uint64)
    offs[1:] = np.cumsum(lens.astype(np.uint64))
    total = int(offs[-1])
    dst = _workspace("dst", max(1, total))
    offs_d = _put("offs", offs, stream)
    check(lib().spa_qr_gather(out.ptr, cap, out_len.ptr, offs_d.ptr, nseg, dst.ptr, stream))
    data = dst.to_host(stream=stream)[:total].copy()
    lap()
    ph = np.diff(clock)
    return {"counts": counts_h, "freq": freq, "used": used, "lens": lens.astype(np.uint32), "stream": data, "mv": mv,
            "seconds": {"setup": ph[0], "hist": ph[1], "tables": ph[2], "encode": ph[3], "gather": ph[4]},
            "tries": tries}


def frame(p):
    """the framed batch of encode_parts' result: zstd-19 tables and lengths, the stream, the model
    version (qr.py:1055-1061). Host work only (zstd releases the interpreter), so callers may run it
    on worker threads while the device codes the next batch, as the reference's pool does
    (repo3.py:946-979)."""
    out = {"t": store_tables(p["freq"], p["used"]), "l": zstd.compress(p["lens"].astype(np.uint32).tobytes(), 19),
           "s": p["stream"].tobytes()}
    if p["mv"] != 1:
        out["v"] = bytes([p["mv"]])
    return pack(out)


def encode(T, items, seed_dev, imx_dev=None, mv=None, stream=None):
    """one coded batch (qr.py:1007-1061) -> bytes"""
    return frame(encode_parts(T, items, seed_dev, imx_dev, mv, stream))


def decode_parts(T, freq, used, lens, stream_bytes, items, seed_dev, imx_dev=None, mv=MODEL, stream=None):
    """the batch's tensors (device uint8, back to back) from its coded parts"""
    _check_type(T)
    bs = BS[T]
    tm, sg, nb = _descriptors(T, [_nbytes(it[0]) // bs for it in items], [it[1:] for it in items])
    nseg = len(sg)
    P = _gather([it[0] for it in items], stream)
    F = dev.DeviceArray(max(1, nb * bs), np.uint8)
    freq = np.ascontiguousarray(freq, np.uint16)
    cum = cum_of(freq)
    remap = np.full(NTAB2, -1, np.int32)
    remap[np.asarray(used, np.int64)] = np.arange(len(used), dtype=np.int32)
    freq_d, cum_d, remap_d = (dev.DeviceArray.from_host(a, stream) for a in (freq, cum, remap))
    lut = dev.DeviceArray((max(1, len(freq)), 1 << PB), np.uint32)
    check(lib().spa_rans_build_lut32(cum_d.ptr, len(freq), lut.ptr, stream))
    lens = np.asarray(lens, np.uint64)
    s = np.frombuffer(bytes(stream_bytes), np.uint8)
    if len(lens) != nseg or int(lens.sum()) > len(s):
        raise ValueError(f"QR batch of type {T}: {len(lens)} segment lengths summing to {int(lens.sum())} bytes for "
                         f"{nseg} segments and a {len(s)}-byte stream")
    offs = np.zeros(max(1, nseg), np.uint64)
    offs[1:nseg] = np.cumsum(lens)[:-1]
    s_d = dev.DeviceArray.from_host(s if len(s) else np.zeros(1, np.uint8), stream)
    tm_d = dev.DeviceArray.from_host(tm.view(np.uint8), stream)
    sg_d = dev.DeviceArray.from_host(sg.view(np.uint8) if nseg else np.zeros(16, np.uint8), stream)
    offs_d = dev.DeviceArray.from_host(offs, stream)
    imx = None if imx_dev is None else imx_dev.ptr
    check(lib().spa_qr_decode(T, s_d.ptr, len(s), offs_d.ptr, P.ptr, seed_dev.ptr, tm_d.ptr, sg_d.ptr, nseg, remap_d.ptr,
                              freq_d.ptr, cum_d.ptr, lut.ptr, F.ptr, _gk_ptr(T), imx, mv, stream))
    dev.synchronize(stream)          # the batch's descriptors and tables go out of scope here
    return F


def decode(T, buf, items, seed_dev, imx_dev=None, stream=None):
    """one coded batch -> device uint8 array of its tensors back to back (qr.py:1064-1090)"""
    ch = unpack(buf)
    mv = bytes(ch["v"])[0] if "v" in ch else 1      # batches without it predate model 2
    freq, used = load_tables(ch["t"])
    lens = np.frombuffer(zstd.decompress(ch["l"]), np.uint32)
    return decode_parts(T, freq, used, lens, ch["s"], items, seed_dev, imx_dev, mv, stream)


# ------------------------------------------------------------------ seeds other than a BF16 base

def intervals(T, blocks, nw, stream=None):
    """device uint8 blocks of non-grid type T -> (lo, hi) float32 DeviceArrays: the interval of values
    each weight's code stands for (qr.py:1093-1098)"""
    blocks = blocks if isinstance(blocks, dev.DeviceArray) else dev.DeviceArray.from_host(np.ascontiguousarray(blocks, np.uint8), stream)
    lo, hi = dev.DeviceArray(nw, np.float32), dev.DeviceArray(nw, np.float32)
    check(lib().spa_qr_intervals(T, blocks.ptr, nw, lo.ptr, hi.ptr, stream))
    return lo, hi


def grid_half_steps(T, blocks, nw, stream=None):
    """half the step between grid levels around each weight of grid-type blocks (float32 DeviceArray)"""
    h = dev.DeviceArray(nw, np.float32)
    check(lib().spa_qr_grid_h(T, blocks.ptr, nw, h.ptr, stream))
    return h


def explicit_seed(T, blocks, x, stream=None):
    """an EXPLICIT seed (99) from a grid-type tensor: float32 (x, h) per weight, x its dequantized values,
    h half the step between its grid's levels (qr.py:1100-1106) -> DeviceArray of 2 nw float32"""
    nw = x.size
    h = grid_half_steps(T, blocks, nw, stream)
    xh = np.stack([x.to_host(stream=stream).reshape(-1), h.to_host(stream=stream)], axis=1).reshape(-1)
    return dev.DeviceArray.from_host(np.ascontiguousarray(xh, np.float32), stream)


def weight_equal(T, F, P, nw, stream=None):
    """device uint8 per weight: code and sub-block integer scale equal in blocks F and P (qr.py:1109-1113)"""
    out = dev.DeviceArray(nw, np.uint8)
    check(lib().spa_qr_weight_equal(T, F.ptr, P.ptr, nw, out.ptr, stream))
    return out


def self_side(T, blocks, cols, gq=None, stream=None):
    """no-seed coding of one tensor (device uint8 blocks, `cols` weights per row) -> (column RMS as fp16,
    template blocks, rows): the RMS of each column of the dequantized tensor (detmath's in-order sums)
    and one row of blocks holding the rounded mean of every block field (qr.py:1116-1136)"""
    from . import detmath
    from .gpuquant import GPUQuant
    gq = gq or GPUQuant(stream=stream)
    x = gq.dequantize(T, blocks, cols)
    rows = x.size // cols
    xs = x.view(0, (rows, cols), np.float32)
    rms = np.sqrt((detmath.cols(xs, True, stream=stream).to_host(stream=stream) / rows).astype(np.float32)).astype(np.float16)
    del x, xs
    nb_row = cols // QK[T]
    nblk = rows * nb_row
    nf = NFIELDS[T]
    fl = dev.DeviceArray(max(1, nblk * nf), np.int32)
    check(lib().spa_qr_block_fields(T, blocks.ptr, nblk, fl.ptr, stream))
    f = fl.to_host(stream=stream)[:nblk * nf].reshape(rows, nb_row, nf)
    # (integer fields: the float64 sum over rows is exact, the mean one rounding)
    v = np.rint(f.astype(np.float64).mean(0)).astype(np.int32)
    vd = dev.DeviceArray.from_host(np.ascontiguousarray(v), stream)
    tpl = dev.DeviceArray(nb_row * BS[T], np.uint8)
    check(lib().spa_qr_blocks_from_fields(T, vd.ptr, nb_row, tpl.ptr, stream))
    return rms, tpl.to_host(stream=stream), rows


def self_encode(T, tensors, stream=None):
    """tensors: [(host or device uint8 blocks, cols)] of non-grid type T, coded without a seed: each
    batch QR-coded against template blocks with the column RMS as the seed (qr.py:1147-1163) -> bytes"""
    from .gpuquant import GPUQuant
    gq = GPUQuant(stream=stream)
    parts, side = {}, []
    for bi in batches(T, [_nbytes(b) for b, _ in tensors]):
        items, seeds, rms_l, tpl_l, o = [], [], [], [], 0
        for i in bi:
            b, cols = tensors[i]
            bd = b if isinstance(b, dev.DeviceArray) else dev.DeviceArray.from_host(np.ascontiguousarray(b, np.uint8).reshape(-1), stream)
            rms, tpl, rows = self_side(T, bd, cols, gq, stream)
            rms_l.append(rms)
            tpl_l.append(tpl)
            seeds.append(rms.astype(np.float32))
            items.append((bd, dev.DeviceArray.from_host(np.tile(tpl, rows), stream), o, COLRMS, cols))
            o += cols * 4
        seed = dev.DeviceArray.from_host(np.concatenate(seeds).view(np.uint8), stream)
        parts[str(len(side))] = encode(T, items, seed, stream=stream)
        side.append([[_nbytes(tensors[i][0]), tensors[i][1]] for i in bi])
        parts[f"r{len(side) - 1}"] = zstd.zstd_c(b"".join(r.tobytes() for r in rms_l), 19)
        parts[f"t{len(side) - 1}"] = zstd.zstd_c(b"".join(t.tobytes() for t in tpl_l), 19)
    return pack({"meta": zstd.zstd_c(json.dumps(side).encode()), **parts})


def self_decode(T, buf, stream=None):
    """-> list of device uint8 arrays, in self_encode's order (qr.py:1166-1186)"""
    ch = unpack(memoryview(buf))
    out = []
    for k, sizes in enumerate(json.loads(zstd.decompress(ch["meta"]))):
        rms_all = np.frombuffer(zstd.decompress(ch[f"r{k}"]), np.float16)
        tpl_all = np.frombuffer(zstd.decompress(ch[f"t{k}"]), np.uint8)
        items, seeds, ro, to, o = [], [], 0, 0, 0
        for nbytes_, cols in sizes:
            nb_row = cols // QK[T]
            rows = nbytes_ // BS[T] // nb_row
            rms = rms_all[ro:ro + cols]
            ro += cols
            tpl = tpl_all[to:to + nb_row * BS[T]]
            to += nb_row * BS[T]
            seeds.append(rms.astype(np.float32))
            items.append((dev.DeviceArray.from_host(np.tile(tpl, rows), stream), o, COLRMS, cols))
            o += cols * 4
        seed = dev.DeviceArray.from_host(np.concatenate(seeds).view(np.uint8), stream)
        F = decode(T, ch[str(k)], items, seed, stream=stream)
        p = 0
        for nbytes_, _ in sizes:
            out.append(F.view(p, (nbytes_,), np.uint8))
            p += nbytes_
    return out
