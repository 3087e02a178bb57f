"""Host side of the R2 BF16 base codec over the HIP C ABI (the reference's seedpack/bf16v2.py BF16v2).

compress(data, layout) -> parts and decompress(parts) -> the tensors' bytes keep BF16v2's
algorithm and stream format (bf16v2.py:185-486): side information per tensor (rfi, cfi, scl),
exact duplicate rows coded once, per-role frequency tables (656 per role: 512 exponent, 128
mantissa, 16 sign contexts) normalised to 2^15, and rANS segments of 16384 weights. The statistics,
fingerprints, histogram, symbol lookups, coding, gather and decoding run as HIP kernels; the
duplicate-row check, the table normalisation (gpu2.normalize_gpu, a loop over a few hundred rows)
and the framing run on the host.

`layout` is BF16v2._layout's dict (bf16v2.py:182-188): {"size": file bytes, "t": [[offset, bytes,
row length, "bf16"], ...] (2-D BF16 tensors by offset), "role": role index per tensor, "nroles"}.
R2Tensors (bf16v2.py:488-617) decodes chosen tensors alone. The file's other bytes travel in the
"rest" part, coded on the host by seedpack_amd.header.
"""
import ctypes
import json
import re
import struct
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import device as dev
from . import zstd
from ._lib import check, lib
from .framing import pack_parts, unpack
from .header import fill_rest, header_d, header_x, rest_of

PB = 15
K = 8
SEG = 16384
NE, NM, NS = 512, 128, 16
TPT = NE + NM + NS                 # tables per role
TB_DT = np.dtype([("doff", "<i8"), ("rowlen", "<i4"), ("rowbase", "<i4"), ("colbase", "<i4"), ("tab", "<i4"),
                  ("rmap", "<i4"), ("pad", "<i4")])
SG_DT = np.dtype([("t", "<i4"), ("n", "<i4"), ("i0", "<i8")])
CAP = SEG * 2 + 1024               # bytes per segment slot (bf16v2.py:389)


def role(name):
    """a tensor's role: its name without the block number (bf16v2.py:166-167)"""
    return re.sub(r"blk\.\d+\.", "", name)


def layout_of(tensors, size):
    """R2 layout from [(name, offset, bytes, row length)] of a file's 2-D BF16 tensors (bf16v2.py:182-188)"""
    ts = sorted(tensors, key=lambda t: t[1])
    roles = []
    for t in ts:
        if role(t[0]) not in roles:
            roles.append(role(t[0]))
    return {"size": size, "t": [[t[1], t[2], t[3], "bf16"] for t in ts],
            "role": [roles.index(role(t[0])) for t in ts], "nroles": len(roles)}


def bases(layout):
    """per tensor its first row and first column in the file-wide side information arrays, and the
    totals: (row bases, column bases, rows, columns) -- rows and columns of the tensors in order"""
    t = layout["t"]
    rl = np.array([x[2] for x in t], np.int64)
    rows = np.array([x[1] for x in t], np.int64) // 2 // np.maximum(rl, 1)
    rb = np.concatenate([[0], np.cumsum(rows)]).astype(np.int64)
    cb = np.concatenate([[0], np.cumsum(rl)]).astype(np.int64)
    return rb[:-1].tolist(), cb[:-1].tolist(), int(rb[-1]), int(cb[-1])


HEW = 64                           # exponent contexts the histogram kernel counts in LDS


def plan(layout, grp, nrows_c, rmap_off, rfi=None, cfi=None):
    """(TB, SG) descriptors of the tensors grp: device offsets relative to the first one, and the
    segments -- each tensor's coded rows cut into SEG-weight runs (the last one shorter), tensors in
    order (the stream format, bf16v2.py:208-220). With the side information given, TB.pad holds the
    base of the histogram kernel's LDS window of exponent contexts, centred on the tensor's median
    context (the counts do not depend on it)."""
    rb, cb, _, _ = bases(layout)
    tb = np.zeros(len(grp), TB_DT)
    a = layout["t"][grp[0]][0]
    sgs = []
    for k, i in enumerate(grp):
        off, nb, rl, _ = layout["t"][i]
        pe0 = 0
        if rfi is not None:
            mid = int(np.median(rfi[rb[i]:rb[i] + nb // 2 // rl])) + int(np.median(cfi[cb[i]:cb[i] + rl])) + 256
            pe0 = min(max(mid - HEW // 2, 0), NE - HEW)
        tb[k] = (off - a, rl, rb[i], cb[i], layout["role"][i] * TPT, rmap_off.get(i, -1), pe0)
        n = nrows_c[i] * rl
        sg = np.zeros(-(-n // SEG), SG_DT)
        sg["t"] = k
        sg["i0"] = np.arange(0, n, SEG)
        sg["n"] = np.minimum(SEG, n - sg["i0"])
        sgs.append(sg)
    return tb, (np.concatenate(sgs) if sgs else np.zeros(0, SG_DT))


def normalize(counts, scale=1 << PB):
    """uint16 frequencies of the used rows and the used row ids (gpu2.normalize_gpu, gpu2.py:460-480):
    rounded proportional frequencies, then up to 64 passes moving a row's surplus onto its largest
    entry and taking one unit from each of its |deficit| largest entries above 1 (stable ranks)"""
    counts = np.asarray(counts)
    tot = counts.sum(1, dtype=np.int64)
    used = np.flatnonzero(tot)
    c = counts[used].astype(np.int64)
    t = tot[used][:, None]
    f = np.where(c > 0, np.maximum(1, (c * scale + t // 2) // t), 0)
    rows = np.arange(len(used))
    for _ in range(64):
        diff = scale - f.sum(1)
        if not (diff != 0).any():
            break
        am = np.argmax(f, 1)
        f[rows, am] += np.maximum(diff, 0)
        need = np.maximum(-diff, 0)
        rank = np.argsort(np.argsort(-f, axis=1, kind="stable"), axis=1, kind="stable")
        f = f - ((rank < need[:, None]) & (f > 1)).astype(np.int64)
    if not ((f.sum(1) == scale).all() and ((c > 0) <= (f > 0)).all()):
        raise RuntimeError("R2: table normalisation did not converge")
    return f.astype(np.uint16), used.astype(np.int32)


def cum_of(freq):
    cum = np.zeros((freq.shape[0], 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    return cum


def store_tables(freq, used):
    """zstd-19 of (u32 n, u32 used deltas, u16 freq[n][256]) (gpu2.py:489-492)"""
    u = np.asarray(used, np.int64)
    du = np.diff(u, prepend=0).astype(np.uint32)
    return zstd.zstd_c(struct.pack("<I", len(u)) + du.tobytes() + np.asarray(freq, np.uint16).tobytes(), 19)


def load_tables(buf):
    raw = zstd.decompress(bytes(buf))
    (n,) = struct.unpack_from("<I", raw)
    used = np.cumsum(np.frombuffer(raw, np.uint32, n, 4).astype(np.int64))
    freq = np.frombuffer(raw, np.uint16, n * 256, 4 + 4 * n).reshape(n, 256)
    return freq, used


def _dups(hashes, rows, rl):
    """duplicate rows of a tensor: every row equal to a row with a lower index is coded once and
    copied from the lowest such row (bf16v2.py:246-271). Rows whose 64-bit fingerprints collide are
    compared byte for byte (`rows(ids)` -> those rows' BF16 bits). -> (the rows kept, sorted, or
    None when there is no duplicate; sorted [(duplicate row, source row)])"""
    _, inv, cnt = np.unique(hashes, return_inverse=True, return_counts=True)
    cand = np.flatnonzero(cnt[inv] > 1)            # rows that share a fingerprint with another
    if len(cand) == 0:
        return None, []
    content = dict(zip(cand.tolist(), (np.asarray(r).tobytes() for r in rows(cand))))
    first, pairs = {}, []
    for r in cand.tolist():                        # increasing row index
        key = (int(inv[r]), content[r])
        src = first.setdefault(key, r)
        if src != r:
            pairs.append((r, src))
    if not pairs:
        return None, []
    isdup = np.zeros(len(hashes), bool)
    isdup[[r for r, _ in pairs]] = True
    return np.flatnonzero(~isdup).astype(np.int32), sorted(pairs)


def _p(a):
    return None if a is None else a.ptr


class _Timer:
    """HIP events around the device phases of one call (kernel time with inputs resident)"""

    def __init__(self, on, stream):
        self.on, self.stream, self.marks = on, stream, []
        self.host, self.t = {}, time.perf_counter()

    def lap(self, name):
        """host wall time since the previous lap, added to `name`"""
        now = time.perf_counter()
        self.host[name] = self.host.get(name, 0.0) + (now - self.t)
        self.t = now

    def mark(self, name):
        if self.on:
            e = dev.Event()
            e.record(self.stream)
            self.marks.append((name, e))

    def result(self):
        """device ms per phase (HIP events), and the host wall seconds per lap under "host_s" """
        out = {}
        for (name, e0), (_, e1) in zip(self.marks, self.marks[1:]):
            if name:
                out[name] = out.get(name, 0.0) + e0.elapsed_ms(e1)
        if self.on:
            out["host_s"] = {k: round(v, 4) for k, v in self.host.items()}
        return out


class BF16v2:
    """R2 codec core on the MI355X (bf16v2.py:170-617).

    The reference works through the file in groups of `group_bytes` (bf16v2.py:178); the groups do
    not enter the format (the tables are per role over the whole file, the segments never cross a
    tensor and the stream is the segments in tensor order), so here the whole coded region is
    resident in HBM at once and each kernel runs over every segment of the file in one launch
    (encode in batches of `enc_batch` segments, for its 12-byte-per-weight symbol workspace).
    `group_bytes` is kept for the reference's interface. A file in host memory whose coded region is
    larger than `stream_bytes` (a base bigger than HBM can hold beside its derived files) is coded
    in groups of tensors of about that size instead, read twice (compress_grouped): the same parts."""

    def __init__(self, group_bytes=400 << 20, dedup=True, stream=None, enc_batch=262144, timing=False,
                 stream_bytes=None):
        self.group_bytes, self.dedup, self.stream = group_bytes, dedup, stream
        self.enc_batch, self.timing, self.last_timing = enc_batch, timing, {}
        self.stream_bytes = stream_bytes

    def stats(self, w_dev, rl, with_hash=True):
        """(rfi, cfi, scl, row hashes or None) of one tensor's BF16 bits on the device, as numpy"""
        nr = w_dev.nbytes // 2 // rl
        rfi, cfi, scl = dev.DeviceArray(nr, np.int16), dev.DeviceArray(rl, np.int16), dev.DeviceArray(rl, np.int8)
        h = dev.DeviceArray(nr, np.uint64) if with_hash else None
        wb = lib().spa_r2_stats_work_bytes(nr, rl)
        work = dev.DeviceArray(wb, np.uint8)
        check(lib().spa_r2_stats(w_dev.ptr, nr, rl, rfi.ptr, cfi.ptr, scl.ptr, _p(h), work.ptr, wb, None, self.stream))
        s = self.stream
        return (rfi.to_host(stream=s), cfi.to_host(stream=s), scl.to_host(stream=s),
                h.to_host(stream=s) if h is not None else None)

    NAUX = 4                        # streams the per-tensor statistics are spread over

    def _side_info(self, d, a, layout, nrow, ncol):
        """every tensor's statistics (and row fingerprints) on the device: the launches forked onto
        NAUX streams so the small tensors overlap, joined back into the codec's stream; returns the
        device arrays (all tensors, at their row / column bases) and their host copies"""
        st = self.stream
        rb, cb, _, _ = bases(layout)
        if not hasattr(self, "_aux"):
            self._aux = [dev.Stream() for _ in range(self.NAUX)]
        rfi_d, cfi_d = dev.DeviceArray(max(nrow, 1), np.int16), dev.DeviceArray(max(ncol, 1), np.int16)
        scl_d = dev.DeviceArray(max(ncol, 1), np.int8)
        h_d = dev.DeviceArray(max(nrow, 1), np.uint64) if self.dedup else None
        wb = max(lib().spa_r2_stats_work_bytes(nb // 2 // rl, rl) for _, nb, rl, _ in layout["t"])
        works = [dev.DeviceArray(wb, np.uint8) for _ in self._aux]
        fork = dev.Event()
        fork.record(st)
        for s in self._aux:
            s.wait(fork)
        for i, (off, nb, rl, _) in enumerate(layout["t"]):
            k = i % len(self._aux)
            check(lib().spa_r2_stats(d.ptr + off - a, nb // 2 // rl, rl, rfi_d.ptr + 2 * rb[i], cfi_d.ptr + 2 * cb[i],
                                     scl_d.ptr + cb[i], None if h_d is None else h_d.ptr + 8 * rb[i], works[k].ptr, wb,
                                     None, self._aux[k].handle))
        joins = []
        for s in self._aux:
            e = dev.Event()
            e.record(s.handle)
            check(lib().spa_stream_wait_event(st, e.handle))
            joins.append(e)
        host = [x.to_host(stream=st) for x in (rfi_d, cfi_d, scl_d)]
        hh = h_d.to_host(stream=st) if h_d is not None else None
        del works, joins
        return (rfi_d, cfi_d, scl_d), host[0][:nrow], host[1][:ncol], host[2][:ncol], hh

    def compress(self, data, layout):
        """the coded parts of the file's 2-D BF16 tensors: dict(meta, side, tables, lens, stream) as
        bytes in the reference's chunk format, and the arrays they hold (rfi, cfi, scl, counts, freq,
        used, lens, nrows_c, dups)"""
        st = self.stream
        tm = _Timer(self.timing, st)
        rb, cb, nrow, ncol = bases(layout)
        nt = len(layout["t"])
        rfi = np.zeros(nrow, np.int16); cfi = np.zeros(ncol, np.int16); scl = np.zeros(ncol, np.int8)
        nrows_c, dup_pairs, rmap_all, rmap_off, nrm = {}, {}, [], {}, 0
        if isinstance(data, dev.DeviceArray):           # the file already resident (compress_dev)
            d, a, host = data, 0, None
        elif self.stream_bytes is not None and nt and \
                max(off + nb for off, nb, _, _ in layout["t"]) - layout["t"][0][0] > self.stream_bytes:
            return self.compress_grouped(np.frombuffer(data, np.uint8), layout)
        else:
            host = np.frombuffer(data, np.uint8)
            a = layout["t"][0][0] if nt else 0
            b = max((off + nb for off, nb, _, _ in layout["t"]), default=0)
            d = dev.DeviceArray.from_host(host[a:b] if b > a else np.zeros(1, np.uint8), st)
        tm.lap("upload")

        def rows_of(off, rl):
            """the BF16 bits of some rows of the tensor at file offset `off`"""
            if host is not None:
                return lambda ids: [host[off + 2 * rl * int(r):off + 2 * rl * (int(r) + 1)].view(np.uint16) for r in ids]
            return lambda ids: [d.view(off - a + 2 * rl * int(r), (rl,), np.uint16).to_host(stream=st) for r in ids]

        tm.mark("stats")
        if nt:
            side_dev, rfi, cfi, scl, hh = self._side_info(d, a, layout, nrow, ncol)
        else:
            side_dev, hh = [dev.DeviceArray(1, x.dtype) for x in (rfi, cfi, scl)], None
        tm.mark(None)
        tm.lap("stats")
        for i in range(nt):
            off, nb, rl, _ = layout["t"][i]
            nr = nb // 2 // rl
            keep, pairs = _dups(hh[rb[i]:rb[i] + nr], rows_of(off, rl), rl) if self.dedup else (None, [])
            nrows_c[i] = nr if keep is None else len(keep)
            if keep is not None:
                rmap_off[i] = nrm; nrm += len(keep); rmap_all.append(keep)
                dup_pairs[i] = pairs
        counts = dev.DeviceArray((layout["nroles"] * TPT, 256), np.uint32).zero(st)
        tb, sg = plan(layout, list(range(nt)), nrows_c, rmap_off, rfi, cfi) if nt else (np.zeros(0, TB_DT), np.zeros(0, SG_DT))
        if nt:
            tb["doff"] += layout["t"][0][0] - a
        nseg = len(sg)
        rowmap = np.concatenate(rmap_all).astype(np.int32) if rmap_all else np.zeros(1, np.int32)
        tb_d = dev.DeviceArray.from_host(tb.view(np.uint8) if nt else np.zeros(32, np.uint8), st)
        sg_d = dev.DeviceArray.from_host(sg.view(np.uint8) if nseg else np.zeros(16, np.uint8), st)
        rm_d = dev.DeviceArray.from_host(rowmap, st)
        tm.mark("hist")
        check(lib().spa_r2_hist(d.ptr, tb_d.ptr, sg_d.ptr, nseg, side_dev[0].ptr, side_dev[1].ptr, side_dev[2].ptr,
                                rm_d.ptr, counts.ptr, st))
        tm.mark(None)
        tm.lap("dups")
        # the side information and the metadata are final here: their zstd-19 runs on the host
        # while the device codes the stream
        dups = [[i, r, s_] for i, ps in dup_pairs.items() for r, s_ in ps]
        meta = dict(layout=layout, dups=dups, nrows_c=[nrows_c[i] for i in range(nt)])
        pool = ThreadPoolExecutor(2)
        meta_job = pool.submit(zstd.compress, json.dumps(meta).encode(), 19)
        side_job = pool.submit(zstd.compress, rfi.tobytes() + cfi.tobytes() + scl.tobytes(), 19)
        counts_h = counts.to_host(stream=st)
        tm.lap("hist")
        freq, used = normalize(counts_h)
        tm.lap("normalize")
        remap = np.full(counts_h.shape[0], -1, np.int32)
        remap[used] = np.arange(len(used), dtype=np.int32)
        remap_d, freq_d, cum_d = (dev.DeviceArray.from_host(x if len(x) else np.zeros((1,) + x.shape[1:], x.dtype), st)
                                  for x in (remap, freq, cum_of(freq)))
        fcw = dev.DeviceArray((max(1, len(remap)), 256), np.uint32)
        check(lib().spa_r2_encode_tables(remap_d.ptr, len(remap), freq_d.ptr, cum_d.ptr, fcw.ptr, st))
        streams, lens_all = [], []
        nbat = min(max(nseg, 1), self.enc_batch)
        fc = dev.DeviceArray(-(-nbat // 64) * 64 * SEG * 3, np.uint32)
        out = dev.DeviceArray(nbat * CAP, np.uint8)
        out_len = dev.DeviceArray(nbat, np.uint32)
        for s0 in range(0, nseg, nbat):
            n = min(nbat, nseg - s0)
            tm.mark("encode")
            check(lib().spa_r2_encode(d.ptr, tb_d.ptr, sg_d.ptr + 16 * s0, n, side_dev[0].ptr, side_dev[1].ptr,
                                      side_dev[2].ptr, rm_d.ptr, fcw.ptr, fc.ptr, out.ptr, CAP, out_len.ptr, st))
            tm.mark(None)
            lens = out_len.to_host(stream=st)[:n]
            if (lens == 0xFFFFFFFF).any():
                raise RuntimeError("R2: rANS segment overflow")
            offs = np.zeros(n + 1, np.uint64)
            offs[1:] = np.cumsum(lens.astype(np.uint64))
            dst = dev.DeviceArray(max(1, int(offs[-1])), np.uint8)
            offs_d = dev.DeviceArray.from_host(offs, st)
            tm.mark("gather")
            check(lib().spa_qr_gather(out.ptr, CAP, out_len.ptr, offs_d.ptr, n, dst.ptr, st))
            tm.mark(None)
            piece = dev.pinned(int(offs[-1]))            # read back at the link's full rate
            if len(piece):
                check(lib().spa_memcpy_d2h(piece.ctypes.data, dst.ptr, len(piece), st))
            streams.append(piece)
            lens_all.append(lens)
        tm.lap("encode")
        lens = np.concatenate(lens_all).astype(np.uint32) if lens_all else np.zeros(0, np.uint32)
        # the coded stream: one piece per encoder batch, kept in pieces (pack_parts splices them)
        stream = streams[0] if len(streams) == 1 else (streams or np.zeros(0, np.uint8))
        small = {"meta": meta_job.result(), "side": side_job.result(), "tables": store_tables(freq, used),
                 "lens": zstd.compress(lens.tobytes(), 19)}
        pool.shutdown()
        tm.lap("zstd")
        self.last_timing = tm.result()
        return {**small, "stream": stream,
                "arrays": dict(rfi=rfi, cfi=cfi, scl=scl, counts=counts_h, freq=freq, used=used, lens=lens,
                               nrows_c=np.array(meta["nrows_c"], np.int64),
                               dups=np.array(dups, np.int64).reshape(-1, 3), rowmap=rowmap)}

    def compress_grouped(self, host, layout):
        """compress() of a file in host memory with at most about `stream_bytes` of it in HBM at a
        time: the tensors in groups (a group ends before the tensor that would take it past
        stream_bytes; a bigger tensor is a group of its own), each group uploaded twice. First pass:
        the group's statistics and duplicate rows, its segment plan (device offsets from the group's
        first tensor; the rows kept index the file-wide row map) and histogram; second pass, once
        the tables are normalised: its segments coded and gathered. The counts are sums, every
        segment is coded alone and the stream is the segments in tensor order, so the parts are
        those of compress() (the reference reads a big base twice as well, bf16v2.py:293-321)."""
        st = self.stream
        tm = _Timer(self.timing, st)
        rb, cb, nrow, ncol = bases(layout)
        t = layout["t"]
        nt = len(t)
        groups, cur, size = [], [], 0
        for i, (off, nb, _, _) in enumerate(t):
            if cur and size + nb > self.stream_bytes:
                groups.append(cur)
                cur, size = [], 0
            cur.append(i)
            size += nb
        if cur:
            groups.append(cur)
        span = lambda g: (t[g[0]][0], t[g[-1]][0] + t[g[-1]][1])
        gbuf = dev.DeviceArray(max(max(b_ - a_ for a_, b_ in map(span, groups)), 1), np.uint8)
        rfi_d, cfi_d = dev.DeviceArray(max(nrow, 1), np.int16), dev.DeviceArray(max(ncol, 1), np.int16)
        scl_d = dev.DeviceArray(max(ncol, 1), np.int8)
        h_d = dev.DeviceArray(max(nrow, 1), np.uint64) if self.dedup else None
        rm_d = dev.DeviceArray(max(nrow, 1), np.int32)
        wb = max(lib().spa_r2_stats_work_bytes(nb // 2 // rl, rl) for _, nb, rl, _ in t)
        work = dev.DeviceArray(wb, np.uint8)
        counts = dev.DeviceArray((layout["nroles"] * TPT, 256), np.uint32).zero(st)
        nrows_c, dup_pairs, rmap_off, nrm, plans = {}, {}, {}, 0, []
        rfi = np.zeros(nrow, np.int16); cfi = np.zeros(ncol, np.int16); scl = np.zeros(ncol, np.int8)
        for g in groups:
            ga, gb_ = span(g)
            check(lib().spa_memcpy_h2d(gbuf.ptr, host[ga:gb_].ctypes.data, gb_ - ga, st))
            tm.lap("upload")
            for i in g:
                off, nb, rl, _ = t[i]
                check(lib().spa_r2_stats(gbuf.ptr + off - ga, nb // 2 // rl, rl, rfi_d.ptr + 2 * rb[i], cfi_d.ptr + 2 * cb[i],
                                         scl_d.ptr + cb[i], None if h_d is None else h_d.ptr + 8 * rb[i], work.ptr, wb,
                                         None, st))
            r0, r1 = rb[g[0]], rb[g[-1]] + t[g[-1]][1] // 2 // t[g[-1]][2]
            c0, c1 = cb[g[0]], cb[g[-1]] + t[g[-1]][2]
            rfi[r0:r1] = rfi_d.view(2 * r0, (r1 - r0,), np.int16).to_host(stream=st)
            cfi[c0:c1] = cfi_d.view(2 * c0, (c1 - c0,), np.int16).to_host(stream=st)
            scl[c0:c1] = scl_d.view(c0, (c1 - c0,), np.int8).to_host(stream=st)
            hh = h_d.view(8 * r0, (r1 - r0,), np.uint64).to_host(stream=st) if h_d is not None else None
            tm.lap("stats")
            for i in g:
                off, nb, rl, _ = t[i]
                nr = nb // 2 // rl
                rows = lambda ids, off=off, rl=rl: [host[off + 2 * rl * int(r):off + 2 * rl * (int(r) + 1)].view(np.uint16)
                                                    for r in ids]
                keep, pairs = _dups(hh[rb[i] - r0:rb[i] - r0 + nr], rows, rl) if self.dedup else (None, [])
                nrows_c[i] = nr if keep is None else len(keep)
                if keep is not None:
                    check(lib().spa_memcpy_h2d(rm_d.ptr + 4 * nrm, keep.ctypes.data, 4 * len(keep), st))
                    rmap_off[i] = nrm
                    nrm += len(keep)
                    dup_pairs[i] = pairs
            tm.lap("dups")
            tb, sg = plan(layout, g, nrows_c, rmap_off, rfi, cfi)
            tb_d = dev.DeviceArray.from_host(tb.view(np.uint8), st)
            sg_d = dev.DeviceArray.from_host(sg.view(np.uint8) if len(sg) else np.zeros(16, np.uint8), st)
            check(lib().spa_r2_hist(gbuf.ptr, tb_d.ptr, sg_d.ptr, len(sg), rfi_d.ptr, cfi_d.ptr, scl_d.ptr, rm_d.ptr,
                                    counts.ptr, st))
            plans.append((ga, gb_, tb_d, sg_d, len(sg)))
            tm.lap("hist")
        dups = [[i, r, s_] for i in sorted(dup_pairs) for r, s_ in dup_pairs[i]]
        meta = dict(layout=layout, dups=dups, nrows_c=[nrows_c[i] for i in range(nt)])
        pool = ThreadPoolExecutor(2)
        meta_job = pool.submit(zstd.compress, json.dumps(meta).encode(), 19)
        side_job = pool.submit(zstd.compress, rfi.tobytes() + cfi.tobytes() + scl.tobytes(), 19)
        counts_h = counts.to_host(stream=st)
        freq, used = normalize(counts_h)
        tm.lap("normalize")
        remap = np.full(counts_h.shape[0], -1, np.int32)
        remap[used] = np.arange(len(used), dtype=np.int32)
        remap_d, freq_d, cum_d = (dev.DeviceArray.from_host(x if len(x) else np.zeros((1,) + x.shape[1:], x.dtype), st)
                                  for x in (remap, freq, cum_of(freq)))
        fcw = dev.DeviceArray((max(1, len(remap)), 256), np.uint32)
        check(lib().spa_r2_encode_tables(remap_d.ptr, len(remap), freq_d.ptr, cum_d.ptr, fcw.ptr, st))
        streams, lens_all = [], []
        nbat = max(1, min(max(n for *_, n in plans), self.enc_batch))
        fc = dev.DeviceArray(-(-nbat // 64) * 64 * SEG * 3, np.uint32)
        out = dev.DeviceArray(nbat * CAP, np.uint8)
        out_len = dev.DeviceArray(nbat, np.uint32)
        for ga, gb_, tb_d, sg_d, nseg in plans:
            check(lib().spa_memcpy_h2d(gbuf.ptr, host[ga:gb_].ctypes.data, gb_ - ga, st))
            tm.lap("upload")
            for s0 in range(0, nseg, nbat):
                n = min(nbat, nseg - s0)
                check(lib().spa_r2_encode(gbuf.ptr, tb_d.ptr, sg_d.ptr + 16 * s0, n, rfi_d.ptr, cfi_d.ptr, scl_d.ptr,
                                          rm_d.ptr, fcw.ptr, fc.ptr, out.ptr, CAP, out_len.ptr, st))
                lens = out_len.to_host(stream=st)[:n]
                if (lens == 0xFFFFFFFF).any():
                    raise RuntimeError("R2: rANS segment overflow")
                offs = np.zeros(n + 1, np.uint64)
                offs[1:] = np.cumsum(lens.astype(np.uint64))
                dst = dev.DeviceArray(max(1, int(offs[-1])), np.uint8)
                offs_d = dev.DeviceArray.from_host(offs, st)
                check(lib().spa_qr_gather(out.ptr, CAP, out_len.ptr, offs_d.ptr, n, dst.ptr, st))
                piece = dev.pinned(int(offs[-1]))
                if len(piece):
                    check(lib().spa_memcpy_d2h(piece.ctypes.data, dst.ptr, len(piece), st))
                streams.append(piece)
                lens_all.append(lens)
            tm.lap("encode")
        lens = np.concatenate(lens_all).astype(np.uint32) if lens_all else np.zeros(0, np.uint32)
        stream = streams[0] if len(streams) == 1 else (streams or np.zeros(0, np.uint8))
        small = {"meta": meta_job.result(), "side": side_job.result(), "tables": store_tables(freq, used),
                 "lens": zstd.compress(lens.tobytes(), 19)}
        pool.shutdown()
        tm.lap("zstd")
        self.last_timing = tm.result()
        rowmap = rm_d.view(0, (nrm,), np.int32).to_host(stream=st) if nrm else np.zeros(1, np.int32)
        return {**small, "stream": stream,
                "arrays": dict(rfi=rfi, cfi=cfi, scl=scl, counts=counts_h, freq=freq, used=used, lens=lens,
                               nrows_c=np.array(meta["nrows_c"], np.int64),
                               dups=np.array(dups, np.int64).reshape(-1, 3), rowmap=rowmap)}

    # the parts' order in a chunk: compress_parts' (bf16v2.py:276-291) and, for a base the reference
    # writes while coding it, compress_stream's (bf16v2.py:293-321); unpack() finds parts by name
    ORDER = {"parts": ("meta", "side", "tables", "lens", "stream", "rest"),
             "stream": ("meta", "side", "tables", "stream", "lens", "rest")}

    def compress_parts(self, data, layout, rest=None, order="parts"):
        """compress() as a chunk, pack_parts' list of buffers: meta, side, tables, lens, stream, rest
        (order="stream": meta, side, tables, stream, lens, rest). `rest`: the header coder's output
        for the file's other bytes (seedpack_amd.header.header_c); default its lzma form; needed when
        `data` is on the device"""
        ch = self.compress(data, layout)
        if rest is None:
            if isinstance(data, dev.DeviceArray):
                raise ValueError("R2: a device-resident file needs its `rest` part from the caller")
            rest = header_x(rest_of(data, layout))
        ch["rest"] = rest
        return pack_parts({k: ch[k] for k in self.ORDER[order]})

    def decompress(self, parts, out=None, device=False, alloc=None, into=None, rest=None, stream_dev=None):
        """the file back (bf16v2.py:422-486): `parts` is compress()'s dict or a packed chunk
        (compress_parts' bytes); the coded tensors are decoded on the device, the other bytes come
        from `out` (already in place) or from the "rest" part when there is one, else zeros.
        alloc(n) -> writable uint8 array for the output. device=True: the result stays in HBM, a
        DeviceArray of the file's bytes up to the end of its last coded tensor, only the coded
        tensors written (decompress_dev); device="full": the whole file in HBM (in `into`, a
        DeviceArray of the file's size, if given), the other bytes uploaded from the "rest" part
        (-> (DeviceArray, rest_of bytes)); rest: that part already decoded (header_d), if it is;
        stream_dev: (device="full") the "stream" part already in HBM (stream_buffer(), filled)."""
        st = self.stream
        tm = _Timer(self.timing, st)
        if not isinstance(parts, dict):
            parts = unpack(parts if isinstance(parts, memoryview) else memoryview(parts))
        dec = _Decoder(parts.__getitem__, st, tm)
        tm.lap("tables")
        layout, nt = dec.layout, len(dec.layout["t"])
        if device == "full":
            return self._decompress_full(parts, dec, tm, into, rest, stream_dev)
        if nt == 0 and device:
            return dev.DeviceArray(1, np.uint8)
        if nt:
            a = 0 if device else layout["t"][0][0]
            b = max(off + nb for off, nb, _, _ in layout["t"])
            d = dev.DeviceArray(b - a, np.uint8)
            s_d = _Decoder.upload(parts["stream"], st)
            tm.lap("upload")
            idxs = list(range(nt))
            dec.run(s_d, dec.soff[:-1], d, idxs, [layout["t"][i][0] - a for i in idxs], tm)
            tm.lap("decode")
            if device:
                dev.synchronize(st)
                self.last_timing = tm.result()
                return d
            g = d.to_host(stream=st)
            tm.lap("readback")
            self.last_timing = tm.result()
        if out is None:
            out = alloc(layout["size"]) if alloc else np.zeros(layout["size"], np.uint8)
        for off, nb, _, _ in layout["t"]:
            out[off:off + nb] = g[off - a:off - a + nb]
        if "rest" in parts:
            fill_rest(out, header_d(bytes(parts["rest"])), layout)
        return out

    def _decompress_full(self, parts, dec, tm, into=None, rest=None, stream_dev=None):
        st, layout = self.stream, dec.layout
        if into is not None and into.nbytes != layout["size"]:
            raise ValueError(f"a file of {layout['size']} bytes for a place of {into.nbytes}")
        d = into if into is not None else dev.DeviceArray(max(1, layout["size"]), np.uint8)
        t = layout["t"]
        if t:
            if stream_dev is not None and stream_dev.nbytes < len(parts["stream"]):
                raise ValueError("the device stream is shorter than the chunk's stream part")
            s_d = stream_dev if stream_dev is not None else _Decoder.upload(parts["stream"], st)
            idxs = list(range(len(t)))
            dec.run(s_d, dec.soff[:-1], d, idxs, [x[0] for x in t], tm)
        if rest is None:
            rest = np.frombuffer(header_d(bytes(parts["rest"])), np.uint8)
        upload_rest(d, layout, rest, st)
        self.last_timing = tm.result()
        return d, rest


def upload_rest(d, layout, rest, st):
    """the file's bytes between its coded tensors (the decoded "rest" part, in file order) into the
    device copy d of the file; returns once they are there"""
    t = layout["t"]
    staged = dev.pinned(max(1, rest.size))
    staged[:] = rest
    pos = taken = 0
    for off, nb, *_ in t + [[layout["size"], 0]]:
        if off > pos:
            check(lib().spa_memcpy_h2d(d.ptr + pos, staged[taken:].ctypes.data, off - pos, st))
            taken += off - pos
        pos = off + nb
    dev.synchronize(st)


def stream_buffer(n):
    """a device buffer for n bytes of coded stream, padded to a whole number of 16-byte blocks (the
    decoder's reads)"""
    return dev.DeviceArray(max(16, -(-n // 16) * 16), np.uint8)


class _Decoder:
    """the decode side's tables and maps (bf16v2.py:425-451, :496-530): side information, compact
    decode tables and remap on the device, segment lengths and stream offsets, duplicate rows"""

    def __init__(self, part, st, tm=None):
        self.st = st
        meta = json.loads(zstd.decompress(bytes(part("meta"))))
        self.layout = layout = meta["layout"]
        t = layout["t"]
        self.rb, self.cb, nrow, ncol = bases(layout)
        side = zstd.decompress(bytes(part("side")))
        host = (np.frombuffer(side, np.int16, nrow, 0), np.frombuffer(side, np.int16, ncol, 2 * nrow),
                np.frombuffer(side, np.int8, ncol, 2 * nrow + 2 * ncol))
        self.side = [dev.DeviceArray.from_host(np.ascontiguousarray(x) if len(x) else np.zeros(1, x.dtype), st) for x in host]
        freq, used = load_tables(part("tables"))
        nctx = layout["nroles"] * TPT
        remap = np.full(max(1, nctx), -1, np.int32)
        remap[used] = np.arange(len(used), dtype=np.int32)
        cum_d = dev.DeviceArray.from_host(cum_of(freq) if len(freq) else np.zeros((1, 257), np.uint32), st)
        remap_d = dev.DeviceArray.from_host(remap, st)
        self.dtab = dev.DeviceArray((max(1, nctx), lib().spa_r2_dec_table_bytes()), np.uint8)
        if tm:
            tm.mark("tables")
        check(lib().spa_r2_build_dec_tables(cum_d.ptr, remap_d.ptr, nctx, self.dtab.ptr, st))
        if tm:
            tm.mark(None)
        self._keep = [cum_d, remap_d]
        lens = np.frombuffer(zstd.decompress(bytes(part("lens"))), np.uint32)
        self.nrows_c = meta["nrows_c"]
        nseg = [-(-self.nrows_c[i] * rl // SEG) for i, (_, _, rl, _) in enumerate(t)]
        self.seg0 = np.zeros(len(t) + 1, np.int64)
        self.seg0[1:] = np.cumsum(nseg)
        if self.seg0[-1] != len(lens):
            raise ValueError("R2: segment lengths do not match the layout")
        self.soff = np.zeros(len(lens) + 1, np.uint64)
        self.soff[1:] = np.cumsum(lens, dtype=np.uint64)
        self.dups = {}
        for i, r, s_ in meta["dups"]:
            self.dups.setdefault(i, []).append((r, s_))
        rmap_all, self.rmap_off = [], {}            # the encoder's construction order
        for i in range(len(t)):
            if i in self.dups:
                rl = t[i][2]
                isdup = np.zeros(t[i][1] // 2 // rl, bool)
                isdup[[r for r, _ in self.dups[i]]] = True
                self.rmap_off[i] = sum(len(x) for x in rmap_all)
                rmap_all.append(np.flatnonzero(~isdup).astype(np.int32))
        self.rowmap = dev.DeviceArray.from_host(np.concatenate(rmap_all) if rmap_all else np.zeros(1, np.int32), st)

    @staticmethod
    def upload(stream_h, st):
        """coded stream bytes (a bytes-like or a list of pieces) -> device, padded to a whole number
        of 16-byte blocks (the decoder's reads)"""
        pieces = [np.frombuffer(p, np.uint8) for p in (stream_h if isinstance(stream_h, list) else [stream_h])]
        n = sum(len(p) for p in pieces)
        d = stream_buffer(n)
        o = 0
        for p in pieces:
            if len(p):
                check(lib().spa_memcpy_h2d(d.ptr + o, np.ascontiguousarray(p).ctypes.data, len(p), st))
            o += len(p)
        return d

    def run(self, s_d, in_off, d, idxs, doffs, tm=None):
        """decode tensors idxs from the device stream s_d (from upload(); in_off: each of their
        segments' byte offset in it, in order) into d at byte offsets doffs, duplicate rows restored"""
        st, t = self.st, self.layout["t"]
        tb = np.zeros(len(idxs), TB_DT)
        segs = []
        for k, i in enumerate(idxs):
            off, nb, rl, _ = t[i]
            tb[k] = (doffs[k], rl, self.rb[i], self.cb[i], self.layout["role"][i] * TPT, self.rmap_off.get(i, -1), 0)
            n = self.nrows_c[i] * rl
            sg = np.zeros(-(-n // SEG), SG_DT)
            sg["t"] = k
            sg["i0"] = np.arange(0, n, SEG)
            sg["n"] = np.minimum(SEG, n - sg["i0"])
            segs.append(sg)
        sg = np.concatenate(segs) if segs else np.zeros(0, SG_DT)
        if len(in_off) != len(sg):
            raise ValueError("R2: segment offsets do not match the tensors")
        keep = [dev.DeviceArray.from_host(np.ascontiguousarray(in_off, np.uint64) if len(sg) else np.zeros(1, np.uint64), st),
                dev.DeviceArray.from_host(tb.view(np.uint8) if len(tb) else np.zeros(32, np.uint8), st),
                dev.DeviceArray.from_host(sg.view(np.uint8) if len(sg) else np.zeros(16, np.uint8), st)]
        if tm:
            tm.mark("decode")
        check(lib().spa_r2_decode(s_d.ptr, s_d.nbytes, keep[0].ptr, d.ptr, keep[1].ptr, keep[2].ptr, len(sg),
                                  self.side[0].ptr, self.side[1].ptr, self.side[2].ptr, self.rowmap.ptr, self.dtab.ptr, st))
        if tm:
            tm.mark("copy_rows")
        for k, i in enumerate(idxs):
            if i in self.dups:
                rl = t[i][2]
                pairs = dev.DeviceArray.from_host(np.array(self.dups[i], np.int64).reshape(-1), st)
                keep.append(pairs)
                check(lib().spa_r2_copy_rows(d.ptr + doffs[k], rl, pairs.ptr, len(self.dups[i]), st))
        if tm:
            tm.mark(None)
        dev.synchronize(st)              # the descriptors above are freed on return
        return d


class R2Tensors:
    """random access to an R2-coded file (bf16v2.py:488-617): any of its 2-D BF16 tensors decoded
    alone on the device, the file's other bytes from the "rest" part. part(name) -> bytes of a small
    part; read(offset, n, out) reads n bytes of the coded stream (offset from its start) into the
    writable uint8 array `out`.

    Per tensor i: its segments are seg0[i]..seg0[i+1] of the stream, their bytes soff[seg0[i]] ..
    soff[seg0[i+1]]. A file position outside the coded tensors maps to position - (coded bytes
    before it) of the rest."""

    def __init__(self, part, read, stream=None):
        self.read, self.stream = read, stream
        self.dec = _Decoder(part, stream)
        self.layout = self.dec.layout
        self.size = self.layout["size"]
        t = self.layout["t"]
        self.index = {x[0]: i for i, x in enumerate(t)}           # file offset -> tensor index
        self._starts = np.array([x[0] for x in t], np.int64)
        self._coded_before = np.concatenate([[0], np.cumsum([x[1] for x in t])]).astype(np.int64)
        seg_off = self.dec.soff[self.dec.seg0].astype(np.int64)       # stream offset of each tensor's first segment
        self._span = np.stack([seg_off[:-1], seg_off[1:]], 1)        # [tensor] -> stream bytes [a, b)
        self.rest = np.frombuffer(header_d(bytes(part("rest"))), np.uint8)

    def coded_bytes(self, i):
        """bytes of the coded stream of tensor i"""
        a, b = self._span[i]
        return int(b - a)

    def outside(self, a, b):
        """bytes [a, b) of the file, a range that no coded tensor overlaps"""
        k = int(np.searchsorted(self._starts, a, side="right"))      # coded tensors starting at or before a
        r = a - int(self._coded_before[k])
        return self.rest[r:r + (b - a)]

    def fetch(self, idxs):
        """the coded streams of tensors idxs read into one host buffer (neighbouring ranges in one
        read) -> argument of decode(): (tensor indices, buffer, each tensor's offset in it)"""
        idxs = list(idxs)
        order = sorted(idxs, key=lambda i: self._span[i][0])
        runs = []                                   # [stream start, stream end, tensors]
        for i in order:
            a, b = (int(v) for v in self._span[i])
            if runs and runs[-1][1] == a:
                runs[-1][1] = b
                runs[-1][2].append(i)
            else:
                runs.append([a, b, [i]])
        host = np.empty(max(1, sum(b - a for a, b, _ in runs)), np.uint8)
        at, o = {}, 0
        for a, b, members in runs:
            self.read(a, b - a, host[o:o + b - a])
            for i in members:
                at[i] = o + int(self._span[i][0]) - a
            o += b - a
        return idxs, host, at

    def decode(self, idxs):
        """coded tensors idxs (layout indices, or what fetch() returned) -> (DeviceArray, byte offset
        of each tensor in it, 256-byte aligned)"""
        t = self.layout["t"]
        idxs, host, at = idxs if isinstance(idxs, tuple) else self.fetch(idxs)
        soff, seg0 = self.dec.soff, self.dec.seg0
        in_off, outs, doff = [], [], 0
        for i in idxs:
            segs = soff[seg0[i]:seg0[i + 1]].astype(np.int64)
            in_off.append((segs - segs[0] + at[i]).astype(np.uint64) if len(segs) else np.zeros(0, np.uint64))
            outs.append(doff)
            doff += -(-t[i][1] // 256) * 256
        d = dev.DeviceArray(max(doff, 1), np.uint8)
        s_d = _Decoder.upload(host, self.stream)
        self.dec.run(s_d, np.concatenate(in_off) if in_off else np.zeros(0, np.uint64), d, idxs, outs)
        return d, outs

    def write_to(self, write, window=1 << 30):
        """the whole file in order through write(bytes-like), decoding about `window` bytes of tensors
        at a time; write() runs on a worker thread, one window behind the decoding (the device work
        stays on the calling thread and its stream)"""
        t = self.layout["t"]
        runs, i = [], 0
        while i < len(t):
            j = i + 1
            total = t[i][1]
            while j < len(t) and total + t[j][1] <= window:
                total += t[j][1]
                j += 1
            runs.append((i, j))
            i = j
        pos = [0]

        def consume(i, j, h, outs):
            for k in range(i, j):
                off, n = t[k][0], t[k][1]
                if off > pos[0]:
                    write(self.outside(pos[0], off))
                write(h[outs[k - i]:outs[k - i] + n])
                pos[0] = off + n

        with ThreadPoolExecutor(1) as ex:
            pending = None
            for i, j in runs:
                d, outs = self.decode(range(i, j))
                h = d.to_host(stream=self.stream)
                del d
                if pending is not None:
                    pending.result()
                pending = ex.submit(consume, i, j, h, outs)
            if pending is not None:
                pending.result()
        if pos[0] < self.size:
            write(self.outside(pos[0], self.size))
