"""Host side of the R2 BF16 base codec over the HIP C ABI (the reference's seedpack/bf16v2.py BF16v2).

compress(data, layout) -> parts and decompress(parts) -> the tensors' bytes keep BF16v2's
algorithm and stream format (bf16v2.py:185-486): side information per tensor (rfi, cfi, scl),
exact duplicate rows coded once, per-role frequency tables (656 per role: 512 exponent, 128
mantissa, 16 sign contexts) normalised to 2^15, and rANS segments of 16384 weights, the tensors
processed in groups of at most `group_bytes`. The statistics, fingerprints, histogram, symbol
lookups, coding, gather and decoding run as HIP kernels; the duplicate-row check, the table
normalisation (gpu2.normalize_gpu, a loop over a few hundred rows) and the framing run on the host.

`layout` is BF16v2._layout's dict (bf16v2.py:182-188): {"size": file bytes, "t": [[offset, bytes,
row length, "bf16"], ...] (2-D BF16 tensors by offset), "role": role index per tensor, "nroles"}.
Outside this module: GGUF parsing and the header coder of the file's other bytes ("rest" part,
gpu_bf16.py:421-428).
"""
import ctypes
import json
import re
import struct

import numpy as np

from . import device as dev
from . import zstd
from ._lib import check, lib

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


def groups(layout, group_bytes):
    gs, cur, cb = [], [], 0
    for i, (off, nb, rl, _) in enumerate(layout["t"]):
        if cur and cb + nb > group_bytes:
            gs.append(cur)
            cur, cb = [], 0
        cur.append(i)
        cb += nb
    if cur:
        gs.append(cur)
    return gs


def bases(layout):
    rb, cb, rowbase, colbase = [], [], 0, 0
    for off, nb, rl, _ in layout["t"]:
        rb.append(rowbase)
        cb.append(colbase)
        rowbase += nb // 2 // rl
        colbase += rl
    return rb, cb, rowbase, colbase


def plan(layout, grp, nrows_c, rmap_off):
    """(TB, SG) descriptors of one group, device offsets relative to the group's first tensor
    (bf16v2.py:208-220)"""
    rb, cb, _, _ = bases(layout)
    tb = np.zeros(len(grp), TB_DT)
    segs = []
    a = layout["t"][grp[0]][0]
    for k, i in enumerate(grp):
        off, nb, rl, _ = layout["t"][i]
        tb[k] = (off - a, rl, rb[i], cb[i], layout["role"][i] * TPT, rmap_off.get(i, -1), 0)
        n = nrows_c[i] * rl
        for i0 in range(0, n, SEG):
            segs.append((k, min(SEG, n - i0), i0))
    return tb, (np.array(segs, SG_DT) if segs else np.zeros(0, SG_DT))


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
    return zstd.compress(struct.pack("<I", len(u)) + du.tobytes() + np.asarray(freq, np.uint16).tobytes(), 19)


def load_tables(buf):
    raw = zstd.decompress(bytes(buf))
    (n,) = struct.unpack_from("<I", raw)
    used = np.cumsum(np.frombuffer(raw, np.uint32, n, 4).astype(np.int64))
    freq = np.frombuffer(raw, np.uint16, n * 256, 4 + 4 * n).reshape(n, 256)
    return freq, used


def _dups(hashes, u_host, rl):
    """(rows kept (sorted) or None, [(duplicate row, source row)]) from the row fingerprints and a
    byte check of every candidate (bf16v2.py:246-271)"""
    nr = len(hashes)
    order = np.argsort(hashes, kind="stable")
    hs = hashes[order]
    same = np.flatnonzero(hs[1:] == hs[:-1])
    if len(same) == 0:
        return None, []
    hu = u_host.reshape(-1, rl)
    pairs, isdup, first = [], np.zeros(nr, bool), {}
    for k in np.unique(np.concatenate([same, same + 1])):
        r = int(order[k])
        cands = first.setdefault(int(hs[k]), [])
        src = next((c for c in cands if np.array_equal(hu[c], hu[r])), None)
        if src is None:
            cands.append(r)
        else:
            pairs.append((r, src))
            isdup[r] = True
    if not pairs:
        return None, []
    return np.flatnonzero(~isdup).astype(np.int32), sorted(pairs)


def _p(a):
    return None if a is None else a.ptr


class BF16v2:
    """R2 codec core on the MI355X (bf16v2.py:170-617)"""

    def __init__(self, group_bytes=400 << 20, dedup=True, stream=None):
        self.group_bytes, self.dedup, self.stream = group_bytes, dedup, stream

    def stats(self, w_dev, rl, with_hash=True):
        """(rfi, cfi, scl, row hashes or None) of one tensor's BF16 bits on the device, as numpy"""
        nr = w_dev.nbytes // 2 // rl
        rfi, cfi, scl = dev.DeviceArray(nr, np.int16), dev.DeviceArray(rl, np.int16), dev.DeviceArray(rl, np.int8)
        h = dev.DeviceArray(nr, np.uint64) if with_hash else None
        work = dev.DeviceArray(nr, np.float32)
        check(lib().spa_r2_stats(w_dev.ptr, nr, rl, rfi.ptr, cfi.ptr, scl.ptr, _p(h), work.ptr, None, self.stream))
        s = self.stream
        return (rfi.to_host(stream=s), cfi.to_host(stream=s), scl.to_host(stream=s),
                h.to_host(stream=s) if h is not None else None)

    def compress(self, data, layout):
        """the coded parts of the file's 2-D BF16 tensors: dict(meta, side, tables, lens, stream) as
        bytes in the reference's chunk format, and the arrays they hold (rfi, cfi, scl, counts, freq,
        used, lens, nrows_c, dups)"""
        st = self.stream
        host = np.frombuffer(data, np.uint8)
        rb, cb, nrow, ncol = bases(layout)
        rfi = np.zeros(nrow, np.int16); cfi = np.zeros(ncol, np.int16); scl = np.zeros(ncol, np.int8)
        grps = groups(layout, self.group_bytes)
        nrows_c, dup_pairs, rmap_all, nrm = {}, {}, [], 0
        per_group = []
        for grp in grps:
            a = layout["t"][grp[0]][0]
            b = layout["t"][grp[-1]][0] + layout["t"][grp[-1]][1]
            d = dev.DeviceArray.from_host(host[a:b], st)
            rmap_off, mine = {}, []
            for i in grp:
                off, nb, rl, _ = layout["t"][i]
                r_, c_, s_, h = self.stats(d.view(off - a, (nb,), np.uint8), rl, self.dedup)
                rfi[rb[i]:rb[i] + len(r_)] = r_; cfi[cb[i]:cb[i] + rl] = c_; scl[cb[i]:cb[i] + rl] = s_
                keep, pairs = _dups(h, host[off:off + nb].view(np.uint16), rl) if self.dedup else (None, [])
                nrows_c[i] = nb // 2 // rl if keep is None else len(keep)
                if keep is not None:
                    rmap_off[i] = nrm; nrm += len(keep); rmap_all.append(keep); mine.append(keep)
                    dup_pairs[i] = pairs
            per_group.append((d, a, rmap_off, mine))
        side_dev = [dev.DeviceArray.from_host(x, st) for x in (rfi, cfi, scl)]
        counts = dev.DeviceArray((layout["nroles"] * TPT, 256), np.uint32).zero(st)
        plans = []
        for grp, (d, a, rmap_off, mine) in zip(grps, per_group):
            tb, sg = plan(layout, grp, nrows_c, rmap_off)
            if mine:
                tb = tb.copy(); m = tb["rmap"] >= 0; tb["rmap"][m] -= min(rmap_off.values())
                rm = np.concatenate(mine).astype(np.int32)
            else:
                rm = np.zeros(1, np.int32)
            tb_d = dev.DeviceArray.from_host(tb.view(np.uint8), st)
            sg_d = dev.DeviceArray.from_host(sg.view(np.uint8) if len(sg) else np.zeros(16, np.uint8), st)
            rm_d = dev.DeviceArray.from_host(rm, st)
            check(lib().spa_r2_hist(d.ptr, tb_d.ptr, sg_d.ptr, len(sg), side_dev[0].ptr, side_dev[1].ptr, side_dev[2].ptr,
                                    rm_d.ptr, counts.ptr, st))
            plans.append((tb_d, sg_d, rm_d, len(sg)))
        counts_h = counts.to_host(stream=st)
        freq, used = normalize(counts_h)
        remap = np.full(counts_h.shape[0], -1, np.int32)
        remap[used] = np.arange(len(used), dtype=np.int32)
        remap_d, freq_d, cum_d = (dev.DeviceArray.from_host(x, st) for x in (remap, freq, cum_of(freq)))
        streams, lens_all = [], []
        for (d, a, _, _), (tb_d, sg_d, rm_d, nseg) in zip(per_group, plans):
            if nseg == 0:
                continue
            fc = dev.DeviceArray(nseg * SEG * 3, np.uint32)
            out = dev.DeviceArray(nseg * CAP, np.uint8)
            out_len = dev.DeviceArray(nseg, np.uint32).zero(st)
            check(lib().spa_r2_encode(d.ptr, tb_d.ptr, sg_d.ptr, nseg, side_dev[0].ptr, side_dev[1].ptr, side_dev[2].ptr,
                                      rm_d.ptr, remap_d.ptr, freq_d.ptr, cum_d.ptr, fc.ptr, out.ptr, CAP, out_len.ptr, st))
            lens = out_len.to_host(stream=st)
            if (lens == 0xFFFFFFFF).any():
                raise RuntimeError("R2: rANS segment overflow")
            offs = np.zeros(nseg + 1, np.uint64)
            offs[1:] = np.cumsum(lens.astype(np.uint64))
            dst = dev.DeviceArray(max(1, int(offs[-1])), np.uint8)
            offs_d = dev.DeviceArray.from_host(offs, st)
            check(lib().spa_qr_gather(out.ptr, CAP, out_len.ptr, offs_d.ptr, nseg, dst.ptr, st))
            streams.append(dst.to_host(stream=st)[:int(offs[-1])].tobytes())
            lens_all.append(lens)
        lens = np.concatenate(lens_all).astype(np.uint32) if lens_all else np.zeros(0, np.uint32)
        dups = [[i, r, s] for i, ps in dup_pairs.items() for r, s in ps]
        meta = dict(layout=layout, dups=dups, nrows_c=[nrows_c[i] for i in range(len(layout["t"]))])
        stream = b"".join(streams)
        return {"meta": zstd.compress(json.dumps(meta).encode(), 19),
                "side": zstd.compress(rfi.tobytes() + cfi.tobytes() + scl.tobytes(), 19),
                "tables": store_tables(freq, used), "lens": zstd.compress(lens.tobytes(), 19), "stream": stream,
                "arrays": dict(rfi=rfi, cfi=cfi, scl=scl, counts=counts_h, freq=freq, used=used, lens=lens,
                               nrows_c=np.array(meta["nrows_c"], np.int64),
                               dups=np.array(dups, np.int64).reshape(-1, 3),
                               rowmap=np.concatenate(rmap_all).astype(np.int32) if rmap_all else np.zeros(1, np.int32))}

    def decompress(self, parts, out=None):
        """parts (compress()'s byte parts) -> the file with its coded tensors written (bf16v2.py:422-476);
        `out`: the file's other bytes already in place (a uint8 array of the file's size), else zeros"""
        st = self.stream
        meta = json.loads(zstd.decompress(bytes(parts["meta"])))
        layout = meta["layout"]
        nt = len(layout["t"])
        rb, cb, nrow, ncol = bases(layout)
        side = zstd.decompress(bytes(parts["side"]))
        rfi = np.frombuffer(side, np.int16, nrow, 0)
        cfi = np.frombuffer(side, np.int16, ncol, 2 * nrow)
        scl = np.frombuffer(side, np.int8, ncol, 2 * nrow + 2 * ncol)
        side_dev = [dev.DeviceArray.from_host(np.ascontiguousarray(x), st) for x in (rfi, cfi, scl)]
        freq, used = load_tables(parts["tables"])
        cum = cum_of(freq)
        remap = np.full(layout["nroles"] * TPT, -1, np.int32)
        remap[used] = np.arange(len(used), dtype=np.int32)
        freq_d, cum_d, remap_d = (dev.DeviceArray.from_host(np.ascontiguousarray(x), st) for x in (freq, cum, remap))
        lut = dev.DeviceArray((max(1, len(freq)), 1 << PB), np.uint8)
        check(lib().spa_rans_build_lut_pb(cum_d.ptr, len(freq), PB, lut.ptr, st))
        lens = np.frombuffer(zstd.decompress(bytes(parts["lens"])), np.uint32)
        nrows_c = {i: n for i, n in enumerate(meta["nrows_c"])}
        dups = {}
        for i, r, s in meta["dups"]:
            dups.setdefault(i, []).append((r, s))
        rmap_all, rmap_off_t = [], {}
        for i in range(nt):
            if i in dups:
                rl = layout["t"][i][2]
                nr = layout["t"][i][1] // 2 // rl
                isdup = np.zeros(nr, bool)
                isdup[[r for r, _ in dups[i]]] = True
                rmap_off_t[i] = sum(len(x) for x in rmap_all)
                rmap_all.append(np.flatnonzero(~isdup).astype(np.int32))
        rowmap = np.concatenate(rmap_all) if rmap_all else np.zeros(1, np.int32)
        rowmap_d = dev.DeviceArray.from_host(rowmap, st)
        out = np.zeros(layout["size"], np.uint8) if out is None else out
        stream_h = np.frombuffer(bytes(parts["stream"]), np.uint8)
        spos, lpos = 0, 0
        for grp in groups(layout, self.group_bytes):
            rmap_off = {i: rmap_off_t[i] for i in grp if i in rmap_off_t}
            tb, sg = plan(layout, grp, nrows_c, rmap_off)
            gl = lens[lpos:lpos + len(sg)]
            lpos += len(sg)
            nbytes = int(gl.sum(dtype=np.uint64))
            offs = np.zeros(max(1, len(sg)), np.uint64)
            offs[1:len(sg)] = np.cumsum(gl.astype(np.uint64))[:-1]
            a = layout["t"][grp[0]][0]
            b = layout["t"][grp[-1]][0] + layout["t"][grp[-1]][1]
            d = dev.DeviceArray(b - a, np.uint8)
            keep = []                   # device inputs of the launches, alive until the group is read back
            if len(sg):
                s_d = dev.DeviceArray.from_host(stream_h[spos:spos + nbytes] if nbytes else np.zeros(1, np.uint8), st)
                offs_d = dev.DeviceArray.from_host(offs, st)
                tb_d = dev.DeviceArray.from_host(tb.view(np.uint8), st)
                sg_d = dev.DeviceArray.from_host(sg.view(np.uint8), st)
                keep += [s_d, offs_d, tb_d, sg_d]
                check(lib().spa_r2_decode(s_d.ptr, offs_d.ptr, d.ptr, tb_d.ptr, sg_d.ptr, len(sg),
                                          side_dev[0].ptr, side_dev[1].ptr, side_dev[2].ptr, rowmap_d.ptr, remap_d.ptr,
                                          freq_d.ptr, cum_d.ptr, lut.ptr, st))
            spos += nbytes
            for i in grp:
                if i in dups:
                    off, nb, rl, _ = layout["t"][i]
                    pairs = dev.DeviceArray.from_host(np.array(dups[i], np.int64).reshape(-1), st)
                    keep.append(pairs)
                    check(lib().spa_r2_copy_rows(d.ptr + (off - a), rl, pairs.ptr, len(dups[i]), st))
            g = d.to_host(stream=st)
            del keep
            for i in grp:
                off, nb, _, _ = layout["t"][i]
                out[off:off + nb] = g[off - a:off - a + nb]
        return out
