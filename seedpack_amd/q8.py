"""M22, the reference's Q8_0 codec (seedpack/gpu3.py M22Fast over gpu2.GPU2), and Q8Parts, which runs
it over a file in parts of whole tensors (gpu3.py:590-643). SeedCodec (seed.py) uses it for a seed's
Q8_0 tensors.

Per Q8_0 block (fp16 d, 32 int8 weights) the codec sends, with context-modelled rANS (PB 12):
  phase A  the scale's two bytes, the position of the largest |weight| (as its rank among the block's
           columns ordered by column factor) and its value, 4096 blocks per segment;
  phase B  the other 31 weights as magnitude and sign in variance bins from the row mean of the scale
           bits, the column factor and a per-tensor offset, 1024 blocks per segment;
  phase C  token_embd's rows predicted from up to four similar rows of earlier waves (128 waves):
           the residuals (q - prediction) & 255 and the maximum by the prediction, 4 rows per segment.
Rows equal to an earlier row of their tensor are sent as references. The side information (column
factors cfi, sign classes, tensor offsets, parents, coefficients, residual classes) is decided with
detmath's float64 sums in index order and its log2 / exp2, so it does not depend on the device.

The chunk is pack({layout, side, cfi, tables, lens, A, B, scls, [C, Clens, Ctables, Cside, Cpar,
Ccoef, Cfbin, Cmu, Ccadj], [rest]}) with the reference's names, orders and zstd levels (gpu2.py:
673-688, gpu3.py:405-418); "rest" (the bytes around the tensors) is header.py's P, T or X form.
"""
import json
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import detmath
from . import device as dev
from . import gguf, header, zstd
from ._lib import check, lib
from .framing import pack, pack_parts, unpack
from .r2 import cum_of, load_tables, normalize, store_tables

PB = 12
SEGA, SEGB = 4096, 1024                       # blocks per segment, phases A and B (gpu2.py:35-36)
TA = 256 * 16 + 256 + 16 + 16                 # phase A tables per group (gpu2.py:47-51, HICF)
TQ = 64 + 1024                                # phase B tables per table set (gpu2.py:52-53, SIGN)
TPC = 64 + 24                                 # phase C tables per predicted tensor (gpu3.py:31, PREDA)
STAT_ELEMS = 32 << 20                         # weights per slice of the column statistics (gpu2.py:39)
WAVES, KPAR, RPT = 128, 4, 4                  # M22Fast (gpu3.py:579-588), rows per phase C segment
PRED_TENSORS = ("token_embd",)
PRED_MEM, PRED_MAX = 7, 8 << 30               # tensors planned only up to PRED_MEM * bytes <= PRED_MAX (gpu3.py:234-236)
LS_CHUNK = 2048                               # rows per least-squares chunk of the planner (gpu3.py:314)
HIST_ITEM = 4096                              # blocks per phase B histogram work item
Q8_0 = 8
NAME = "M22 = M21 with row prediction for token_embd only, 128 waves (3.7x faster decoding, +0.03%)"

META_DT = np.dtype([(n, "<i4") for n in ("first", "nblocks", "nb_row", "grp", "colbase", "rowbase", "off", "qset")])
ITEM_DT = np.dtype([("t", "<i4"), ("b0", "<i4"), ("nb", "<i4")])
CSEG_DT = np.dtype([("t", "<i4"), ("r0", "<i4"), ("nr", "<i4"), ("slot", "<i4")])
SLOT_DT = np.dtype([("rbase", "<i8"), ("pbase", "<i8"), ("first", "<i4"), ("nbr", "<i4"), ("mubase", "<i4"),
                    ("pad", "<i4")])


def group_of(name):
    """blk.13.ffn_up.weight -> ffn_up; token_embd.weight -> token_embd (codecs_gguf.py:163-166)"""
    p = name.split(".")
    return p[2] if p[0] == "blk" else p[0]


def layout_of(g, size):
    """the Q8_0 tensors by offset: {"size", "t": [[offset, bytes, row length, group]]} (gpu2.py:316-320)"""
    q = sorted((t for t in g.tensors if t.type == Q8_0), key=lambda t: t.offset)
    return {"size": size, "t": [[t.offset, t.nbytes, t.shape[0], group_of(t.name)] for t in q]}


def _meta(layout, off, qset):
    """per tensor META_DT records and the row descriptors (gpu2.py:541-552)"""
    groups = sorted({t[3] for t in layout["t"]})
    m = np.zeros(len(layout["t"]), META_DT)
    first = colbase = rowbase = 0
    for i, (_, nbytes, rowlen, grp) in enumerate(layout["t"]):
        nb, nbr = nbytes // 34, rowlen // 32
        m[i] = (first, nb, nbr, groups.index(grp), colbase, rowbase, off[i], qset[i])
        first += nb
        colbase += rowlen
        rowbase += nb // nbr
    return groups, m


def colblock_side(cfi):
    """per block-column (32 columns): the columns by descending factor (ties by index), its inverse and
    the factor spread bin (gpu2.py:560-567)"""
    c = cfi.reshape(-1, 32).astype(np.int32)
    key = -c * 64 + np.arange(32, dtype=np.int32)[None, :]
    perm = np.argsort(key, axis=1, kind="stable").astype(np.uint8)
    rankof = np.argsort(perm, axis=1, kind="stable").astype(np.uint8)
    spread = np.clip((c.max(1) - np.sort(c, axis=1)[:, 16]) // 2, 0, 15).astype(np.uint8)
    return perm.ravel(), rankof.ravel(), spread


def block_factor_bins(cfi, layout):
    """per block-column: its largest factor against the tensor's mean, quarter-octave bins (gpu2.py:569-575)"""
    out, cb = [], 0
    for _, _, rowlen, _ in layout["t"]:
        c = cfi[cb:cb + rowlen].reshape(-1, 32).astype(np.int32).max(1)
        out.append(np.clip((c - int(c.mean())) // 2 + 8, 0, 15).astype(np.uint8))
        cb += rowlen
    return np.concatenate(out) if out else np.zeros(0, np.uint8)


def _in_order(parts):
    """sum of the rows of `parts` (float64), added in row order"""
    s = np.zeros(parts.shape[1], np.float64)
    for p in parts:
        s = s + p
    return s


def _total(x):
    """float64 sum in index order"""
    x = np.asarray(x, np.float64).ravel()
    return float(np.add.accumulate(x)[-1]) if len(x) else 0.0


def _int8_nan0(v):
    """float array to int8 with NaN as 0 (values already clipped to the int8 range)"""
    v = np.asarray(v)
    return np.where(np.isnan(v), 0, v).astype(np.int8)


def waves_of(n, waves):
    """first and end row of each wave of n rows (gpu3.py:315-319)"""
    wave = (np.arange(n) * waves) // n
    starts = np.searchsorted(wave, np.arange(waves))
    return starts, np.append(starts[1:], n)


def segments(plans, waves, rpt):
    """phase C segments ordered (wave, tensor): CSEG_DT records and wave_start (gpu3.py:321-335)"""
    segs, wave_start = [], []
    se = [waves_of(p["nrows"], waves) for p in plans]
    for w in range(waves):
        wave_start.append(len(segs))
        for slot, p in enumerate(plans):
            a, b = int(se[slot][0][w]), int(se[slot][1][w])
            segs += [(p["t"], r0, min(rpt, b - r0), slot) for r0 in range(a, b, rpt)]
    wave_start.append(len(segs))
    return np.array(segs, CSEG_DT) if segs else np.zeros(0, CSEG_DT), wave_start


class _Tables:
    """normalised tables of device counts: freq / cum / remap / reciprocals on the device"""

    def __init__(self, counts, nrows, st, with_rcp=True):
        c = counts.to_host(stream=st).reshape(nrows, 256)
        self.freq, self.used = normalize(c, 1 << PB)
        self.remap = np.full(max(1, nrows), -1, np.int32)
        self.remap[self.used] = np.arange(len(self.used), dtype=np.int32)
        n = max(1, len(self.used))
        freq = self.freq if len(self.used) else np.zeros((1, 256), np.uint16)
        self.freq_d = dev.DeviceArray.from_host(freq, st)
        self.cum_d = dev.DeviceArray.from_host(cum_of(freq), st)
        self.remap_d = dev.DeviceArray.from_host(self.remap, st)
        self.rcp_d = dev.DeviceArray((n, 256), np.uint32)
        if with_rcp:
            check(lib().spa_q8_rcp(self.freq_d.ptr, n, self.rcp_d.ptr, st))

    def stored(self):
        return store_tables(self.freq, self.used)


def _decoder_tables(buf, ntab, st):
    freq, used = load_tables(buf)
    n = max(1, len(freq))
    used = np.asarray(used, np.int64)
    if len(used) and (used.max() >= ntab or used.min() < 0):
        raise ValueError(f"Q8_0 codec: table id {int(used.max())} outside {ntab} tables")
    remap = np.full(max(1, ntab), -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    freq = np.ascontiguousarray(freq, np.uint16) if len(freq) else np.zeros((1, 256), np.uint16)
    cum = cum_of(freq)
    if (cum[:, 256] != (1 << PB)).any():
        raise ValueError("Q8_0 codec: a stored table does not sum to 4096")
    freq_d, cum_d, remap_d = (dev.DeviceArray.from_host(a, st) for a in (freq, cum, remap))
    lut = dev.DeviceArray((n, 1 << PB), np.uint32)
    check(lib().spa_q8_lut32(freq_d.ptr, cum_d.ptr, n, lut.ptr, st))
    return remap_d, lut


def _gather(out, cap, out_len, nseg, st, what):
    """the segments' bytes back to back and their u16 lengths"""
    lens = out_len.to_host(stream=st)
    if (lens == 0xFFFFFFFF).any():
        raise RuntimeError(f"Q8_0 codec: phase {what} segment overflow")
    if len(lens) and int(lens.max()) >= 65536:
        raise RuntimeError(f"Q8_0 codec: phase {what} segment of {int(lens.max())} bytes (lengths are 16-bit)")
    offs = np.zeros(nseg + 1, np.uint64)
    offs[1:] = np.cumsum(lens.astype(np.uint64))
    dst = dev.DeviceArray(max(1, int(offs[-1])), np.uint8)
    offs_d = dev.DeviceArray.from_host(offs, st)
    check(lib().spa_qr_gather(out.ptr, cap, out_len.ptr, offs_d.ptr, nseg, dst.ptr, st))
    return dst.to_host(stream=st)[:int(offs[-1])], lens.astype(np.uint16)


def _log2(x, st):
    return detmath.log2(np.ascontiguousarray(x, np.float64), st).to_host(stream=st)


class M22:
    """the Q8_0 codec: compress(data, ...) -> chunk bytes, decompress(buf, out=...)"""
    name = NAME

    def __init__(self, stream=None, stat_elems=STAT_ELEMS, timing=False):
        self.stream = stream
        self.stat_elems = stat_elems
        self.timing_on, self.timing = timing, {}
        self._t = time.perf_counter()

    def _lap(self, name):
        """with timing on: the stream drained, the wall seconds since the previous lap added to `name`"""
        if self.timing_on:
            dev.synchronize(self.stream)
            now = time.perf_counter()
            self.timing[name] = round(self.timing.get(name, 0.0) + now - self._t, 4)
            self._t = now

    # ---------------------------------------------------------- encoder
    def compress(self, data, tensors=None, header=True, parsed=None, d=None):
        """data: the file (bytes-like, host); tensors: indices of the Q8_0 tensors to code (default all);
        header=False leaves the other bytes out (the caller stores them); parsed: (layout, GGUF) when the
        caller has them; d: the file already in HBM (DeviceArray), else its tensors are uploaded"""
        return pack(self.compress_dict(data, tensors, header, parsed, d))

    def compress_parts(self, data, tensors=None, header=True, parsed=None, d=None):
        """compress() as pack_parts' list of buffers (the streams are not joined)"""
        return pack_parts(self.compress_dict(data, tensors, header, parsed, d))

    def compress_dict(self, data, tensors=None, header=True, parsed=None, d=None):
        st = self.stream
        host = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1)
        if parsed is None:
            g = gguf.GGUF(host)
            parsed = (layout_of(g, len(host)), g)
        layout, g = parsed
        with ThreadPoolExecutor(1) as ex:
            rest = ex.submit(self._header_c, host, g, layout) if header else None
            if tensors is not None:
                layout = dict(layout, t=[layout["t"][i] for i in tensors])
            ch = self._compress(host, layout, d)
            if rest is not None:
                ch["rest"] = rest.result()
        return ch

    @staticmethod
    def _header_c(host, g, layout):
        return header.header_c(host, g, layout, tokz=True)

    def _compress(self, host, layout, d):
        st = self.stream
        T = len(layout["t"])
        if not T:
            raise ValueError("Q8_0 codec: no tensors to code")
        for _, nbytes, rowlen, _ in layout["t"]:
            if rowlen % 32 or nbytes % 34 or (nbytes // 34) % (rowlen // 32):
                raise ValueError(f"Q8_0 codec: a tensor of {nbytes} bytes with rows of {rowlen}")
        n = sum(nb for _, nb, _, _ in layout["t"]) // 34
        if n >= 1 << 31:
            raise ValueError(f"Q8_0 codec: {n} blocks in one part")
        self._t = time.perf_counter()
        allb = dev.DeviceArray(n * 34, np.uint8)
        pos_b = 0
        for o, nb, _, _ in layout["t"]:
            if d is not None:
                check(lib().spa_memcpy_d2d(allb.ptr + pos_b, d.ptr + o, nb, st))
            else:
                check(lib().spa_memcpy_h2d(allb.ptr + pos_b, host[o:o + nb].ctypes.data, nb, st))
            pos_b += nb
        pos = dev.DeviceArray(n, np.uint8)
        check(lib().spa_q8_pos(allb.ptr, n, pos.ptr, st))
        groups, meta0 = _meta(layout, [0] * T, [0] * T)
        nrows_all = int(sum(int(m["nblocks"]) // int(m["nb_row"]) for m in meta0))
        meta_d = dev.DeviceArray.from_host(meta0.view(np.uint8), st)
        row_m = dev.DeviceArray(nrows_all, np.int32)
        check(lib().spa_q8_row_means(allb.ptr, meta_d.ptr, T, nrows_all, row_m.ptr, st))
        cfi, scls, off = self._column_side(allb, layout, meta0, row_m)
        self._lap("column statistics")
        perm, rankof, spread = colblock_side(cfi)
        bcf = block_factor_bins(cfi, layout)
        skip, dups = self._dedup(allb, layout, meta0)
        self._lap("duplicate rows")
        plans = self._plans(allb, layout, meta0, skip)
        self._lap("row planner")
        for p in plans:
            sl = skip[p["first"]:p["first"] + p["nrows"] * p["nbr"]]
            sl[...] = np.where(sl == 1, 1, 6).astype(np.uint8)

        G = len(groups)
        qbase = G * TA
        nalloc = qbase + G * TQ                     # the per-tensor sets stay empty: tables per group (no TSEL)
        meta = meta0.copy()
        meta["off"] = off
        meta["qset"] = meta["grp"]
        meta_d = dev.DeviceArray.from_host(meta.view(np.uint8), st)
        side_d = {k: dev.DeviceArray.from_host(v, st) for k, v in
                  (("skip", skip), ("bcf", bcf), ("spread", spread), ("rankof", rankof), ("scls", scls), ("cfi", cfi))}
        items = [(t, b0, min(HIST_ITEM, int(m["first"] + m["nblocks"]) - b0)) for t, m in enumerate(meta)
                 for b0 in range(int(m["first"]), int(m["first"] + m["nblocks"]), HIST_ITEM)]
        items_d = dev.DeviceArray.from_host(np.array(items, ITEM_DT).view(np.uint8), st)
        counts = dev.DeviceArray((nalloc, 256), np.uint32).zero(st)
        a_side = (side_d["bcf"].ptr, side_d["spread"].ptr, side_d["rankof"].ptr, side_d["scls"].ptr)
        check(lib().spa_q8_hist_a(allb.ptr, pos.ptr, side_d["skip"].ptr, meta_d.ptr, T, n, *a_side, counts.ptr, st))
        check(lib().spa_q8_hist_b(allb.ptr, pos.ptr, side_d["skip"].ptr, meta_d.ptr, T, n, items_d.ptr, len(items),
                                  side_d["cfi"].ptr, side_d["scls"].ptr, row_m.ptr, qbase, counts.ptr, st))
        tabs = _Tables(counts, nalloc, st)
        del counts
        self._lap("histograms + tables A/B")
        tab_args = (tabs.remap_d.ptr, tabs.freq_d.ptr, tabs.cum_d.ptr, tabs.rcp_d.ptr)
        streams = []
        nsa, nsb = (n + SEGA - 1) // SEGA, (n + SEGB - 1) // SEGB
        for what, nseg, seg in (("A", nsa, SEGA), ("B", nsb, SEGB)):
            cap = seg * 34 * 2 + 16
            out = dev.DeviceArray(nseg * cap, np.uint8)
            out_len = dev.DeviceArray(nseg, np.uint32)
            if what == "A":
                check(lib().spa_q8_enc_a(allb.ptr, pos.ptr, side_d["skip"].ptr, meta_d.ptr, T, n, *a_side, *tab_args,
                                         out.ptr, cap, out_len.ptr, st))
            else:
                check(lib().spa_q8_enc_b(allb.ptr, pos.ptr, side_d["skip"].ptr, meta_d.ptr, T, n, side_d["cfi"].ptr,
                                         side_d["scls"].ptr, row_m.ptr, qbase, *tab_args, out.ptr, cap, out_len.ptr, st))
            streams.append(_gather(out, cap, out_len, nseg, st, what))
            del out
            self._lap(f"phase {what}")
        extra = self._encode_extra(allb, pos, plans, meta, meta_d, side_d, cfi, row_m) if plans else {}
        self._lap("phase C")

        side = {"off": [int(v) for v in off], "qset": [int(v) for v in meta["qset"]],
                "dups": [[int(a) for a in r] for r in dups]}
        ch = {
            "layout": zstd.zstd_c(json.dumps(layout).encode()),
            "side": zstd.zstd_c(json.dumps(side).encode()),
            "cfi": zstd.zstd_c(cfi.tobytes()),
            "tables": tabs.stored(),
            "lens": zstd.zstd_c(streams[0][1].tobytes() + streams[1][1].tobytes()),
            "A": streams[0][0],
            "B": streams[1][0],
            "scls": zstd.zstd_c(scls.tobytes()),
        }
        ch.update(extra)
        return ch

    def _column_side(self, allb, layout, meta, row_m):
        """cfi / scls per column and the tensor offsets (gpu2.py:577-605)"""
        st = self.stream
        cfi_l, scls_l, off = [], [], []
        for i, (_, nbytes, rowlen, _) in enumerate(layout["t"]):
            f, nb, nbr, rb = (int(meta[i][k]) for k in ("first", "nblocks", "nb_row", "rowbase"))
            nrows = nb // nbr
            step = max(1, self.stat_elems // rowlen)
            nsl = (nrows + step - 1) // step
            rel = dev.DeviceArray(nb, np.float32)
            p1, p2 = dev.DeviceArray((nsl, rowlen), np.float64), dev.DeviceArray((nsl, rowlen), np.float64)
            check(lib().spa_q8_col_stats(allb.ptr, f, nbr, nrows, row_m.ptr + 4 * rb, rel.ptr, step, p1.ptr, p2.ptr, st))
            s1, s2 = _in_order(p1.to_host(stream=st)), _in_order(p2.to_host(stream=st))
            ms = (s2 / nrows).astype(np.float32)
            cf = _log2((np.sqrt(ms) + np.float32(1e-6)).astype(np.float64), st)
            ci = np.clip(np.rint(cf * 8), -32768, 32767).astype(np.int16)
            cfi_l.append(ci)
            bias = (s1 / nrows).astype(np.float32) / np.sqrt(ms + np.float32(1e-12))
            scls_l.append(np.clip(np.floor(bias * np.float32(16)) + np.float32(8), 0, 15).astype(np.uint8))
            off.append(int(float(np.sum(ci, dtype=np.int64)) / len(ci) * 128) - 32 * 128)
        return np.concatenate(cfi_l), np.concatenate(scls_l), off

    def _dedup(self, allb, layout, meta):
        """rows equal to an earlier row of their tensor: skip bit 0 and (tensor, row, source) triples
        (gpu2.py:693-716: random 64-bit word multipliers from RandomState(1234), np.unique, byte check)"""
        st = self.stream
        n = int(meta["first"][-1] + meta["nblocks"][-1])
        skip = np.zeros(n, np.uint8)
        dups = []
        rng = np.random.RandomState(1234)
        for i, (_, nbytes, rowlen, _) in enumerate(layout["t"]):
            nbr = rowlen // 32
            f, nb = int(meta["first"][i]), int(meta["nblocks"][i])
            nrows = nb // nbr
            if (nbr * 34) % 8:
                raise ValueError(f"Q8_0 codec: rows of {nbr * 34} bytes are not whole 64-bit words")
            mult = rng.randint(1, 2 ** 62, size=nbr * 34 // 8, dtype=np.int64).astype(np.uint64) | np.uint64(1)
            mult_d = dev.DeviceArray.from_host(mult, st)
            h_d = dev.DeviceArray(nrows, np.uint64)
            check(lib().spa_q8_row_hash(allb.ptr, f, nbr, nrows, mult_d.ptr, h_d.ptr, st))
            h = h_d.to_host(stream=st)
            _, first_idx, inv = np.unique(h, return_index=True, return_inverse=True)
            src = first_idx[inv.reshape(-1)]
            cand = np.nonzero(src != np.arange(len(h)))[0]
            if not len(cand):
                continue
            ra = dev.DeviceArray.from_host(cand.astype(np.int32), st)
            rb = dev.DeviceArray.from_host(src[cand].astype(np.int32), st)
            eq_d = dev.DeviceArray(len(cand), np.uint8)
            check(lib().spa_q8_rows_equal(allb.ptr, f, nbr, ra.ptr, rb.ptr, len(cand), eq_d.ptr, st))
            eq = eq_d.to_host(stream=st).astype(bool)
            for r, s in zip(cand[eq], src[cand][eq]):
                dups.append((i, int(r), int(s)))
                skip[f + r * nbr:f + (r + 1) * nbr] = 1
        return skip, np.array(dups, np.int64).reshape(-1, 3)

    def _plans(self, allb, layout, meta, skip):
        """row prediction plans of the token_embd tensors (gpu3.py:355-375)"""
        plans = []
        for i, (_, nbytes, rowlen, grp) in enumerate(layout["t"]):
            if grp not in PRED_TENSORS:
                continue
            f, nb, nbr = int(meta["first"][i]), int(meta["nblocks"][i]), int(meta["nb_row"][i])
            nrows = nb // nbr
            if nrows < 2 * WAVES or PRED_MEM * nb * 34 > PRED_MAX:
                continue
            valid = skip[f:f + nb].reshape(nrows, nbr)[:, 0] == 0
            p = self._plan_tensor(allb, f, nbr, nrows, valid)
            p.update(t=i, nrows=nrows, nbr=nbr, first=f)
            plans.append(p)
        return plans

    def _plan_tensor(self, allb, f, nbr, n, valid):
        """parents (n, 4), coefficients (n, 4), residual class per row, column means and residual
        column adjustments (gpu3.py:272-353 with M22's K 4, int8 coefficients, adaptive k, COLRES)"""
        st = self.stream
        C = nbr * 32
        wave = (np.arange(n) * WAVES) // n
        wstart = np.searchsorted(wave, wave, side="left").astype(np.int32)
        nvalid = float(int(valid.sum()))
        valid_d = dev.DeviceArray.from_host(valid.astype(np.uint8), st)
        W = dev.DeviceArray((n, C), np.float32)
        check(lib().spa_q8_row_matrix(allb.ptr, f, nbr, n, W.ptr, st))
        mu = (detmath.cols(W, mask=valid_d, stream=st).to_host(stream=st) / max(nvalid, 1.0)).astype(np.float32)
        col_w = detmath.cols(W, True, mask=valid_d, stream=st).to_host(stream=st)
        mu_d = dev.DeviceArray.from_host(mu, st)
        check(lib().spa_q8_center(W.ptr, mu_d.ptr, n, C, st))
        self._lap("planner: row matrix, column means")
        nrm = np.maximum(np.sqrt(detmath.rows(W, True, stream=st).to_host(stream=st)), 1e-12)
        nrm_d = dev.DeviceArray.from_host(nrm, st)
        Wq = dev.DeviceArray((n, C), np.int8)
        check(lib().spa_q8_norm_i8(W.ptr, nrm_d.ptr, valid_d.ptr, n, C, Wq.ptr, st))
        cand = dev.DeviceArray((n, KPAR), np.int32)
        wstart_d = dev.DeviceArray.from_host(wstart, st)
        check(lib().spa_q8_neighbours(Wq.ptr, n, C, wstart_d.ptr, valid_d.ptr, cand.ptr, st))
        self._lap("planner: norms, int8 rows, neighbours")
        del Wq
        frac_d, kuse_d = dev.DeviceArray(n, np.float32), dev.DeviceArray(n, np.int32)
        coefs_d = dev.DeviceArray((n, KPAR), np.float32)
        check(lib().spa_q8_fit_rows(W.ptr, cand.ptr, n, C, frac_d.ptr, kuse_d.ptr, coefs_d.ptr, st))
        self._lap("planner: least squares")
        nch = (n + LS_CHUNK - 1) // LS_CHUNK
        part = dev.DeviceArray((nch, C), np.float64)
        check(lib().spa_q8_col_res(W.ptr, cand.ptr, coefs_d.ptr, kuse_d.ptr, valid_d.ptr, n, C, LS_CHUNK, part.ptr, st))
        col_res = _in_order(part.to_host(stream=st))
        self._lap("planner: residual columns")
        par, kuse = cand.to_host(stream=st), kuse_d.to_host(stream=st)
        coefs, frac = coefs_d.to_host(stream=st), frac_d.to_host(stream=st)
        valid_par = (np.arange(KPAR)[None, :] < kuse[:, None]) & valid[:, None]
        par = np.where(valid_par, par, -1).astype(np.int32)
        coefs = np.where(valid_par, coefs, 0).astype(np.float32)
        frac = np.where(kuse > 0, frac, np.float32(1.0)).astype(np.float32)
        gfrac = _total(col_res) / max(_total(col_w), 1e-30)
        ratio = np.maximum(col_res / np.maximum(col_w, 1e-30), 1e-6)
        # a NaN (from fp16 infinity / NaN scales) becomes 0, the device float-to-int conversion's value
        # for NaN that the reference's planner stores; numpy leaves that cast undefined
        cadj = _int8_nan0(np.clip(np.rint(4 * _log2(ratio, st)), -60, 0))
        q = frac / np.float32(max(gfrac, 1e-6))
        fbin = _int8_nan0(np.clip(np.rint(_log2(q.astype(np.float64), st) * 4), -40, 20))
        return dict(par=par, coefs=coefs, fbin=fbin, mu=mu, cadj=cadj)

    def _encode_extra(self, allb, pos, plans, meta, meta_d, side_d, cfi, row_m):
        """phase C: predictions, histograms, tables, segments (gpu3.py:377-418)"""
        st = self.stream
        rbase = np.cumsum([0] + [p["nrows"] for p in plans])[:-1].astype(np.int64)
        pbase = np.cumsum([0] + [p["nrows"] * p["nbr"] * 32 for p in plans])[:-1].astype(np.int64)
        mubase = np.cumsum([0] + [p["nbr"] * 32 for p in plans])[:-1].astype(np.int64)
        total = int(pbase[-1] + plans[-1]["nrows"] * plans[-1]["nbr"] * 32)
        pint = dev.DeviceArray(total, np.int8)
        par_all = np.concatenate([p["par"].ravel() for p in plans]).astype(np.int32)
        coef_all = np.concatenate([p["coefs"].ravel() for p in plans]).astype(np.float32)
        mu_all = np.concatenate([p["mu"] for p in plans]).astype(np.float32)
        fbin_all = np.concatenate([p["fbin"] for p in plans]).astype(np.int8)
        par_d, coef_d, mu_d = (dev.DeviceArray.from_host(a, st) for a in (par_all, coef_all, mu_all))
        for slot, p in enumerate(plans):
            ro, mo = int(rbase[slot]), int(mubase[slot])
            check(lib().spa_q8_predict(allb.ptr, p["first"], p["nbr"], p["nrows"], par_d.ptr + 4 * KPAR * ro,
                                       coef_d.ptr + 4 * KPAR * ro, mu_d.ptr + 4 * mo, pint.ptr + int(pbase[slot]), st))
        prk, pinv, rctx = dev.DeviceArray(total, np.int8), dev.DeviceArray(total, np.int8), dev.DeviceArray(total // 32, np.int8)
        check(lib().spa_q8_ranks(pint.ptr, total // 32, prk.ptr, pinv.ptr, rctx.ptr, st))
        segs, _ = segments(plans, WAVES, RPT)
        nseg = len(segs)
        slots = np.zeros(len(plans), SLOT_DT)
        for slot, p in enumerate(plans):
            slots[slot] = (rbase[slot], pbase[slot], p["first"], p["nbr"], mubase[slot], 0)
        cfi_c = cfi.copy()
        for p in plans:
            cb = int(meta["colbase"][p["t"]])
            C = p["nbr"] * 32
            cfi_c[cb:cb + C] = (cfi_c[cb:cb + C].astype(np.int32) + p["cadj"].astype(np.int32)).astype(np.int16)
        segs_d, slots_d, cfi_d, fbin_d = (dev.DeviceArray.from_host(a, st) for a in
                                          (segs.view(np.uint8), slots.view(np.uint8), cfi_c, fbin_all))
        c_args = (side_d["skip"].ptr, meta_d.ptr, segs_d.ptr, nseg, slots_d.ptr, cfi_d.ptr, row_m.ptr, fbin_d.ptr, pint.ptr,
                  prk.ptr, pinv.ptr, rctx.ptr)
        ntab = len(plans) * TPC
        counts = dev.DeviceArray((ntab, 256), np.uint32).zero(st)
        check(lib().spa_q8_hist_c(allb.ptr, pos.ptr, *c_args, counts.ptr, st))
        tabs = _Tables(counts, ntab, st)
        cap = max(RPT * p["nbr"] * 34 * 2 + 64 for p in plans)
        out = dev.DeviceArray(nseg * cap, np.uint8)
        out_len = dev.DeviceArray(nseg, np.uint32)
        check(lib().spa_q8_enc_c(allb.ptr, pos.ptr, *c_args, tabs.remap_d.ptr, tabs.freq_d.ptr, tabs.cum_d.ptr,
                                 tabs.rcp_d.ptr, out.ptr, cap, out_len.ptr, st))
        stream, lens = _gather(out, cap, out_len, nseg, st, "C")
        side = {"tensors": [p["t"] for p in plans], "waves": WAVES, "K": KPAR, "rpt": RPT}
        return {
            "C": stream,
            "Clens": zstd.zstd_c(lens.tobytes()),
            "Ctables": tabs.stored(),
            "Cside": zstd.zstd_c(json.dumps(side).encode()),
            "Cpar": zstd.zstd_c(par_all.tobytes(), 19),
            "Ccoef": zstd.zstd_c(_int8_nan0(np.rint(coef_all * np.float32(64))).tobytes(), 19),
            "Cfbin": zstd.zstd_c(fbin_all.tobytes(), 19),
            "Cmu": zstd.zstd_c(mu_all.tobytes()),
            "Ccadj": zstd.zstd_c(np.concatenate([p["cadj"] for p in plans]).astype(np.int8).tobytes(), 19),
        }

    # ---------------------------------------------------------- decoder
    def decompress(self, buf, out=None):
        """-> the file (numpy uint8) with the coded tensors (and, if the chunk has it, the other bytes);
        with `out` (a host buffer of the file's size) only the tensors (and rest) are written into it"""
        allb, layout, meta, rest = self._decode(buf)
        st = self.stream
        if out is None:
            out = np.zeros(layout["size"], np.uint8)
        for (o, nbytes, _, _), f in zip(layout["t"], meta["first"]):
            check(lib().spa_memcpy_d2h(out[o:o + nbytes].ctypes.data, allb.ptr + int(f) * 34, nbytes, st))
        dev.synchronize(st)
        if rest is not None:
            header.fill_rest(out, rest.result(), layout)
        return out

    def decompress_dev(self, buf, out_dev):
        """the coded tensors written into the device buffer out_dev (the file's size); -> the "rest"
        bytes (rest_of's) if the chunk has them, else None"""
        allb, layout, meta, rest = self._decode(buf)
        st = self.stream
        if out_dev.nbytes < layout["size"]:
            raise ValueError("Q8_0 codec: output buffer smaller than the file")
        for (o, nbytes, _, _), f in zip(layout["t"], meta["first"]):
            check(lib().spa_memcpy_d2d(out_dev.ptr + o, allb.ptr + int(f) * 34, nbytes, st))
        dev.synchronize(st)
        return rest.result() if rest is not None else None

    def _decode(self, buf):
        st = self.stream
        self._t = time.perf_counter()
        ch = unpack(memoryview(buf) if not isinstance(buf, memoryview) else buf)
        pool = ThreadPoolExecutor(1)
        rest = pool.submit(header.header_d, bytes(ch["rest"])) if "rest" in ch else None
        pool.shutdown(wait=False)
        layout = json.loads(zstd.decompress(ch["layout"]))
        side = json.loads(zstd.decompress(ch["side"]))
        T = len(layout["t"])
        groups, meta = _meta(layout, side["off"], side["qset"])
        G = len(groups)
        qbase = G * TA
        ntab = qbase + (G + T) * TQ
        n = int(meta["first"][-1] + meta["nblocks"][-1])
        nsa, nsb = (n + SEGA - 1) // SEGA, (n + SEGB - 1) // SEGB
        lens = np.frombuffer(zstd.decompress(ch["lens"]), np.uint16).astype(np.uint64)
        if len(lens) != nsa + nsb:
            raise ValueError(f"Q8_0 codec: {len(lens)} segment lengths for {nsa} + {nsb} segments")
        cfi = np.frombuffer(zstd.decompress(ch["cfi"]), np.int16).copy()
        scls = np.frombuffer(zstd.decompress(ch["scls"]), np.uint8).copy()
        ncol = sum(rl for _, _, rl, _ in layout["t"])
        if len(cfi) != ncol or len(scls) != ncol:
            raise ValueError("Q8_0 codec: column side information does not match the layout")
        remap_d, lut = _decoder_tables(ch["tables"], ntab, st)
        perm, rankof, spread = colblock_side(cfi)
        bcf = block_factor_bins(cfi, layout)
        skip = np.zeros(n, np.uint8)
        dups = np.array(side["dups"], np.int64).reshape(-1, 3)
        for i, r, _ in dups:
            nbr, f = int(meta["nb_row"][i]), int(meta["first"][i])
            skip[f + r * nbr:f + (r + 1) * nbr] = 1
        cside = json.loads(zstd.decompress(ch["Cside"])) if "Cside" in ch else None
        if cside is not None:
            for t in cside["tensors"]:
                f, nb = int(meta["first"][t]), int(meta["nblocks"][t])
                sl = skip[f:f + nb]
                sl[...] = np.where(sl == 1, 1, 6).astype(np.uint8)
        meta_d = dev.DeviceArray.from_host(meta.view(np.uint8), st)
        side_d = {k: dev.DeviceArray.from_host(v, st) for k, v in
                  (("skip", skip), ("bcf", bcf), ("spread", spread), ("perm", perm), ("scls", scls), ("cfi", cfi))}
        allb = dev.DeviceArray(n * 34, np.uint8).zero(st)
        pos = dev.DeviceArray(n, np.uint8).zero(st)
        tab_args = (remap_d.ptr, lut.ptr)
        for what, ns, lo in (("A", nsa, 0), ("B", nsb, nsa)):
            ln = lens[lo:lo + ns]
            offs = np.zeros(ns, np.uint64)
            offs[1:] = np.cumsum(ln)[:-1]
            s = np.frombuffer(ch[what], np.uint8)
            if int(ln.sum()) > len(s):
                raise ValueError(f"Q8_0 codec: phase {what} stream shorter than its segment lengths")
            s_d = dev.DeviceArray.from_host(s if len(s) else np.zeros(1, np.uint8), st)
            offs_d = dev.DeviceArray.from_host(offs, st)
            if what == "A":
                check(lib().spa_q8_dec_a(s_d.ptr, len(s), offs_d.ptr, side_d["skip"].ptr, meta_d.ptr, T, n,
                                         side_d["bcf"].ptr, side_d["spread"].ptr, side_d["perm"].ptr, side_d["scls"].ptr,
                                         *tab_args, allb.ptr, pos.ptr, st))
                nrows_all = int(sum(int(m["nblocks"]) // int(m["nb_row"]) for m in meta))
                row_m = dev.DeviceArray(nrows_all, np.int32)
                check(lib().spa_q8_row_means(allb.ptr, meta_d.ptr, T, nrows_all, row_m.ptr, st))
            else:
                check(lib().spa_q8_dec_b(s_d.ptr, len(s), offs_d.ptr, side_d["skip"].ptr, meta_d.ptr, T, n,
                                         side_d["cfi"].ptr, side_d["scls"].ptr, row_m.ptr, qbase, *tab_args, allb.ptr,
                                         pos.ptr, st))
            dev.synchronize(st)
            self._lap(f"decode phase {what}")
        if cside is not None:
            self._decode_extra(ch, cside, allb, pos, meta, meta_d, side_d, cfi, row_m)
            self._lap("decode phase C")
        if len(dups):
            for i, r, s_ in dups:
                nbr, f = int(meta["nb_row"][i]), int(meta["first"][i])
                check(lib().spa_memcpy_d2d(allb.ptr + (f + int(r) * nbr) * 34, allb.ptr + (f + int(s_) * nbr) * 34,
                                           nbr * 34, st))
        return allb, layout, meta, rest

    def _decode_extra(self, ch, cside, allb, pos, meta, meta_d, side_d, cfi, row_m):
        """phase C wave by wave: the wave's predictions, then its segments (gpu3.py:444-511)"""
        st = self.stream
        K, waves, rpt = cside["K"], cside["waves"], cside["rpt"]
        if K != KPAR or waves <= 0 or rpt <= 0:
            raise ValueError(f"Q8_0 codec: phase C with {K} parents, {waves} waves, {rpt} rows per segment")
        par_all = np.frombuffer(zstd.decompress(ch["Cpar"]), np.int32)
        coef_all = np.frombuffer(zstd.decompress(ch["Ccoef"]), np.int8).astype(np.float32) / np.float32(64)
        fbin_all = np.frombuffer(zstd.decompress(ch["Cfbin"]), np.int8)
        mu_all = np.frombuffer(zstd.decompress(ch["Cmu"]), np.float32)
        cadj_all = np.frombuffer(zstd.decompress(ch["Ccadj"]), np.int8)
        plans, ro, co = [], 0, 0
        for t in cside["tensors"]:
            nbr = int(meta["nb_row"][t])
            nrows = int(meta["nblocks"][t]) // nbr
            plans.append(dict(t=t, nrows=nrows, nbr=nbr, first=int(meta["first"][t]), rbase=ro, mubase=co,
                              cadj=cadj_all[co:co + nbr * 32]))
            ro += nrows
            co += nbr * 32
        if len(par_all) != ro * K or len(coef_all) != ro * K or len(fbin_all) != ro or len(mu_all) != co \
                or len(cadj_all) != co:
            raise ValueError("Q8_0 codec: phase C side information does not match its tensors")
        if len(par_all) and (par_all.max() >= max(p["nrows"] for p in plans)):
            raise ValueError("Q8_0 codec: a parent row outside its tensor")
        pbase = np.cumsum([0] + [p["nrows"] * p["nbr"] * 32 for p in plans])[:-1].astype(np.int64)
        total = int(pbase[-1] + plans[-1]["nrows"] * plans[-1]["nbr"] * 32)
        pint = dev.DeviceArray(total, np.int8).zero(st)
        prk, pinv, rctx = dev.DeviceArray(total, np.int8), dev.DeviceArray(total, np.int8), dev.DeviceArray(total // 32, np.int8)
        segs, wave_start = segments(plans, waves, rpt)
        nseg = len(segs)
        slots = np.zeros(len(plans), SLOT_DT)
        for slot, p in enumerate(plans):
            slots[slot] = (p["rbase"], pbase[slot], p["first"], p["nbr"], p["mubase"], 0)
        cfi_c = cfi.copy()
        for p in plans:
            cb = int(meta["colbase"][p["t"]])
            C = p["nbr"] * 32
            cfi_c[cb:cb + C] = (cfi_c[cb:cb + C].astype(np.int32) + p["cadj"].astype(np.int32)).astype(np.int16)
        remap_d, lut = _decoder_tables(ch["Ctables"], len(plans) * TPC, st)
        lens = np.frombuffer(zstd.decompress(ch["Clens"]), np.uint16).astype(np.uint64)
        if len(lens) != nseg:
            raise ValueError(f"Q8_0 codec: {len(lens)} phase C lengths for {nseg} segments")
        offs = np.zeros(nseg, np.uint64)
        offs[1:] = np.cumsum(lens)[:-1]
        s = np.frombuffer(ch["C"], np.uint8)
        if int(lens.sum()) > len(s):
            raise ValueError("Q8_0 codec: phase C stream shorter than its segment lengths")
        s_d = dev.DeviceArray.from_host(s if len(s) else np.zeros(1, np.uint8), st)
        offs_d = dev.DeviceArray.from_host(offs, st)
        se = [waves_of(p["nrows"], waves) for p in plans]
        es, er, ent_start = [], [], [0]
        for w in range(waves):
            k = 0
            for slot in range(len(plans)):
                a, b = int(se[slot][0][w]), int(se[slot][1][w])
                es.append(np.full(b - a, slot, np.int32))
                er.append(np.arange(a, b, dtype=np.int32))
                k += b - a
            ent_start.append(ent_start[-1] + k)
        ent_slot_d = dev.DeviceArray.from_host(np.concatenate(es), st)
        ent_row_d = dev.DeviceArray.from_host(np.concatenate(er), st)
        cmax = max(p["nbr"] for p in plans) * 32
        segs_d, slots_d, cfi_d, fbin_d = (dev.DeviceArray.from_host(a, st) for a in
                                          (segs.view(np.uint8), slots.view(np.uint8), cfi_c, fbin_all))
        par_d, coef_d, mu_d = (dev.DeviceArray.from_host(a, st) for a in (par_all, coef_all, mu_all))
        for w in range(waves):
            e0, e1 = ent_start[w], ent_start[w + 1]
            check(lib().spa_q8_predict_multi(allb.ptr, ent_slot_d.ptr + 4 * e0, ent_row_d.ptr + 4 * e0, e1 - e0, cmax,
                                             slots_d.ptr, par_d.ptr, coef_d.ptr, mu_d.ptr, pint.ptr, st))
            for slot, p in enumerate(plans):           # the wave's rows of each tensor: one run of pint
                a, b = int(se[slot][0][w]), int(se[slot][1][w])
                if b > a:
                    q0 = int(pbase[slot]) + a * p["nbr"] * 32
                    check(lib().spa_q8_ranks(pint.ptr + q0, (b - a) * p["nbr"], prk.ptr + q0, pinv.ptr + q0,
                                             rctx.ptr + q0 // 32, st))
            check(lib().spa_q8_dec_c(s_d.ptr, len(s), offs_d.ptr, wave_start[w], wave_start[w + 1], side_d["skip"].ptr,
                                     meta_d.ptr, segs_d.ptr, nseg, slots_d.ptr, cfi_d.ptr, row_m.ptr, fbin_d.ptr, pint.ptr,
                                     prk.ptr, pinv.ptr, rctx.ptr, remap_d.ptr, lut.ptr, allb.ptr, pos.ptr, st))
        dev.synchronize(st)


class Q8Parts:
    """M22 over a file in parts of whole Q8_0 tensors of at most `budget` bytes each (a tensor larger
    than the budget is a part of its own); the bytes around the tensors are stored once (gpu3.py:590-643).
    The default budget is a fixed size, so the archive does not depend on the device."""
    PART = 1 << 30

    def __init__(self, budget=None, stream=None, timing=False):
        self.c = M22(stream, timing=timing)
        self.budget = budget or self.PART
        self.parts = 0

    def groups(self, layout):
        groups, cur, size = [], [], 0
        for i, (_, nb, _, _) in enumerate(layout["t"]):
            if cur and size + nb > self.budget:
                groups.append(cur)
                cur, size = [], 0
            cur.append(i)
            size += nb
        if cur:
            groups.append(cur)
        return groups

    def compress(self, data, with_rest=True, g=None, d=None):
        """with_rest=False: only the Q8_0 tensors (the caller stores the other bytes); d: the file in HBM"""
        host = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1)
        g = g or gguf.GGUF(host)
        layout = layout_of(g, len(host))
        with ThreadPoolExecutor(1) as ex:
            hdr = ex.submit(M22._header_c, host, g, layout) if with_rest else None
            groups = self.groups(layout)
            ch = {"layout": zstd.zstd_c(json.dumps(layout).encode())}
            for k, idx in enumerate(groups):
                ch[f"p{k}"] = self.c.compress_parts(host, tensors=idx, header=False, parsed=(layout, g), d=d)
            if hdr is not None:
                ch["rest"] = hdr.result()
        self.parts = len(groups)
        return pack(ch)

    def decompress(self, buf, out=None):
        """-> the file (numpy uint8); with `out`, the Q8_0 tensors (and rest) are written into it"""
        ch = unpack(memoryview(buf) if not isinstance(buf, memoryview) else buf)
        layout = json.loads(zstd.decompress(ch["layout"]))
        if out is None:
            out = np.zeros(layout["size"], np.uint8)
        k = 0
        while f"p{k}" in ch:
            self.c.decompress(ch[f"p{k}"], out=out)
            k += 1
        if "rest" in ch:
            header.fill_rest(out, header.header_d(bytes(ch["rest"])), layout)
        return out

    def decompress_dev(self, buf, out_dev):
        """the Q8_0 tensors into the device buffer out_dev; -> the layout and rest_of's bytes (or None)"""
        ch = unpack(memoryview(buf) if not isinstance(buf, memoryview) else buf)
        layout = json.loads(zstd.decompress(ch["layout"]))
        k = 0
        while f"p{k}" in ch:
            self.c.decompress_dev(ch[f"p{k}"], out_dev)
            k += 1
        return layout, (header.header_d(bytes(ch["rest"])) if "rest" in ch else None)
