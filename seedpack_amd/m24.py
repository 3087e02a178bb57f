"""M24, the reference's first-generation GPU BF16 codec (seedpack/gpu_bf16.py M24BF16GPU, the base
codec of archive method m28) on the MI355X.

Every 2-D BF16 tensor is coded weight by weight with three symbols (exponent, mantissa, sign) in
contexts from integer side information: the row and column RMS in quarter octaves (rfi, cfi, from
detmath's sums, log2 and exp2) and a per-column sign-bias class (scl); 160 tables per tensor, one
rANS state per segment of 16384 weights (PB 12). The chunk is pack({layout, side, tables, lens,
stream, rest}); "rest" is the file's other bytes in the header coder's P or X form (header.py).
"""
import json
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import detmath
from . import device as dev
from . import gguf, header, zstd
from ._lib import check, lib
from .framing import pack, unpack
from .r2 import cum_of, load_tables, normalize, store_tables

SEG = 16384            # BF16 weights per segment (gpu_bf16.py:27)
TPT = 160              # tables per tensor: 128 exponent + 16 mantissa + 16 sign (gpu_bf16.py:29)
PB = 12
BF16 = 30
TB_DT = np.dtype([("off", "<i8"), ("rowlen", "<i4"), ("rowbase", "<i4"), ("colbase", "<i4"), ("tab", "<i4")])
SG_DT = np.dtype([("t", "<i4"), ("n", "<i4"), ("i0", "<i8")])


def layout_of(g, size):
    """the BF16 matrices by offset: {"size", "t": [[offset, bytes, row length, "bf16"]]} (gpu_bf16.py:328-330)"""
    ts = sorted((t for t in g.tensors if t.type == BF16 and len(t.shape) == 2), key=lambda t: t.offset)
    return {"size": size, "t": [[t.offset, t.nbytes, t.shape[0], "bf16"] for t in ts]}


def tables(layout):
    """TB / SG descriptors: each tensor's row / column bases and tables, its segments (gpu_bf16.py:332-342)"""
    tb = np.zeros(len(layout["t"]), TB_DT)
    segs = []
    rowbase = colbase = 0
    for i, (off, nbytes, rowlen, _) in enumerate(layout["t"]):
        n = nbytes // 2
        tb[i] = (off, rowlen, rowbase, colbase, i * TPT)
        segs += [(i, min(SEG, n - i0), i0) for i0 in range(0, n, SEG)]
        rowbase += n // rowlen
        colbase += rowlen
    return tb, np.array(segs, SG_DT) if segs else np.zeros(0, SG_DT)


def _log2(x, st):
    return detmath.log2(np.ascontiguousarray(x, np.float64), st).to_host(stream=st)


def _exp2(x, st):
    return detmath.exp2(np.ascontiguousarray(x, np.float64), st).to_host(stream=st)


def _i16(v):
    return np.clip(np.rint(v), -32768, 32767).astype(np.int16)


class M24BF16:
    name = "M24 BF16 context rANS on GPU (port of M22)"            # gpu_bf16.py:324

    def __init__(self, stream=None):
        self.stream = stream

    def side_info(self, d, layout):
        """rfi (per row), cfi and scl (per column) of every tensor of the device-resident file d
        (gpu_bf16.py:352-371: detmath's row sums of squares, log2 / exp2, the row-normalised column sums)"""
        st = self.stream
        rfi_l, cfi_l, scl_l = [], [], []
        for off, nbytes, rowlen, _ in layout["t"]:
            nr = nbytes // 2 // rowlen
            u = d.view(off, (nr, rowlen), np.uint16)
            rows = dev.DeviceArray(nr, np.float64)
            check(lib().spa_dm_rows(u.ptr, 2, nr, rowlen, 1, rows.ptr, st))
            rf = _log2(np.sqrt(rows.to_host(stream=st) / rowlen) + 1e-30, st)
            rfa = dev.DeviceArray.from_host(_exp2(rf, st).astype(np.float32), st)
            s1, s2 = dev.DeviceArray(rowlen, np.float64), dev.DeviceArray(rowlen, np.float64)
            check(lib().spa_m24_cols(u.ptr, rfa.ptr, nr, rowlen, s1.ptr, s2.ptr, st))
            s1, s2 = s1.to_host(stream=st), s2.to_host(stream=st)
            cf = _log2(np.sqrt(s2 / nr) + 1e-30, st)
            rfi, cfi = _i16(rf * 4), _i16(cf * 4)
            bias = (s1 / nr) / _exp2(cfi.astype(np.float64) / 4, st)
            rfi_l.append(rfi)
            cfi_l.append(cfi)
            scl_l.append(np.clip(np.floor(bias * 16) + 8, 0, 15).astype(np.int8))
        cat = (lambda a, t: np.concatenate(a) if a else np.zeros(0, t))
        return cat(rfi_l, np.int16), cat(cfi_l, np.int16), cat(scl_l, np.int8)

    def compress_dev(self, data, d=None, g=None):
        """the chunk's parts for the file `data` (bytes-like, host); d: the file already in HBM"""
        st = self.stream
        host = np.frombuffer(data, np.uint8)
        g = g or gguf.GGUF(host)
        layout = layout_of(g, len(host))
        with ThreadPoolExecutor(1) as ex:
            rest = ex.submit(header.header_c, host, g, layout)
            if d is None:
                d = dev.DeviceArray.from_host(host, st)
            rfi, cfi, scl = self.side_info(d, layout)
            stream, lens, tabs = self.encode(d, layout, rfi, cfi, scl)
            return {"layout": zstd.zstd_c(json.dumps(layout).encode()),
                    "side": zstd.zstd_c(rfi.tobytes() + cfi.tobytes() + scl.tobytes(), 19),
                    "tables": tabs, "lens": zstd.zstd_c(lens.astype(np.uint32).tobytes()), "stream": stream,
                    "rest": rest.result()}

    def encode(self, d, layout, rfi, cfi, scl):
        """histogram, tables, per-segment rANS, gather -> (stream bytes, segment lengths, tables chunk)"""
        st = self.stream
        tb, sg = tables(layout)
        nseg, ntab = len(sg), len(tb) * TPT
        if not nseg:
            return b"", np.zeros(0, np.uint32), store_tables(np.zeros((0, 256), np.uint16), [])
        tb_d = dev.DeviceArray.from_host(tb.view(np.uint8), st)
        sg_d = dev.DeviceArray.from_host(sg.view(np.uint8), st)
        side = [dev.DeviceArray.from_host(a, st) for a in (rfi, cfi, scl)]
        counts = dev.DeviceArray((ntab, 256), np.uint32).zero(st)
        check(lib().spa_m24_hist(d.ptr, tb_d.ptr, sg_d.ptr, nseg, *(a.ptr for a in side), counts.ptr, st))
        freq, used = normalize(counts.to_host(stream=st), 1 << PB)
        remap = np.full(ntab, -1, np.int32)
        remap[used] = np.arange(len(used), dtype=np.int32)
        freq_d, cum_d, remap_d = (dev.DeviceArray.from_host(a, st) for a in (freq, cum_of(freq), remap))
        rcp = dev.DeviceArray(max(1, lib().spa_m24_rcp_bytes(ntab)), np.uint8)
        cap = SEG * 2 + 1024
        out = dev.DeviceArray(nseg * cap, np.uint8)
        out_len = dev.DeviceArray(nseg, np.uint32)
        check(lib().spa_m24_encode(d.ptr, tb_d.ptr, sg_d.ptr, nseg, *(a.ptr for a in side), remap_d.ptr, ntab,
                                   freq_d.ptr, cum_d.ptr, rcp.ptr, out.ptr, cap, out_len.ptr, st))
        lens = out_len.to_host(stream=st)
        if (lens == 0xFFFFFFFF).any():
            raise RuntimeError("M24: rANS segment overflow")
        offs = np.zeros(nseg + 1, np.uint64)
        offs[1:] = np.cumsum(lens.astype(np.uint64))
        dst = dev.DeviceArray(max(1, int(offs[-1])), np.uint8)
        offs_d = dev.DeviceArray.from_host(offs, st)
        check(lib().spa_qr_gather(out.ptr, cap, out_len.ptr, offs_d.ptr, nseg, dst.ptr, st))
        return dst.to_host(stream=st)[:int(offs[-1])].tobytes(), lens, store_tables(freq, used)

    def decompress_dev(self, ch, into=None, rest=None):
        """the chunk's parts -> the whole file as a DeviceArray (`into`, of the file's size, if given;
        rest: the "rest" part already decoded, if it is)"""
        st = self.stream
        layout = json.loads(zstd.decompress(ch["layout"]))
        with ThreadPoolExecutor(1) as ex:
            rest = ex.submit(header.header_d, bytes(ch["rest"])) if rest is None else ex.submit(bytes, rest)
            tb, sg = tables(layout)
            nrow = int(sum(nb // 2 // rl for _, nb, rl, _ in layout["t"]))
            ncol = int(sum(rl for _, _, rl, _ in layout["t"]))
            side = zstd.decompress(ch["side"])
            rfi = np.frombuffer(side, np.int16, nrow, 0)
            cfi = np.frombuffer(side, np.int16, ncol, 2 * nrow)
            scl = np.frombuffer(side, np.int8, ncol, 2 * nrow + 2 * ncol)
            if into is not None and into.nbytes != layout["size"]:
                raise ValueError(f"a file of {layout['size']} bytes for a place of {into.nbytes}")
            out = into if into is not None else dev.DeviceArray(max(1, layout["size"]), np.uint8)
            nseg = len(sg)
            if nseg:
                freq, used = load_tables(ch["tables"])
                ntab = len(tb) * TPT
                remap = np.full(ntab, -1, np.int32)
                remap[np.asarray(used, np.int64)] = np.arange(len(used), dtype=np.int32)
                freq = np.ascontiguousarray(freq, np.uint16)
                cum = cum_of(freq)
                freq_d, cum_d, remap_d = (dev.DeviceArray.from_host(a, st) for a in (freq, cum, remap))
                lut = dev.DeviceArray((max(1, len(freq)), 1 << PB), np.uint8)
                check(lib().spa_rans_build_lut(cum_d.ptr, len(freq), lut.ptr, st))
                lens = np.frombuffer(zstd.decompress(ch["lens"]), np.uint32)
                s = np.frombuffer(bytes(ch["stream"]), np.uint8)
                if len(lens) != nseg or int(lens.astype(np.uint64).sum()) > len(s):
                    raise ValueError(f"M24: {len(lens)} segment lengths for {nseg} segments and a {len(s)}-byte stream")
                offs = np.zeros(nseg, np.uint64)
                offs[1:] = np.cumsum(lens.astype(np.uint64))[:-1]
                s_d = dev.DeviceArray.from_host(s if len(s) else np.zeros(1, np.uint8), st)
                side_d = [dev.DeviceArray.from_host(np.ascontiguousarray(a), st) for a in (rfi, cfi, scl)]
                tb_d = dev.DeviceArray.from_host(tb.view(np.uint8), st)
                sg_d = dev.DeviceArray.from_host(sg.view(np.uint8), st)
                offs_d = dev.DeviceArray.from_host(offs, st)
                check(lib().spa_m24_decode(s_d.ptr, len(s), offs_d.ptr, out.ptr, tb_d.ptr, sg_d.ptr, nseg,
                                           *(a.ptr for a in side_d), remap_d.ptr, freq_d.ptr, cum_d.ptr, lut.ptr, st))
            # the bytes around the tensors
            full = np.zeros(layout["size"], np.uint8)
            header.fill_rest(full, rest.result(), layout)
            pos = 0
            for off, nbytes, _, _ in layout["t"] + [[layout["size"], 0, 1, "bf16"]]:
                if off > pos:
                    check(lib().spa_memcpy_h2d(out.ptr + pos, full[pos:off].ctypes.data, off - pos, st))
                pos = off + nbytes
            dev.synchronize(st)
        return out

    def compress(self, data):
        return pack(self.compress_dev(data))

    def decompress(self, buf):
        d = self.decompress_dev(unpack(memoryview(buf)))
        return d.to_host(stream=self.stream)[:d.nbytes]
