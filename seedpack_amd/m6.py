"""Method M6 (the reference's seedpack/gpu_codec.py): a Q8_0 GGUF coded by segmented context rANS, one
of codecs_gguf's single-file methods (no archive method uses it).

The file splits into its Q8_0 tensors (by offset) and every other byte (the header, metadata, other
tensors, padding: "rest", xz). The tensors' blocks are coded back to back in segments of 512 blocks,
one rANS state per segment, the symbols of a block with contexts from its own bytes and two per-tensor
statistics (csrc/m6.hip states the model): the median of its scale bits, and its input columns in 16
classes by the quantiles of their RMS. Statistics, histogram, coding and decoding run on the device;
the host forms the medians from the device histogram, the column classes from the device RMS with
numpy's quantile and searchsorted (the reference's own calls), and normalises the tables.

Chunk (gpu_codec.py:270-281): pack({"layout", "rest", "meta", "colmap", "used", "tables", "seglen",
"stream"}): zstd JSON of the layout {"size", "t": [[offset, bytes, row length, group], ...]}; xz of the
rest; zstd JSON {"groups": sorted group names, "med": per tensor}; zstd of the column classes; zstd of
the used table ids (u32); the used tables (tables_c, zstd level 22); zstd of the segment lengths (u16);
the segments' bytes back to back.
"""
import json
import lzma
import struct
import subprocess
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import device as dev
from . import gguf, zstd
from ._lib import check, lib
from .framing import pack, unpack
from .q8 import layout_of

NAME = "M6 GPU segmented context rANS (CUDA)"     # gpu_codec.py:215
SEG, PB, N_COL, N_SB = 512, 12, 16, 16
TPG = 256 + 256 + 1 + 1 + N_SB * N_COL           # tables per tensor group (gpu_codec.py:31)
META = np.dtype([("first", "<i4"), ("nblocks", "<i4"), ("nb_row", "<i4"), ("grp", "<i4"), ("colbase", "<i4"),
                 ("med", "<i4")])
CAP = SEG * 34 * 2 + 16                          # bytes of a segment's coding slot
XZ_SMALL = 8 << 20


# ---------------------------------------------------------------- the generic codecs of codecs_gguf
def xz_c(data):
    """xz of the reference's codecs (codecs_gguf.py:86-89): lzma preset 9e below 8 MiB, else the xz tool
    with -9e on all cores"""
    data = bytes(data)
    if len(data) < XZ_SMALL:
        return lzma.compress(data, preset=9 | lzma.PRESET_EXTREME)
    return subprocess.run(["xz", "-9e", "-T0", "-c"], input=data, capture_output=True, check=True).stdout


def xz_d(data):
    data = bytes(data)
    if len(data) < XZ_SMALL:
        return lzma.decompress(data)
    return subprocess.run(["xz", "-d", "-T0", "-c"], input=data, capture_output=True, check=True).stdout


def tables_c(tables):
    """uint16 tables with their shapes: u32 count, u32 (rows, cols) each, the rows; zstd level 22
    (codecs_gguf.py:121-125)"""
    shapes = np.array([t.shape for t in tables], np.uint32).reshape(-1)
    body = b"".join(np.asarray(t, np.uint16).tobytes() for t in tables)
    return zstd.zstd_c(struct.pack("<I", len(tables)) + shapes.tobytes() + body, 22)


def tables_d(buf):
    raw = zstd.decompress(bytes(buf))
    (n,) = struct.unpack_from("<I", raw)
    shapes = np.frombuffer(raw, np.uint32, 2 * n, 4).reshape(n, 2)
    out, at = [], 4 + 8 * n
    for r, c in shapes:
        out.append(np.frombuffer(raw, np.uint16, int(r) * int(c), at).reshape(int(r), int(c)))
        at += 2 * int(r) * int(c)
    return out


def split(data):
    """(layout, rest bytes, the Q8_0 blocks back to back as an (n, 34) array) (codecs_gguf.py:139-149)"""
    host = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1)
    layout = layout_of(gguf.GGUF(host, light=True), host.size)
    gaps, at = [], 0
    for off, nb, _, _ in layout["t"]:
        gaps.append(host[at:off])
        at = off + nb
    gaps.append(host[at:])
    blocks = np.concatenate([host[off:off + nb] for off, nb, _, _ in layout["t"]]) if layout["t"] else np.zeros(0, np.uint8)
    return layout, np.concatenate(gaps).tobytes(), blocks.reshape(-1, 34)


def join(layout, rest, blocks):
    """the file from its layout, rest bytes and blocks (codecs_gguf.py:152-160)"""
    out = np.empty(layout["size"], np.uint8)
    rest = np.frombuffer(rest, np.uint8)
    at = rat = b = 0
    blocks = blocks.reshape(-1)
    for off, nb, _, _ in layout["t"]:
        out[at:off] = rest[rat:rat + off - at]
        rat += off - at
        out[off:off + nb] = blocks[b:b + nb]
        b += nb
        at = off + nb
    out[at:] = rest[rat:]
    return out.tobytes()


def normalize(counts, scale=1 << PB):
    """frequencies summing to `scale` per row with data (gpu_codec.py:193-209): each count rounded to the
    nearest multiple (at least 1 for a seen symbol), then the rounding drift taken from or given to the
    largest entries one unit at a time, in numpy's descending order of the current row, until it is gone"""
    counts = np.asarray(counts, np.int64)
    tot = counts.sum(1, keepdims=True)
    f = np.where(counts > 0, np.maximum(1, (counts * scale + tot // 2) // np.maximum(tot, 1)), 0)
    for r in np.flatnonzero(tot.reshape(-1)):
        drift = scale - int(f[r].sum())
        while drift:
            for j in np.argsort(-f[r]):
                if drift == 0:
                    break
                if drift > 0:
                    f[r, j] += 1
                    drift -= 1
                elif f[r, j] > 1:
                    f[r, j] -= 1
                    drift += 1
    return f.astype(np.uint16)


def _median_bits(counts, n):
    """numpy's median of n values given their histogram over 0..65535, as an int (gpu_codec.py:231)"""
    c = np.cumsum(counts, dtype=np.int64)
    at = lambda k: int(np.searchsorted(c, k, side="right"))       # the value of the k-th smallest (0-based)
    return at(n // 2) if n % 2 else (at(n // 2 - 1) + at(n // 2)) // 2


def _cum(freq):
    cum = np.zeros((freq.shape[0], 257), np.uint32)
    np.cumsum(freq.astype(np.uint32), axis=1, out=cum[:, 1:])
    return cum


class M6:
    """compress(file bytes) -> chunk bytes; decompress(chunk) -> file bytes"""
    name = NAME

    def __init__(self, stream=None):
        self.stream = stream

    def _meta(self, layout, med):
        groups = sorted({t[3] for t in layout["t"]})
        meta = np.zeros(len(layout["t"]), META)
        first = colbase = 0
        for i, (_, nbytes, rowlen, grp) in enumerate(layout["t"]):
            nb = nbytes // 34
            meta[i] = (first, nb, rowlen // 32, groups.index(grp), colbase, med[i])
            first += nb
            colbase += rowlen
        return groups, meta

    def compress(self, data):
        st = self.stream
        layout, rest, blocks = split(data)
        with ThreadPoolExecutor(1) as side:
            rest_job = side.submit(xz_c, rest)
            n = blocks.shape[0]
            allb = dev.DeviceArray.from_host(np.ascontiguousarray(blocks).reshape(-1), st)
            med, colmaps, first = [], [], 0
            hist = dev.DeviceArray(65536, np.uint32)
            for _, nbytes, rowlen, _ in layout["t"]:
                nb = nbytes // 34
                hist.zero(st)
                check(lib().spa_m6_scale_hist(allb.ptr, first, nb, hist.ptr, st))
                med.append(_median_bits(hist.to_host(stream=st), nb))
                rms = dev.DeviceArray(rowlen, np.float32)
                check(lib().spa_m6_col_rms(allb.ptr, first, nb // (rowlen // 32), rowlen // 32, rms.ptr, st))
                r = rms.to_host(stream=st)
                edges = np.quantile(r, np.linspace(0, 1, N_COL + 1)[1:-1])
                colmaps.append(np.searchsorted(edges, r).astype(np.uint8))
                first += nb
            colmap = np.concatenate(colmaps) if colmaps else np.zeros(0, np.uint8)
            groups, meta = self._meta(layout, med)
            ntab = len(groups) * TPG
            if n == 0:
                counts = np.zeros((ntab, 256), np.uint32)
                lens = np.zeros(0, np.uint32)
                stream_bytes = b""
                freq = np.zeros((ntab, 256), np.uint16)
            else:
                pos = dev.DeviceArray(n, np.uint8)
                check(lib().spa_m6_pos(allb.ptr, n, pos.ptr, st))
                meta_d = dev.DeviceArray.from_host(meta.view(np.uint8), st)
                tfirst = dev.DeviceArray.from_host(meta["first"].astype(np.int32), st)
                cm_d = dev.DeviceArray.from_host(colmap, st)
                cnt = dev.DeviceArray(ntab * 256, np.uint32).zero(st)
                args = (allb.ptr, pos.ptr, meta_d.ptr, tfirst.ptr, len(meta), cm_d.ptr, n)
                check(lib().spa_m6_hist(*args, cnt.ptr, st))
                counts = cnt.to_host(stream=st).reshape(ntab, 256)
                freq = normalize(counts)
                f_d = dev.DeviceArray.from_host(freq, st)
                c_d = dev.DeviceArray.from_host(_cum(freq), st)
                nseg = lib().spa_m6_segments(n)
                out = dev.DeviceArray(nseg * CAP, np.uint8)
                out_len = dev.DeviceArray(nseg, np.uint32)
                check(lib().spa_m6_encode(*args, f_d.ptr, c_d.ptr, out.ptr, CAP, out_len.ptr, st))
                lens = out_len.to_host(stream=st)
                off = np.zeros(nseg, np.uint64)
                off[1:] = np.cumsum(lens.astype(np.uint64))[:-1]
                total = int(lens.astype(np.uint64).sum())
                sbuf = dev.DeviceArray(max(total, 1), np.uint8)
                off_d = dev.DeviceArray.from_host(off, st)
                check(lib().spa_qr_gather(out.ptr, CAP, out_len.ptr, off_d.ptr, nseg, sbuf.ptr, st))
                stream_bytes = sbuf.to_host(stream=st)[:total].tobytes()
            if lens.size and int(lens.max()) >= 65536:
                raise RuntimeError("M6: a segment longer than 65535 bytes (the format stores u16 lengths)")
            used = np.flatnonzero(counts.sum(1)).astype(np.uint32)
            parts = {
                "layout": zstd.zstd_c(json.dumps(layout).encode()),
                "rest": rest_job.result(),
                "meta": zstd.zstd_c(json.dumps({"groups": groups, "med": med}).encode()),
                "colmap": zstd.zstd_c(colmap.tobytes()),
                "used": zstd.zstd_c(used.tobytes()),
                "tables": tables_c([freq[used]]),
                "seglen": zstd.zstd_c(lens.astype(np.uint16).tobytes()),
                "stream": stream_bytes,
            }
        return pack(parts)

    def decompress(self, buf):
        st = self.stream
        parts = unpack(buf if isinstance(buf, memoryview) else memoryview(bytes(buf)))
        layout = json.loads(zstd.decompress(parts["layout"]))
        with ThreadPoolExecutor(1) as side:
            rest_job = side.submit(xz_d, parts["rest"])
            m = json.loads(zstd.decompress(parts["meta"]))
            groups, meta = self._meta(layout, m["med"])
            ntab = len(groups) * TPG
            used = np.frombuffer(zstd.decompress(parts["used"]), np.uint32)
            if used.size and int(used.max()) >= ntab:
                raise ValueError("M6: a table id beyond the tensor groups")
            freq = np.zeros((ntab, 256), np.uint16)
            if used.size:
                freq[used] = tables_d(parts["tables"])[0]
            lens = np.frombuffer(zstd.decompress(parts["seglen"]), np.uint16).astype(np.uint64)
            colmap = np.frombuffer(zstd.decompress(parts["colmap"]), np.uint8)
            n = sum(t[1] for t in layout["t"]) // 34
            if colmap.size != sum(t[2] for t in layout["t"]) or (colmap.size and int(colmap.max()) >= N_COL):
                raise ValueError("M6: the column classes do not fit the layout")
            nseg = lib().spa_m6_segments(n)
            if len(lens) != nseg:
                raise ValueError(f"M6: {len(lens)} segment lengths for {nseg} segments")
            blocks = np.zeros(0, np.uint8)
            if n:
                off = np.zeros(nseg, np.uint64)
                off[1:] = np.cumsum(lens)[:-1]
                sbytes = np.frombuffer(bytes(parts["stream"]), np.uint8)
                s_d = dev.DeviceArray.from_host(sbytes if sbytes.size else np.zeros(1, np.uint8), st)
                f_d = dev.DeviceArray.from_host(freq, st)
                c_d = dev.DeviceArray.from_host(_cum(freq), st)
                lut = dev.DeviceArray(ntab << PB, np.uint8)
                check(lib().spa_rans_build_lut(c_d.ptr, ntab, lut.ptr, st))
                out = dev.DeviceArray(n * 34, np.uint8).zero(st)
                # (every device array stays referenced until the blocks are read back: the frees would
                # otherwise hand memory to later allocations while the decoder still reads it)
                off_d, meta_d = dev.DeviceArray.from_host(off, st), dev.DeviceArray.from_host(meta.view(np.uint8), st)
                tfirst = dev.DeviceArray.from_host(meta["first"].astype(np.int32), st)
                cm_d = dev.DeviceArray.from_host(colmap, st)
                check(lib().spa_m6_decode(s_d.ptr, sbytes.size, off_d.ptr, meta_d.ptr, tfirst.ptr, len(meta), cm_d.ptr, n,
                                          f_d.ptr, c_d.ptr, lut.ptr, out.ptr, st))
                blocks = out.to_host(stream=st)
            return join(layout, rest_job.result(), blocks)
