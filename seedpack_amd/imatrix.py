"""llama.cpp importance matrices: the repository's imatrix file read as {tensor name: float32 per input
column}, as the reference's requant.load_imatrix returns it (seedpack/requant.py:59-113).

Two file forms:
  * legacy .dat: i32 entry count; per entry i32 name length, name, i32 call count, i32 value count,
    f32 values (sums over the calls); then optionally i32 chunk count and the dataset name. Values
    are divided by the call count (f32) when it is positive, as llama-quantize does;
  * GGUF (general.type "imatrix"): per tensor "<name>.in_sum2" (matrices x columns) and
    "<name>.counts" (per matrix); value = in_sum2 / count per matrix, 1 where a matrix saw no token.
"""
import struct

import numpy as np

from .gguf import GGUF


def load(buf):
    """bytes of an imatrix file -> {tensor name: float32 array}"""
    buf = bytes(buf)
    if buf[:4] == b"GGUF":
        return _load_gguf(buf)
    out = {}
    (n,) = struct.unpack_from("<i", buf, 0)
    pos = 4
    for _ in range(n):
        (ln,) = struct.unpack_from("<i", buf, pos)
        name = buf[pos + 4:pos + 4 + ln].decode()
        ncall, nval = struct.unpack_from("<ii", buf, pos + 4 + ln)
        pos += 12 + ln
        v = np.frombuffer(buf, np.float32, nval, pos).copy()
        pos += 4 * nval
        if ncall > 0:
            v /= np.float32(ncall)
        out[name] = v
    return out


def chunks(buf):
    """the number of chunks the imatrix was computed on (GGUF imatrix.chunk_count, or the count a
    legacy file stores after its entries), None when it is not recorded"""
    buf = bytes(buf)
    if buf[:4] == b"GGUF":
        c = GGUF(buf, light=True).meta.get("imatrix.chunk_count")
        return None if c is None else int(c)
    try:
        (n,) = struct.unpack_from("<i", buf, 0)
        pos = 4
        for _ in range(n):
            (ln,) = struct.unpack_from("<i", buf, pos)
            (nval,) = struct.unpack_from("<i", buf, pos + 8 + ln)
            pos += 12 + ln + 4 * nval
        return struct.unpack_from("<i", buf, pos)[0] if len(buf) >= pos + 4 else None
    except struct.error:
        return None


def _load_gguf(buf):
    g = GGUF(buf)
    ts = {t.name: t for t in g.tensors}
    out = {}
    for name, t in ts.items():
        if not name.endswith(".in_sum2"):
            continue
        base = name[:-len(".in_sum2")]
        c = ts[base + ".counts"]
        counts = np.frombuffer(buf, np.float32, c.nbytes // 4, c.offset)
        sums = np.frombuffer(buf, np.float32, t.nbytes // 4, t.offset).reshape(len(counts), -1)
        with np.errstate(divide="ignore", invalid="ignore"):
            e = sums / counts[:, None]
        e[counts <= 0] = 1
        out[base] = e.reshape(-1).astype(np.float32)
    return out


def write_dat(entries, ncall=1, chunk_count=None, dataset=None):
    """a legacy .dat file of {name: float32 values} (each entry's sums = values * ncall)"""
    parts = [struct.pack("<i", len(entries))]
    for name, v in entries.items():
        nb = name.encode()
        v = np.asarray(v, np.float32) * np.float32(ncall)
        parts += [struct.pack("<i", len(nb)), nb, struct.pack("<ii", ncall, len(v)), v.astype("<f4").tobytes()]
    if chunk_count is not None:
        parts.append(struct.pack("<i", chunk_count))
        if dataset is not None:
            d = dataset.encode()
            parts += [struct.pack("<i", len(d)), d]
    return b"".join(parts)
