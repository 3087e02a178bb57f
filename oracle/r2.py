"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

CPU restatement of the reference's R2 BF16 base codec core (seedpack/bf16v2.py, cited as
bf16v2.py:LINES) and of the deterministic arithmetic it decides with (seedpack/detmath.py):

  * side information per tensor: rfi (per row) and cfi (per column) = rint(8 log2 rms) in 1/8
    octave, scl (per column) = the column's mean class (bf16v2.py:225-244), from in-order float64
    sums and detmath's log2 / exp2 polynomials (detmath.py:20-58);
  * exact duplicate rows by a 64-bit row fingerprint and a byte check (bf16v2.py:148-155, :246-271);
  * three symbols per weight -- exponent (context: predicted 1/8-octave level, 512), mantissa
    (context: exponent minus prediction, 128), sign (context: the column's class, 16) -- counted
    into tables shared by all tensors of a role (bf16v2.py:54-75);
  * table normalisation to 2^15 (gpu2.py:460-480) and per-segment rANS (16384 weights, PB 15,
    byte renormalisation, backwards with a 4-byte flush; bf16v2.py:77-111).

Pinned by tests/test_oracle_r2.py: every intermediate (side information, duplicate pairs, counts,
tables, segment lengths, stream bytes) against tests/golden/r2_vectors.npz, written by running the
reference's own code through its --cpu backend (tests/golden/make_r2_golden.py); log2 / exp2 against
the C library within 1 ulp and exactly at powers of two.
"""
import re

import numpy as np

PB = 15
RANS_L = 1 << 23
K = 8
SEG = 16384
NE, NM, NS = 512, 128, 16
TPT = NE + NM + NS
TB_DT = np.dtype([("doff", "<i8"), ("rowlen", "<i4"), ("rowbase", "<i4"), ("colbase", "<i4"), ("tab", "<i4"),
                  ("rmap", "<i4"), ("pad", "<i4")])
SG_DT = np.dtype([("t", "<i4"), ("n", "<i4"), ("i0", "<i8")])

F64 = np.float64
_TWO52 = 4503599627370496.0


# ------------------------------------------------------------------ detmath (detmath.py:20-58)

def dm_rint(x):
    """half to even by adding 2^52 (detmath.py:20-25)"""
    x = np.asarray(x, F64)
    y = (np.abs(x) + _TWO52) - _TWO52
    return np.where(np.abs(x) < _TWO52, np.copysign(y, x), x)


_LOG2_P = [0.043478260869565216, 0.047619047619047616, 0.05263157894736842, 0.058823529411764705,
           0.06666666666666667, 0.07692307692307693, 0.09090909090909091, 0.1111111111111111,
           0.14285714285714285, 0.2, 0.3333333333333333, 1.0]
_EXP2_P = [4.779477332387385e-14, 7.647163731819816e-13, 1.1470745597729725e-11, 1.6059043836821613e-10,
           2.08767569878681e-09, 2.505210838544172e-08, 2.7557319223985893e-07, 2.755731922398589e-06,
           2.48015873015873e-05, 0.0001984126984126984, 0.001388888888888889, 0.008333333333333333,
           0.041666666666666664, 0.16666666666666666, 0.5, 1.0, 1.0]


def dm_log2(x):
    """log2 from IEEE basic operations: mantissa in [sqrt(1/2), sqrt(2)), ln m = 2 atanh((m-1)/(m+1))
    by its series (detmath.py:27-45)"""
    x = np.atleast_1d(np.asarray(x, F64)).copy()
    out = np.empty_like(x)
    with np.errstate(all="ignore"):
        special = np.isnan(x) | (x <= 0) | np.isinf(x)
        out[np.isnan(x)] = np.nan
        out[x < 0] = np.nan
        out[x == 0] = -np.inf
        out[np.isposinf(x)] = np.inf
        v = np.where(special, 1.0, x)
        u = v.view(np.int64)
        e = ((u >> 52) & 0x7FF).astype(np.int64)
        sub = e == 0
        vs = np.where(sub, v * 18014398509481984.0, v)
        u = vs.view(np.int64)
        e = np.where(sub, ((u >> 52) & 0x7FF) - 54, e) - 1023
        m = ((u & 0x000FFFFFFFFFFFFF) | 0x3FF0000000000000).view(F64)
        big = m > 1.4142135623730951
        m = np.where(big, m * 0.5, m)
        e = e + big
        s = (m - 1.0) / (m + 1.0)
        z = s * s
        p = np.full_like(s, 0.04)
        for c in _LOG2_P:
            p = p * z + c
        r = e.astype(F64) + (2.0 * s * p) * 1.4426950408889634
    out[~special] = r[~special]
    return out


def dm_exp2(y):
    """2^y from IEEE basic operations: e^t series on the fraction, 2^k as two normal factors
    (detmath.py:47-58)"""
    y = np.atleast_1d(np.asarray(y, F64)).copy()
    out = np.empty_like(y)
    with np.errstate(all="ignore"):
        nan = np.isnan(y)
        hi = y >= 1024.0
        lo = y < -1075.0
        ok = ~(nan | hi | lo)
        yy = np.where(ok, y, 0.0)
        n = dm_rint(yy)
        t = (yy - n) * 0.6931471805599453
        p = np.full_like(t, 2.8114572543455206e-15)
        for c in _EXP2_P:
            p = p * t + c
        k = n.astype(np.int64)
        k1 = np.trunc(k / 2).astype(np.int64)           # C integer division truncates toward zero
        k2 = k - k1
        f1 = ((k1 + 1023) << 52).view(F64)
        f2 = ((k2 + 1023) << 52).view(F64)
        r = p * f1 * f2
    out[nan] = np.nan
    out[hi] = np.inf
    out[lo] = 0.0
    out[ok] = r[ok]
    return out


def rows_sum(w, square):
    """float64 sums along the rows in index order (detmath.py:77-85): s = s + v*v (or v)"""
    v = np.asarray(w, np.float32).astype(F64)
    t = v * v if square else v
    z = np.zeros((t.shape[0], 1), F64)
    return np.add.accumulate(np.concatenate([z, t], 1), axis=1)[:, -1]


def cols_sum(w, square):
    """float64 sums down the columns in row order (detmath.py:95-106)"""
    v = np.asarray(w, np.float32).astype(F64)
    t = v * v if square else v
    z = np.zeros((1, t.shape[1]), F64)
    return np.add.accumulate(np.concatenate([z, t], 0), axis=0)[-1]


# ------------------------------------------------------------------ side information

def bf16_f32(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


def stats(u, rl):
    """(rfi int16 per row, cfi int16 per column, scl int8 per column) of one tensor of BF16 bits
    (bf16v2.py:225-244); row and column sums run over chunks of 16M weights as in the reference"""
    u = np.asarray(u, np.uint16).reshape(-1, rl)
    nr = u.shape[0]
    step = max(1, (16 << 20) // rl)
    rf = np.empty(nr, F64)
    with np.errstate(all="ignore"):
        for r0 in range(0, nr, step):
            w = bf16_f32(u[r0:r0 + step])
            rf[r0:r0 + step] = dm_log2(np.sqrt(rows_sum(w, True) / rl) + 1e-30)
        rfa = dm_exp2(rf).astype(np.float32)
        s2 = np.zeros(rl, F64)
        s1 = np.zeros(rl, F64)
        for r0 in range(0, nr, step):
            w = (bf16_f32(u[r0:r0 + step]) / rfa[r0:r0 + step, None]).astype(np.float32)
            s2 = s2 + cols_sum(w, True)
            s1 = s1 + cols_sum(w, False)
        cf = dm_log2(np.sqrt(s2 / nr) + 1e-30)
        rfi = np.clip(np.rint(rf * K), -32768, 32767).astype(np.int16)
        cfi = np.clip(np.rint(cf * K), -32768, 32767).astype(np.int16)
        bias = (s1 / nr) / dm_exp2(cfi.astype(F64) / K)
        scl = np.clip(np.floor(bias * 16) + 8, 0, 15).astype(np.int8)
    return rfi, cfi, scl


def row_hash(u, rl):
    """64-bit fingerprint per row: FNV-style, with a xor-shift (bf16v2.py:148-155)"""
    u = np.asarray(u, np.uint16).reshape(-1, rl).astype(np.uint64)
    a = np.full(u.shape[0], 1469598103934665603, np.uint64)
    prime = np.uint64(1099511628211)
    with np.errstate(over="ignore"):
        for j in range(rl):
            a ^= u[:, j]
            a *= prime
            a ^= a >> np.uint64(29)
    return a


def dups(u, rl):
    """(rows kept (sorted) or None, [(duplicate row, source row)]) (bf16v2.py:246-271)"""
    u = np.asarray(u, np.uint16).reshape(-1, rl)
    nr = u.shape[0]
    h = row_hash(u, rl)
    order = np.argsort(h, kind="stable")
    hs = h[order]
    same = np.flatnonzero(hs[1:] == hs[:-1])
    if len(same) == 0:
        return None, []
    pairs, isdup, first = [], np.zeros(nr, bool), {}
    for k in np.unique(np.concatenate([same, same + 1])):
        r = int(order[k])
        cands = first.setdefault(int(hs[k]), [])
        src = next((c for c in cands if np.array_equal(u[c], u[r])), None)
        if src is None:
            cands.append(r)
        else:
            pairs.append((r, src))
            isdup[r] = True
    if not pairs:
        return None, []
    return np.flatnonzero(~isdup).astype(np.int32), sorted(pairs)


# ------------------------------------------------------------------ layout and symbols

def role(name):
    return re.sub(r"blk\.\d+\.", "", name)


def groups(layout, group_bytes):
    """tensors in groups of at most group_bytes (bf16v2.py:190-198)"""
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
    """each tensor's first row / column in the side-information arrays (bf16v2.py:200-206)"""
    rb, cb, rowbase, colbase = [], [], 0, 0
    for off, nb, rl, _ in layout["t"]:
        rb.append(rowbase)
        cb.append(colbase)
        rowbase += nb // 2 // rl
        colbase += rl
    return rb, cb, rowbase, colbase


def symbols(u, rl, rows_kept, rfi_t, cfi_t, scl_t, tab):
    """the forward symbol sequence (table, symbol) of one tensor's coded rows, three per weight"""
    u = np.asarray(u, np.uint16).reshape(-1, rl)
    rows = np.arange(u.shape[0]) if rows_kept is None else rows_kept
    w = u[rows].astype(np.int64)
    ex, man, sgn = (w >> 7) & 255, w & 127, w >> 15
    pred = rfi_t[rows].astype(np.int64)[:, None] + cfi_t.astype(np.int64)[None, :]
    pe = np.clip(pred + 256, 0, 511)
    rlc = np.clip(8 * ex - pred - 1016 + 64, 0, 127)
    sc = np.broadcast_to(scl_t.astype(np.int64)[None, :], w.shape)
    t = np.stack([tab + pe, tab + 512 + rlc, tab + 640 + sc], -1).reshape(-1)
    s = np.stack([ex, man, sgn], -1).reshape(-1)
    return t, s


def normalize(counts, scale=1 << PB):
    """gpu2.py:460-480: proportional frequencies rounded to nearest, then up to 64 passes moving the
    surplus onto each row's largest entry and taking one unit from each of its |deficit| largest
    entries above 1 (ranks by a stable sort)"""
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
    assert (f.sum(1) == scale).all() and ((c > 0) <= (f > 0)).all()
    return f.astype(np.uint16), used.astype(np.int32)


def cum_of(freq):
    cum = np.zeros((freq.shape[0], 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    return cum


def rans_encode(tabs, syms, remap, freq, cum):
    """one segment: forward symbols coded backwards, 4-byte flush; the segment's bytes"""
    x = RANS_L
    out = bytearray()
    tt_all = remap[tabs]
    for tt, s in zip(tt_all[::-1].tolist(), syms[::-1].tolist()):
        f, c = int(freq[tt, s]), int(cum[tt, s])
        xm = ((RANS_L >> PB) << 8) * f
        while x >= xm:
            out.append(x & 0xFF)
            x >>= 8
        x = ((x // f) << PB) + (x % f) + c
    for _ in range(4):
        out.append(x & 0xFF)
        x >>= 8
    return bytes(reversed(out))


def compress(data, layout, group_bytes):
    """the coded parts of a file's 2-D BF16 tensors: side information, duplicate rows, tables,
    segment lengths, stream (bf16v2.py:323-411 without the GGUF header)"""
    host = np.frombuffer(data, np.uint8)
    rb, cb, nrow, ncol = bases(layout)
    rfi = np.zeros(nrow, np.int16); cfi = np.zeros(ncol, np.int16); scl = np.zeros(ncol, np.int8)
    counts = np.zeros((layout["nroles"] * TPT, 256), np.uint32)
    per_tensor, nrows_c, dup_rows, rowmap = [], [], [], []
    for i, (off, nb, rl, _) in enumerate(layout["t"]):
        u = host[off:off + nb].view(np.uint16)
        r_, c_, s_ = stats(u, rl)
        rfi[rb[i]:rb[i] + len(r_)] = r_; cfi[cb[i]:cb[i] + rl] = c_; scl[cb[i]:cb[i] + rl] = s_
        keep, pairs = dups(u, rl)
        nrows_c.append(nb // 2 // rl if keep is None else len(keep))
        dup_rows += [[i, r, s] for r, s in pairs]
        if keep is not None:
            rowmap.append(keep)
        t, s = symbols(u, rl, keep, r_, c_, s_, layout["role"][i] * TPT)
        np.add.at(counts, (t, s), 1)
        per_tensor.append((t, s))
    freq, used = normalize(counts)
    remap = np.full(counts.shape[0], -1, np.int64)
    remap[used] = np.arange(len(used))
    cum = cum_of(freq)
    lens, parts = [], []
    for grp in groups(layout, group_bytes):
        for i in grp:
            t, s = per_tensor[i]
            n = len(t) // 3
            for i0 in range(0, n, SEG):
                seg = rans_encode(t[3 * i0:3 * min(n, i0 + SEG)], s[3 * i0:3 * min(n, i0 + SEG)], remap, freq, cum)
                lens.append(len(seg))
                parts.append(seg)
    return dict(rfi=rfi, cfi=cfi, scl=scl, counts=counts, freq=freq, used=used, lens=np.array(lens, np.uint32),
                stream=np.frombuffer(b"".join(parts), np.uint8), nrows_c=np.array(nrows_c, np.int64),
                dups=np.array(sorted(dup_rows), np.int64).reshape(-1, 3),
                rowmap=np.concatenate(rowmap).astype(np.int32) if rowmap else np.zeros(1, np.int32))
