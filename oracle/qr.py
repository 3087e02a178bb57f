"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

CPU restatement of the reference's QR residual coder for the non-grid quant types
(seedpack/qr.py, cited as qr.py:LINES): the per-block model (block flag, scale fields coded against
the prediction, codes coded against round((x - c) / a) of the seed), the host table normalisation,
and the interleaved-segment rANS (PB = 12, RANS_L = 2^23, byte renormalisation).

Formulation: the model is computed for all blocks at once with numpy (float32 IEEE operations in the
kernel's order); the rANS coder runs per segment over the symbol sequence in Python integers.

Pinned by: tests/test_oracle_qr.py checks the histogram, the normalised tables, the segment lengths
and the stream bytes against tests/golden/qr_vectors.npz, written by running the reference's own
QR kernels (qr.py KERNELS) on the CPU through the reference's --cpu backend
(tests/golden/make_qr_golden.py).
"""
import numpy as np

F32 = np.float32
PB = 12
RANS_L = 1 << 23
NSB_MAX = 20
FLAG = NSB_MAX + 64
NTAB = NSB_MAX + 64 + 2
CODE2 = NTAB
NTAB2 = NTAB + 208
FESC_LO, FESC_HI = 8, 9

SELF_TYPES = (2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 20, 23, 42)
BS = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 20: 18, 23: 136, 42: 18}
QK = {t: (32 if t in (2, 3, 6, 7, 8, 20) else 64 if t == 42 else 256) for t in SELF_TYPES}
NFIELD = {2: 1, 6: 1, 8: 1, 20: 1, 42: 1, 3: 2, 7: 2, 10: 34, 11: 17, 14: 17, 12: 18, 13: 18, 23: 9}
QMIN = {8: -128}
QMAX = {10: 3, 42: 3, 11: 7, 6: 31, 7: 31, 13: 31, 14: 63, 8: 127}
KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], F32)   # kvalues_iq4nl
SUBLEN = {10: 16, 11: 16, 14: 16}


def seg_blocks(T):
    """blocks per rANS segment (qr.py:952-954)"""
    return max(16, 16384 // QK[T])


# ------------------------------------------------------------------ block layouts (columns = blocks)

def _u16(B, o):
    return B[:, o].astype(np.int64) | (B[:, o + 1].astype(np.int64) << 8)


def h2f(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(F32)


def _s8(v):
    return ((np.asarray(v, np.int64) + 128) & 255) - 128


def scale_min_k4(B, j, off=4):
    q = lambda i: B[:, off + i].astype(np.int64)   # noqa: E731
    if j < 4:
        return q(j) & 63, q(j + 4) & 63
    return (q(j + 4) & 0xF) | ((q(j - 4) >> 6) << 4), (q(j + 4) >> 4) | ((q(j) >> 6) << 4)


def q3k_scale(B, i, off=96):
    """the 6-bit scale i of a Q3_K block (0..63)"""
    lo = (B[:, off + i].astype(np.int64) & 15) if i < 8 else (B[:, off + i - 8].astype(np.int64) >> 4)
    hi = (B[:, off + 8 + (i % 4)].astype(np.int64) >> (2 * (i // 4))) & 3
    return lo | (hi << 4)


def get_code(T, B, w):
    """code of weight w of every block (qr.py:136-156)"""
    b = lambda i: B[:, i].astype(np.int64)   # noqa: E731
    if T in (2, 20):
        return b(2 + w) & 15 if w < 16 else b(2 + w - 16) >> 4
    if T == 3:
        return b(4 + w) & 15 if w < 16 else b(4 + w - 16) >> 4
    if T in (6, 7):
        qs, qh = (6, 2) if T == 6 else (8, 4)
        lo = b(qs + w) & 15 if w < 16 else b(qs + w - 16) >> 4
        return lo | (((b(qh + (w >> 3)) >> (w & 7)) & 1) << 4)
    if T == 8:
        return _s8(b(2 + w))
    n, r = w >> 7, w & 127
    if T == 10:
        return (b(16 + 32 * n + (r & 31)) >> (2 * (r >> 5))) & 3
    if T == 11:
        j, l = r >> 5, r & 31
        return ((b(32 + 32 * n + l) >> (2 * j)) & 3) | (((b(l) >> (4 * n + j)) & 1) << 2)
    if T in (12, 13):
        c, hf, l = w >> 6, (w >> 5) & 1, w & 31
        v = b((16 if T == 12 else 48) + 32 * c + l)
        q = v >> 4 if hf else v & 15
        return q if T == 12 else q | (((b(16 + l) >> (2 * c + hf)) & 1) << 4)
    if T == 14:
        g, l = r >> 5, r & 31
        v = b(64 * n + l + (32 if g & 1 else 0))
        return ((v & 15) if g < 2 else (v >> 4)) | (((b(128 + 32 * n + l) >> (2 * g)) & 3) << 4)
    if T == 23:
        ib, l = w >> 5, w & 31
        v = b(8 + 16 * ib + (l & 15))
        return v & 15 if l < 16 else v >> 4
    if T == 42:
        return (b(2 + (w >> 2)) >> (2 * (w & 3))) & 3
    raise ValueError(T)


def fkind(T, k):
    """0 fp16 scale, 1 fp16 min, 2 sub-scale, 3 sub-min (qr.py:189-197)"""
    if T in (3, 7):
        return 0 if k == 0 else 1
    if T == 10:
        return 0 if k == 0 else 1 if k == 1 else 2 if k < 18 else 3
    if T in (12, 13):
        return 0 if k == 0 else 1 if k == 1 else 2 if k < 10 else 3
    if T in (11, 14, 23):
        return 0 if k == 0 else 2
    return 0


def get_field(T, B, k):
    """integer scale field k of every block (qr.py:205-222)"""
    b = lambda i: B[:, i].astype(np.int64)   # noqa: E731
    if T in (2, 6, 8, 20, 42):
        return _u16(B, 0)
    if T in (3, 7):
        return _u16(B, 2 * k)
    if T == 10:
        return _u16(B, 80) if k == 0 else _u16(B, 82) if k == 1 else (b(k - 2) & 15) if k < 18 else (b(k - 18) >> 4)
    if T == 11:
        return _u16(B, 108) if k == 0 else q3k_scale(B, k - 1)
    if T in (12, 13):
        if k < 2:
            return _u16(B, 2 * k)
        sc, m = scale_min_k4(B, k - 2 if k < 10 else k - 10)
        return sc if k < 10 else m
    if T == 14:
        return _u16(B, 208) if k == 0 else _s8(b(192 + k - 1))
    if T == 23:
        if k == 0:
            return _u16(B, 0)
        ib = k - 1
        return ((b(4 + ib // 2) >> (4 * (ib % 2))) & 15) | (((_u16(B, 2) >> (2 * ib)) & 3) << 4)
    raise ValueError(T)


def fpred(T, mv, PB_, k, t0, t1):
    """prediction of field k given the true fp16 fields t0, t1 (qr.py:259-283)"""
    pr = get_field(T, PB_, k)
    two = T in (10, 12, 13)
    if mv < 2 or T not in (10, 12, 13, 11, 14, 23) or k < (2 if two else 1):
        return pr
    ref = 1 if (two and k >= (18 if T == 10 else 10)) else 0
    tv = h2f(t1 if ref else t0)
    pv = h2f(get_field(T, PB_, ref))
    ok = (tv != 0) & np.isfinite(tv) & np.isfinite(pv)
    with np.errstate(all="ignore"):
        if T in (11, 23):
            v = np.rint(((pr - 32).astype(F32) * pv).astype(F32) / tv).astype(F32)
            q = np.clip(np.nan_to_num(v, nan=0.0), -32, 31).astype(np.int64) + 32
        else:
            v = np.rint((pr.astype(F32) * pv).astype(F32) / tv).astype(F32)
            lo, hi = (-128, 127) if T == 14 else (0, 15 if T == 10 else 63)
            q = np.clip(np.nan_to_num(v, nan=0.0), lo, hi).astype(np.int64)
    return np.where(ok, q, pr)


def wscale(T, B, w):
    """(a, c) of weight w: value = a * code + c (IQ4: a * KV[code]) (qr.py:295-316)"""
    d = h2f(_u16(B, 0))
    if T == 2:
        return d, (F32(-8) * d).astype(F32)
    if T in (3, 7):
        return d, h2f(_u16(B, 2))
    if T == 6:
        return d, (F32(-16) * d).astype(F32)
    if T in (8, 20):
        return d, np.zeros_like(d)
    if T == 42:
        return d, -d
    n, r = w >> 7, w & 127
    if T == 10:
        sc = B[:, 8 * n + 2 * (r >> 5) + ((r & 31) >= 16)].astype(np.int64)
        a = (h2f(_u16(B, 80)) * (sc & 15).astype(F32)).astype(F32)
        return a, -(h2f(_u16(B, 82)) * (sc >> 4).astype(F32)).astype(F32)
    if T == 11:
        s = q3k_scale(B, 8 * n + 2 * (r >> 5) + ((r & 31) >= 16))
        a = (h2f(_u16(B, 108)) * (s - 32).astype(F32)).astype(F32)
        return a, (F32(-4) * a).astype(F32)
    if T in (12, 13):
        sc, m = scale_min_k4(B, w >> 5)
        a = (d * sc.astype(F32)).astype(F32)
        return a, -(h2f(_u16(B, 2)) * m.astype(F32)).astype(F32)
    if T == 14:
        g, l = r >> 5, r & 31
        s = _s8(B[:, 192 + 8 * n + (l >> 4) + 2 * g])
        a = (h2f(_u16(B, 208)) * s.astype(F32)).astype(F32)
        return a, (F32(-32) * a).astype(F32)
    if T == 23:
        ib = w >> 5
        ls = ((B[:, 4 + ib // 2].astype(np.int64) >> (4 * (ib % 2))) & 15) | (((_u16(B, 2) >> (2 * ib)) & 3) << 4)
        return (d * (ls - 32).astype(F32)).astype(F32), np.zeros_like(d)
    raise ValueError(T)


def _ilogb(v):
    """ilogbf of positive finite floats (subnormals included)"""
    m, e = np.frexp(v.astype(np.float64))
    return (e - 1).astype(np.int64)


def predict(T, a, c, code_pred, x, h, mv, p8):
    """predicted code r, mirror sign s and context (qr.py:348-377) for a normal seed (hboff = 8)"""
    with np.errstate(all="ignore"):
        if T in (20, 23):
            t = (x / a).astype(F32)
            i = np.zeros(t.shape, np.int64)
            for _ in range(14):
                i = np.where((i < 14) & (t >= KV[np.minimum(i + 1, 15)]), i + 1, i)
            g = (KV[i + 1] - KV[i]).astype(F32)
            u = (i.astype(F32) + ((t - KV[i]).astype(F32) / g).astype(F32)).astype(F32)
            hu = (h / (np.abs(a) * g).astype(F32)).astype(F32)
        else:
            u = ((x - c).astype(F32) / a).astype(F32)
            hu = (h / np.abs(a)).astype(F32)
        bad = ~(np.isfinite(u) & np.isfinite(hu))
        ru = np.rint(u).astype(F32)
        fr = (u - ru).astype(F32)
        q = np.clip(np.nan_to_num(ru, nan=0.0, posinf=1e9, neginf=-1e9), QMIN.get(T, 0), QMAX.get(T, 15)).astype(np.int64)
        s = np.where(fr >= 0, 1, -1)
        mb = np.minimum(7, (np.abs(fr) * F32(16)).astype(F32).astype(np.int64) if True else 0)
        hb = np.zeros(u.shape, np.int64)
        pos = hu > 0
        if pos.any():
            hb = np.where(pos, np.maximum(1, np.minimum(7, _ilogb(np.where(pos, hu, 1)) + 8)), 0)
        ctx = NSB_MAX + hb * 8 + mb
        if mv >= 2:
            m32 = np.minimum(15, (np.abs(fr) * F32(32)).astype(F32).astype(np.int64))
            ctx = np.where(hu == 0, CODE2 + p8 * 16 + m32, ctx)
    r = np.where(bad, code_pred, q)
    s = np.where(bad, 1, s)
    ctx = np.where(bad, NSB_MAX + 63, ctx)
    return r, s, ctx


def pos8(col, cols):
    col = np.asarray(col, np.int64)
    if cols <= 0:
        return np.zeros_like(col)
    return np.where(col < 256, 0, 1 + np.minimum(6, col * 7 // cols))


def seed_values(seed, seed_type):
    """(x, h) of every weight of a float seed (qr.py:323-331): BF16 (30), F32 (0), F16 (1); h = 0"""
    if seed_type == 30:
        x = (np.frombuffer(seed, np.uint16).astype(np.uint32) << 16).view(F32)
    elif seed_type == 0:
        x = np.frombuffer(seed, F32).copy()
    elif seed_type == 1:
        x = np.frombuffer(seed, np.float16).astype(F32)
    else:
        raise NotImplementedError(f"oracle: seed type {seed_type}")
    return x, np.zeros_like(x)


# ------------------------------------------------------------------ symbol sequences

def block_symbols(T, F, P, seed, seed_type, cols, mv=2):
    """the forward (decode-order) symbols of every block, as a list of lists of (table, symbol),
    and the per-block equality flags (qr.py:674-710)"""
    bs, qk, nf = BS[T], QK[T], NFIELD[T]
    Fb = np.frombuffer(F, np.uint8).reshape(-1, bs)
    Pb = np.frombuffer(P, np.uint8).reshape(-1, bs)
    nb = len(Fb)
    eq = (Fb == Pb).all(1)
    x, h = seed_values(seed, seed_type)
    tv = [get_field(T, Fb, k) for k in range(nf)]
    t1 = tv[1] if nf > 1 else np.zeros(nb, np.int64)
    fsyms = []
    anyv = np.zeros(nb, bool)
    for k in range(nf):
        kd = fkind(T, k)
        pr = fpred(T, mv, Pb, k, tv[0], t1)
        dlt = tv[k] - pr
        esc = (kd < 2) & ((dlt < -127) | (dlt > 127))
        fsyms.append((kd * 2 + anyv.astype(np.int64), np.where(esc, 128, dlt & 255), esc, tv[k]))
        anyv = anyv | (dlt != 0)
    gw0 = np.arange(nb, dtype=np.int64) * qk
    col0 = gw0 % cols if cols > 0 else np.zeros(nb, np.int64)
    ctxs = np.zeros((nb, qk), np.int64)
    syms = np.zeros((nb, qk), np.int64)
    for w in range(qk):
        a, c = wscale(T, Fb, w)
        r, s, ctx = predict(T, a, c, get_code(T, Pb, w), x[gw0 + w], h[gw0 + w], mv, pos8(col0 + w, cols))
        ctxs[:, w] = ctx
        syms[:, w] = (s * (get_code(T, Fb, w) - r)) & 255
    out = []
    for b in range(nb):
        if eq[b]:
            out.append(None)
            continue
        seq = []
        for (tab, sym, esc, t) in fsyms:
            seq.append((int(tab[b]), int(sym[b])))
            if esc[b]:
                seq.append((FESC_LO, int(t[b]) & 255))
                seq.append((FESC_HI, int(t[b]) >> 8))
        seq.extend(zip(ctxs[b].tolist(), syms[b].tolist()))
        out.append(seq)
    return out, eq


def segments(T, nb):
    sb = seg_blocks(T)
    return [(b0, min(sb, nb - b0)) for b0 in range(0, nb, sb)]


def segment_sequence(T, blocks, b0, n):
    """forward symbols of segment [b0, b0+n): flag (context = previous block's flag) then the block"""
    seq = []
    prev = 1
    for b in range(b0, b0 + n):
        e = blocks[b] is None
        seq.append((FLAG + prev, 1 if e else 0))
        if not e:
            seq.extend(blocks[b])
        prev = 1 if e else 0
    return seq


def histogram(T, F, P, seed, seed_type, cols, mv=2):
    blocks, _ = block_symbols(T, F, P, seed, seed_type, cols, mv)
    counts = np.zeros((NTAB2, 256), np.uint32)
    for b0, n in segments(T, len(blocks)):
        for tab, s in segment_sequence(T, blocks, b0, n):
            counts[tab, s] += 1
    return counts, blocks


def normalize(counts, scale=1 << PB):
    """counts (T, 256) -> (uint16 freqs of the used rows, used row ids), every row summing to scale
    and every seen symbol >= 1 (qr.py:904-923)"""
    c = np.asarray(counts).astype(np.int64)
    tot = c.sum(1)
    used = np.flatnonzero(tot)
    f = np.zeros((len(used), 256), np.int64)
    for k, r in enumerate(used):
        row = c[r]
        fr = np.where(row > 0, np.maximum(1, row * scale // tot[r]), 0)
        diff = scale - int(fr.sum())
        while diff != 0:
            j = int(np.argmax(fr))
            if diff > 0:
                step = diff
            else:
                step = -min(-diff, int(fr[j]) - 1)
            if step == 0:
                j = int(np.flatnonzero(fr > 1)[0])
                step = -1
            fr[j] += step
            diff -= step
        f[k] = fr
    return f.astype(np.uint16), used.astype(np.int32)


def cum_of(freq):
    cum = np.zeros((freq.shape[0], 257), np.uint32)
    cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    return cum


def rans_encode(seq, remap, freq, cum):
    """one segment: the forward symbol sequence coded backwards; returns the segment's bytes"""
    x = RANS_L
    out = bytearray()
    for tab, s in reversed(seq):
        tt = int(remap[tab])
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


def encode(T, F, P, seed, seed_type, cols, mv=2):
    """-> dict(counts, freq, used, lens, stream) of one single-tensor batch"""
    counts, blocks = histogram(T, F, P, seed, seed_type, cols, mv)
    freq, used = normalize(counts)
    remap = np.full(NTAB2, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    cum = cum_of(freq)
    parts = [rans_encode(segment_sequence(T, blocks, b0, n), remap, freq, cum) for b0, n in segments(T, len(blocks))]
    return {"counts": counts, "freq": freq, "used": used, "lens": np.array([len(p) for p in parts], np.uint32),
            "stream": np.frombuffer(b"".join(parts), np.uint8)}
