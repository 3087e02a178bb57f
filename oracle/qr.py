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
GRID_TYPES = (16, 17, 18, 19, 21, 22, 29)
BS = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 20: 18, 23: 136, 42: 18,
      16: 66, 17: 74, 18: 98, 19: 50, 21: 110, 22: 82, 29: 56}
QK = {t: (32 if t in (2, 3, 6, 7, 8, 20) else 64 if t == 42 else 256) for t in SELF_TYPES + GRID_TYPES}
NFIELD = {2: 1, 6: 1, 8: 1, 20: 1, 42: 1, 3: 2, 7: 2, 10: 34, 11: 17, 14: 17, 12: 18, 13: 18, 23: 9,
          16: 9, 18: 9, 19: 9, 21: 9, 17: 17, 22: 17, 29: 17}
# grid-type contexts (qr.py:386-388, :72-73): rank (model 1), signs (model 1), IQ1_M shift bit,
# rank and signs by the unit's position in its row (model 2)
GRID_RANK, GRID_SIGN, GRID_SHIFT = NSB_MAX, NSB_MAX + 8, NSB_MAX + 24
GRANK2, GSIGN2 = NTAB + 128, NTAB + 144
TOPK = 16
GSIZE = {16: 256, 18: 256, 17: 512, 21: 512, 22: 1024, 19: 2048, 29: 2048}
PARITY = (16, 17, 18)           # 7 stored sign bits per 8, the 8th by even parity
# x / literal in the QR kernels is x * RN(1 / literal) (the reference's ptxas and --cpu build, cpukernels.py:254-264)
INV = {22: F32(1) / F32(0.9875), 21: F32(1) / F32(1.033), 19: F32(1) / F32(1.125), 29: F32(1) / F32(1.1125)}
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
    if T in (11, 14, 23) or T in GRID_TYPES:
        return 0 if k == 0 else 2
    return 0


def iq1m_d(B):
    """IQ1_M: the fp16 super-scale bits kept in the top nibbles of the four scale words (qr.py:200-203)"""
    return ((_u16(B, 48) >> 12) | ((_u16(B, 50) >> 8) & 0xF0) | ((_u16(B, 52) >> 4) & 0xF00) | (_u16(B, 54) & 0xF000))


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
    # grid types (qr.py:223-230): fp16 d, then the 4-bit (IQ1: 3-bit, IQ1_S with its shift bit) scales
    if T == 29:
        if k == 0:
            return iq1m_d(B)
        j = k - 1
        return (_u16(B, 48 + 2 * (j >> 2)) >> (3 * (j & 3))) & 7
    if k == 0:
        return _u16(B, 0)
    j = k - 1
    if T == 16:
        return b(2 + 8 * j + 7) >> 4
    if T == 18:
        return b(66 + 4 * j + 3) >> 4
    if T in (17, 22, 21):
        return (b({17: 66, 22: 74, 21: 106}[T] + j // 2) >> (4 * (j % 2))) & 15
    if T == 19:
        return b(34 + 2 * j + 1) >> 4
    raise ValueError(T)


def fpred(T, mv, PB_, k, t0, t1):
    """prediction of field k given the true fp16 fields t0, t1 (qr.py:259-283)"""
    pr = get_field(T, PB_, k)
    two = T in (10, 12, 13)
    if T in GRID_TYPES:
        return _fpred_grid(T, mv, PB_, k, pr, t0)
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


def _fpred_grid(T, mv, PB_, k, pr, t0):
    """grid types: the predicted sub-scale rescaled so that d (2 ls + 1) stays the prediction's
    (qr.py:272-277); IQ1_S keeps its shift bit"""
    if mv < 2 or k < 1:
        return pr
    tv = h2f(t0)
    pv = h2f(get_field(T, PB_, 0))
    ok = (tv != 0) & np.isfinite(tv) & np.isfinite(pv)
    hi = 7 if T in (19, 29) else 15
    ls = pr & 7 if T == 19 else pr
    with np.errstate(all="ignore"):
        v = ((F32(2) * ls.astype(F32) + F32(1)) * pv).astype(F32)     # (float)(2 ls + 1) is exact
        v = np.rint(((v / tv).astype(F32) - F32(1)).astype(F32) * F32(0.5)).astype(F32)
        q = np.fmin(np.fmax(v, F32(0)), F32(hi)).astype(np.int64)
    q = (pr & 8) | q if T == 19 else q
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


# ------------------------------------------------------------------ grid types (qr.py:385-646)

def _b(B, i):
    return int(B[i])


def _u16s(B, o):
    return int(B[o]) | (int(B[o + 1]) << 8)


def _u32s(B, o):
    return _u16s(B, o) | (_u16s(B, o + 2) << 16)


def get_gidx(T, B, g):
    """grid index of group g (8 weights; IQ3: 4) of one block (qr.py:396-407)"""
    if T == 16:
        return _b(B, 2 + 8 * (g >> 2) + (g & 3))
    if T == 17:
        return _u16s(B, 2 + 2 * g) & 511
    if T == 22:
        return _b(B, 2 + g) | ((_b(B, 66 + (g >> 2)) << (8 - 2 * (g & 3))) & 0x300)
    if T == 18:
        return _b(B, 2 + g)
    if T == 21:
        return _b(B, 2 + g) | ((_b(B, 66 + (g >> 3)) << (8 - (g & 7))) & 256)
    if T == 19:
        return _b(B, 2 + g) | (((_u16s(B, 34 + 2 * (g >> 2)) >> (3 * (g & 3))) & 7) << 8)
    if T == 29:
        return _b(B, g) | ((_b(B, 32 + 2 * (g >> 2) + ((g & 3) >> 1)) << (4 if g & 1 else 8)) & 0x700)
    raise ValueError(T)


def get_neg(T, B, w):
    """1 if weight w is stored negative; parity types: the 8th sign of a group from the other 7
    (qr.py:420-432)"""
    j = w & 7
    if T == 16:
        s7 = (_u32s(B, 2 + 8 * (w >> 5) + 4) >> (7 * ((w >> 3) & 3))) & 127
    elif T == 17:
        s7 = _u16s(B, 2 + 2 * (w >> 3)) >> 9
    elif T == 18:
        s7 = (_u32s(B, 66 + 4 * (w >> 5)) >> (7 * ((w >> 3) & 3))) & 127
    elif T == 22:
        return (_b(B, 34 + (w >> 3)) >> j) & 1
    elif T == 21:
        return (_b(B, 74 + (w >> 3)) >> j) & 1
    else:
        return 0
    return (s7 >> j) & 1 if j < 7 else bin(s7).count("1") & 1


def get_shift(B, u):
    """IQ1_M: unit u's shift bit (qr.py:445)"""
    return (_b(B, 32 + 2 * (u >> 2) + ((u & 3) >> 1)) >> (7 if u & 1 else 3)) & 1


def gscale(T, B, u):
    """(s, dl) of unit u: level l has the value s (2 l + 1) (IQ1: s (l - 1 + dl)); the quantizers'
    fudge factors on the stored fp16 taken back out (qr.py:449-463)"""
    dl = F32(0)
    if T == 29:
        d = (h2f(iq1m_d(B[None, :]))[0] * INV[29]).astype(F32)
        j = 2 * (u >> 2) + ((u & 3) >> 1)
        ls = (_u16s(B, 48 + 2 * (j >> 2)) >> (3 * (j & 3))) & 7
        dl = F32(-0.125) if get_shift(B, u) else F32(0.125)
    else:
        d = h2f(_u16s(B, 0))
        if T in INV:
            d = (d * INV[T]).astype(F32)
        if T == 16:
            ls = _b(B, 2 + 8 * (u >> 2) + 7) >> 4
        elif T == 17:
            ls = (_b(B, 66 + (u >> 2)) >> (4 * ((u & 3) >> 1))) & 15
        elif T == 22:
            ls = (_b(B, 74 + (u >> 2)) >> (4 * ((u & 3) >> 1))) & 15
        elif T == 18:
            ls = _b(B, 66 + 4 * (u >> 2) + 3) >> 4
        elif T == 21:
            ib = u >> 2
            ls = (_b(B, 106 + (ib >> 1)) >> (4 * (ib & 1))) & 15
        else:                                   # IQ1_S
            qh = _u16s(B, 34 + 2 * (u >> 2))
            ls = (qh >> 12) & 7
            dl = F32(-0.125) if qh & 0x8000 else F32(0.125)
    with np.errstate(all="ignore"):
        return F32(F32(d) * F32(2 * ls + 1)), dl


def pos4(col, cols):
    return 0 if cols <= 0 or col < 256 else 1 + min(2, col * 3 // cols)


def grid_distances(T, gk, uu, ww, dl):
    """weighted squared error of every grid point against the unit's targets: pair tables of level
    errors (qr.py:505-517), then N/2 lookups summed in pair order, NaN -> inf (qr.py:518-525)"""
    sgn = T not in (19, 29)
    n = len(uu)
    bits = 2 if n == 8 else 3
    lv = np.arange(1 << bits)
    qv = (2 * lv + 1).astype(F32) if sgn else ((lv - 1).astype(F32) + dl).astype(F32)
    d = np.zeros(len(gk), F32)
    with np.errstate(all="ignore"):
        for p in range(n // 2):
            ea = (qv - uu[2 * p]).astype(F32)
            eb = (qv - uu[2 * p + 1]).astype(F32)
            # table entry e = la | lb << bits: ww[2p] ea^2 + ww[2p+1] eb^2
            tab = ((ww[2 * p] * (ea * ea)).astype(F32)[None, :] + (ww[2 * p + 1] * (eb * eb)).astype(F32)[:, None]).astype(F32)
            tab = tab.reshape(-1)
            key = (gk.astype(np.int64) >> (2 * bits * p)) & ((1 << 2 * bits) - 1)
            d = (d + tab[key]).astype(F32)
    d[np.isnan(d)] = np.inf
    return d


def gapctx(d1, d2):
    with np.errstate(all="ignore"):
        g = F32(F32(d2 - d1) / F32(d1 + F32(1e-30)))
    return int(g >= F32(0.05)) + int(g >= F32(0.2)) + int(g >= F32(0.6))


def grid_symbols(T, fb, pb, x, imw, col0, cols, mv, gk):
    """decode-order symbols of the grid codes of one block (qr.py:553-637): per unit of 8 weights,
    IQ1_M's shift bit, then per lattice group the rank of the true point among all grid points in
    (distance, index) order (escape 16 + the index's two bytes beyond rank 15), then the signs"""
    n = 4 if T in (18, 21) else 8
    ng = 8 // n
    sgn = T not in (19, 29)
    par = T in PARITY
    sx2 = np.add.accumulate(np.concatenate([[F32(0)], (x * x).astype(F32)]).astype(F32))[-1]
    sigma2 = F32(sx2 * F32(1 / 256)) if T in (16, 17) else F32(F32(F32(2) * sx2) * F32(1 / 256))
    out = []
    for u in range(32):
        rank0 = GRANK2 + 4 * pos4(col0 + 8 * u, cols) if mv >= 2 else GRID_RANK
        sign0 = GSIGN2 + 16 * pos4(col0 + 8 * u, cols) if mv >= 2 else GRID_SIGN
        if T == 29:
            out.append((GRID_SHIFT, get_shift(fb, u) ^ get_shift(pb, u)))
        s, dl = gscale(T, fb, u)
        xu = x[8 * u:8 * u + 8]
        with np.errstate(all="ignore"):
            w = np.sqrt((sigma2 + (xu * xu).astype(F32)).astype(F32)).astype(F32)
            if imw is not None:
                w = (w * imw[8 * u:8 * u + 8]).astype(F32)
        pn = (xu < 0).astype(np.int64)
        v = np.abs(xu) if sgn else xu.copy()
        if sgn and par and pn.sum() & 1:
            a = ((w * xu).astype(F32) * xu).astype(F32)
            im = 0
            for i in range(1, 8):
                if a[i] < a[im]:
                    im = i
            pn[im] ^= 1
            v[im] = -v[im]
        with np.errstate(all="ignore"):
            uu = (v / s).astype(F32)
        tg = [get_gidx(T, fb, u * ng + gg) for gg in range(ng)]
        for gg in range(ng):
            d = grid_distances(T, gk, uu[gg * n:(gg + 1) * n], w[gg * n:(gg + 1) * n], dl)
            t = tg[gg]
            dt = d[t]
            k = np.arange(len(d))
            rank = int(((d < dt) | ((d == dt) & (k < t))).sum())
            srt = np.sort(d)
            ctx = gapctx(srt[0], srt[1])
            if rank >= TOPK:
                out += [(rank0 + ctx, TOPK), (FESC_LO, t & 255), (FESC_HI, t >> 8)]
            else:
                out.append((rank0 + ctx, rank))
        if sgn:
            bits, mask = (2, 3) if n == 8 else (3, 7)
            for j in range(8):
                if par and j == 7:
                    continue
                lev = (int(gk[tg[j // n]]) >> (bits * (j % n))) & mask
                with np.errstate(all="ignore"):
                    m4 = F32(abs(uu[j]) * F32(4))
                ctx = (lev == 0) * 8 + (int(m4) if m4 < F32(7) else 7)
                out.append((sign0 + ctx, get_neg(T, fb, 8 * u + j) ^ int(pn[j])))
    return out


# ------------------------------------------------------------------ symbol sequences

def block_symbols(T, F, P, seed, seed_type, cols, mv=2, imx=None, gk=None):
    """the forward (decode-order) symbols of every block, as a list of lists of (table, symbol),
    and the per-block equality flags (qr.py:674-710). Grid types need the grid keys gk (uint16 per
    grid point: its levels, 2 bits each, IQ3 3 bits) and take the imatrix imx (float32 per column)."""
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
    if T in GRID_TYPES:
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
            cidx = (gw0[b] + np.arange(qk)) % cols if cols > 0 else None
            imw = None if imx is None else np.asarray(imx, F32)[cidx]
            seq += grid_symbols(T, Fb[b], Pb[b], x[gw0[b]:gw0[b] + qk], imw, int(col0[b]), cols, mv,
                                np.asarray(gk, np.uint16))
            out.append(seq)
        return out, eq
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


def histogram(T, F, P, seed, seed_type, cols, mv=2, imx=None, gk=None):
    blocks, _ = block_symbols(T, F, P, seed, seed_type, cols, mv, imx, gk)
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


def encode(T, F, P, seed, seed_type, cols, mv=2, imx=None, gk=None):
    """-> dict(counts, freq, used, lens, stream) of one single-tensor batch"""
    counts, blocks = histogram(T, F, P, seed, seed_type, cols, mv, imx, gk)
    freq, used = normalize(counts)
    remap = np.full(NTAB2, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    cum = cum_of(freq)
    parts = [rans_encode(segment_sequence(T, blocks, b0, n), remap, freq, cum) for b0, n in segments(T, len(blocks))]
    return {"counts": counts, "freq": freq, "used": used, "lens": np.array([len(p) for p in parts], np.uint32),
            "stream": np.frombuffer(b"".join(parts), np.uint8)}
