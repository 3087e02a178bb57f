"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

CPU restatement of the reference's static context-mixed rANS (seedpack/rans.py, cited as rans.py:LINES):
every symbol is coded with the frequency table of its context; tables are counts per (context, symbol)
normalised to rows of 2^14 (rans.py:15-44); the coder has a 32-bit state, RANS_L 2^23, byte
renormalisation, encodes from the last symbol to the first and ends with the state's 4 bytes (low
byte last written, first read) (rans.py:55-78); the decoder (rans.py:81-105) reads the state first; an
order-1 stream's context is the previous symbol, 0 every `period` symbols (rans.py:108-146).

Pinned by tests/test_oracle_m6.py against tests/golden/m6_vectors.npz, written by running the reference's
own rans.py (tests/golden/make_m6_golden.py), and by round trips and a planted mistake (an order-1
context not reset at the period).
"""
import numpy as np

PROB_BITS = 14
PROB_SCALE = 1 << PROB_BITS
RANS_L = 1 << 23


def normalize(counts):
    """rows of counts -> uint16 frequencies summing to PROB_SCALE (rows without data stay zero): each
    seen symbol round(c * PROB_SCALE / total), at least 1; the drift then fixed one unit at a time over
    the entries in descending order of the rounded row (numpy's argsort), cycling (rans.py:21-44)"""
    counts = np.asarray(counts, np.float64)
    freqs = np.zeros(counts.shape, np.int64)
    for r in range(counts.shape[0]):
        c = counts[r]
        tot = c.sum()
        if tot == 0:
            continue
        f = np.where(c > 0, np.maximum(1, np.round(c * PROB_SCALE / tot)), 0).astype(np.int64)
        drift = PROB_SCALE - int(f.sum())
        order = np.argsort(-f)
        i = 0
        while drift:
            j = order[i % len(order)]
            if drift > 0:
                f[j] += 1
                drift -= 1
            elif f[j] > 1:
                f[j] -= 1
                drift += 1
            i += 1
        freqs[r] = f
    return freqs.astype(np.uint16)


def build_freqs(sym, ctx, n_ctx, n_sym=256):
    counts = np.bincount(np.asarray(ctx, np.int64) * n_sym + np.asarray(sym, np.int64), minlength=n_ctx * n_sym)
    return normalize(counts.reshape(n_ctx, n_sym))


def _cum(freqs):
    cum = np.zeros((freqs.shape[0], freqs.shape[1] + 1), np.int64)
    cum[:, 1:] = np.cumsum(freqs.astype(np.int64), axis=1)
    return cum


def encode(sym, ctx, freqs):
    freqs = np.asarray(freqs)
    cum = _cum(freqs)
    out = bytearray()
    x = RANS_L
    for i in range(len(sym) - 1, -1, -1):
        c, s = int(ctx[i]), int(sym[i])
        f = int(freqs[c, s])
        x_max = ((RANS_L >> PROB_BITS) << 8) * f
        while x >= x_max:
            out.append(x & 0xFF)
            x >>= 8
        x = ((x // f) << PROB_BITS) + (x % f) + int(cum[c, s])
    for _ in range(4):
        out.append(x & 0xFF)
        x >>= 8
    return bytes(out[::-1])


def decode(buf, ctx, freqs, n=None, period=0):
    """ctx per symbol, or (period > 0) the previous symbol, reset every period symbols"""
    freqs = np.asarray(freqs)
    cum = _cum(freqs)
    n = len(ctx) if n is None else n
    out = np.zeros(n, np.uint8)
    x = int.from_bytes(bytes(buf[:4]), "big")
    pos, prev = 4, 0
    for i in range(n):
        if period:
            if i % period == 0:
                prev = 0
            c = prev
        else:
            c = int(ctx[i])
        slot = x & (PROB_SCALE - 1)
        s = int(np.searchsorted(cum[c], slot, side="right")) - 1
        out[i] = s
        prev = s
        x = int(freqs[c, s]) * (x >> PROB_BITS) + slot - int(cum[c, s])
        while x < RANS_L:
            x = (x << 8) | buf[pos]
            pos += 1
    return out


def o1_context(sym, period, plant=False):
    ctx = np.zeros(len(sym), np.int32)
    ctx[1:] = sym[:-1]
    if not plant:
        ctx[::period] = 0
    return ctx
