"""The reference's static context-mixed rANS (seedpack/rans.py: the coder of its CPU single-file methods
M3-M5 and of bf16codec) on the device.

Every symbol (8 bits) is coded with the frequency table of its context; the tables are counts per
(context, symbol) normalised to rows of 2^14 on the host (rans.py:15-44). A stream's state is serial,
so each stream is one lane of spa_crans_encode / spa_crans_decode and independent streams go in one
launch (encode_many, decode_many); the stream bytes equal rans.encode's, and an order-1 stream (the
context is the previous symbol, 0 every `period` symbols, rans.py:108-146) decodes from its bytes alone.
"""
import numpy as np

from . import device as dev
from ._lib import check, lib

PROB_BITS = 14
PROB_SCALE = 1 << PROB_BITS
STREAM = np.dtype([("sym_off", "<i8"), ("n", "<i8"), ("ctx_off", "<i8"), ("tab_row", "<i8"), ("out_off", "<i8"),
                   ("period", "<i4"), ("pad", "<i4")])


def normalize(counts):
    """rows of counts -> uint16 rows summing to 2^14 (rows without data stay zero): a seen symbol gets
    round(count * 2^14 / total) (at least 1), then the rounding drift is spread one unit at a time over
    the row's entries taken cyclically in numpy's descending order of the rounded row, never taking an
    entry below 1 (rans.py:21-44)"""
    counts = np.asarray(counts, np.float64)
    out = np.zeros(counts.shape, np.int64)
    for r, c in enumerate(counts):
        total = c.sum()
        if total == 0:
            continue
        f = np.where(c > 0, np.maximum(1, np.round(c * PROB_SCALE / total)), 0).astype(np.int64)
        drift = PROB_SCALE - int(f.sum())
        order = np.argsort(-f)
        k = 0
        while drift:
            j = order[k % len(order)]
            if drift > 0:
                f[j] += 1
                drift -= 1
            elif f[j] > 1:
                f[j] -= 1
                drift += 1
            k += 1
        out[r] = f
    return out.astype(np.uint16)


def build_freqs(sym, ctx, n_ctx, n_sym=256):
    """the tables of symbols `sym` in contexts `ctx` (rans.py:15-18)"""
    counts = np.bincount(np.asarray(ctx, np.int64) * n_sym + np.asarray(sym, np.int64), minlength=n_ctx * n_sym)
    return normalize(counts.reshape(n_ctx, n_sym))


def o1_context(sym, period):
    """the previous symbol, 0 at every period-th position (rans.py:141-146)"""
    ctx = np.zeros(len(sym), np.int32)
    ctx[1:] = np.asarray(sym)[:-1]
    ctx[::period] = 0
    return ctx


def _tables(freqs_list):
    freq = np.concatenate([np.asarray(f, np.uint16).reshape(-1, 256) for f in freqs_list])
    cum = np.zeros((len(freq), 257), np.uint32)
    np.cumsum(freq.astype(np.uint32), axis=1, out=cum[:, 1:])
    rows = np.cumsum([0] + [np.asarray(f).shape[0] for f in freqs_list])[:-1]
    return freq, cum, rows


def _check(ctx, freqs, what):
    ctx = np.asarray(ctx)
    f = np.asarray(freqs)
    if f.ndim != 2 or f.shape[1] != 256:
        raise ValueError(f"{what}: tables of 256 symbols per context expected, got {f.shape}")
    if ctx.size and (int(ctx.min()) < 0 or int(ctx.max()) >= f.shape[0]):
        raise ValueError(f"{what}: a context outside the {f.shape[0]} tables")


def encode_many(items, stream=None):
    """[(symbols uint8, contexts, tables)] -> [stream bytes] (rans.encode for each, rans.py:149-152)"""
    if not items:
        return []
    for _, ctx, f in items:
        _check(ctx, f, "encode")
    sym = np.concatenate([np.asarray(s, np.uint8).reshape(-1) for s, _, _ in items])
    ctx = np.concatenate([np.asarray(c, np.int32).reshape(-1) for _, c, _ in items])
    freq, cum, rows = _tables([f for _, _, f in items])
    st = np.zeros(len(items), STREAM)
    at = out_at = 0
    for k, (s, _, _) in enumerate(items):
        n = len(s)
        st[k] = (at, n, at, rows[k], out_at, 0, 0)
        at += n
        out_at += 2 * n + 16
    keep = [dev.DeviceArray.from_host(a if a.size else np.zeros(1, a.dtype), stream) for a in (sym, ctx, freq, cum)]
    st_d = dev.DeviceArray.from_host(st.view(np.uint8), stream)
    out = dev.DeviceArray(max(out_at, 1), np.uint8)
    lens = dev.DeviceArray(len(items), np.uint32)
    check(lib().spa_crans_encode(keep[0].ptr, keep[1].ptr, 256, keep[2].ptr, keep[3].ptr, st_d.ptr, len(items), out.ptr,
                                 lens.ptr, stream))
    ln = lens.to_host(stream=stream)
    host = out.to_host(stream=stream)
    ends = st["out_off"] + 2 * st["n"] + 16
    return [host[int(e) - int(m):int(e)].tobytes() for e, m in zip(ends, ln)]


def decode_many(items, stream=None):
    """[(stream bytes, contexts or None, tables, count, period)] -> [symbols uint8]; period > 0: the
    context is the previous symbol, reset every period symbols (rans.py:152-164)"""
    if not items:
        return []
    for _, ctx, f, n, period in items:
        if period <= 0:
            if ctx is None or len(ctx) != n:
                raise ValueError("decode: a context per symbol expected")
            _check(ctx, f, "decode")
        elif np.asarray(f).shape[0] < 256:
            raise ValueError("decode: an order-1 stream needs a table per previous symbol")
    bufs = [np.frombuffer(bytes(b), np.uint8) for b, _, _, _, _ in items]
    ins = np.concatenate(bufs)
    ctxs = [np.asarray(c, np.int32).reshape(-1) if p <= 0 else np.zeros(0, np.int32) for _, c, _, _, p in items]
    ctx = np.concatenate(ctxs)
    freq, cum, rows = _tables([f for _, _, f, _, _ in items])
    st = np.zeros(len(items), STREAM)
    at = in_at = c_at = 0
    for k, (_, _, _, n, period) in enumerate(items):
        st[k] = (at, n, c_at, rows[k], in_at, max(period, 0), 0)
        at += n
        in_at += len(bufs[k])
        c_at += len(ctxs[k])
    keep = [dev.DeviceArray.from_host(a if a.size else np.zeros(1, a.dtype), stream) for a in (ins, ctx, freq, cum)]
    st_d = dev.DeviceArray.from_host(st.view(np.uint8), stream)
    lut = dev.DeviceArray(len(freq) << PROB_BITS, np.uint8)
    check(lib().spa_rans_build_lut_pb(keep[3].ptr, len(freq), PROB_BITS, lut.ptr, stream))
    out = dev.DeviceArray(max(at, 1), np.uint8)
    check(lib().spa_crans_decode(keep[0].ptr, ins.size, keep[1].ptr, 256, keep[2].ptr, keep[3].ptr, lut.ptr, st_d.ptr,
                                 len(items), out.ptr, stream))
    host = out.to_host(stream=stream)
    return [host[int(o):int(o) + int(n)].copy() for o, n in zip(st["sym_off"], st["n"])]


def encode(sym, ctx, freqs, stream=None):
    return encode_many([(sym, ctx, freqs)], stream)[0]


def decode(buf, ctx, freqs, stream=None):
    return decode_many([(buf, ctx, freqs, len(ctx), 0)], stream)[0]


def decode_o1(buf, n, freqs, period, stream=None):
    return decode_many([(buf, None, freqs, n, period)], stream)[0]
