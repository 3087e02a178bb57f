"""Difference residual of a quantized file against its regrown prediction, on the device.

Host side of SeedPack's residual stage (seedpack/repo3.py:691-700 _kind, :1861-1867 _v0, :1071-1188
_residual_tensors) over the HIP C ABI: the prediction never leaves the GPU; XOR, comparison and
byte-difference counts run as kernels (spa_xor / spa_xor3 / spa_diff_count), and only the counts
come back to the host, which makes the same decisions as the reference:

  * kind: a float tensor of the file is predicted by converting the base ('xor'); a quantized one
    by requantizing the base ('rq'); anything else is not predicted (None);
  * variant: first v0 (unit importance weights, UNIT_W, when the repository has no imatrix for the
    tensor; a fitted importance set k * RECOV; else 0), then, if a residual is left, the candidates
    (the quantizer's code variants, and the unweighted path for unit weights / fitted sets), the
    first with the fewest differing bytes winning;
  * a QR-coded tensor keeps its file bytes and best prediction for the QR coder; an XOR tensor
    keeps file ^ prediction in place; an exact prediction leaves an all-zero XOR residual.
"""
import collections
import threading

import numpy as np

from . import device as dev
from ._lib import check, lib
from .gpuquant import GPUQuant
from .qr import QR_TYPES, SELF_TYPES as QR_SELF_TYPES
from .requant import QFUN, VARIANTS

F32, F16, BF16 = 0, 1, 30
FLOAT_TYPES = (F32, F16, BF16)
SEED_TYPES = QR_SELF_TYPES | {F32, F16, BF16}   # base tensor types the QR coder takes as seeds (qr.py:41)
UNIT_W = 100                                     # variant offset: unit importance weights (repo3.py:540)
RECOV = 1000                                     # variant k * RECOV + v: fitted importance set k (repo3.py:541)


def kind(base_type, base_numel, t_type, t_numel, t_nbytes):
    """how a file tensor is predicted from its base tensor: 'rq', 'xor' or None (repo3.py:691-700)"""
    if base_type is None or not (base_type in FLOAT_TYPES or base_type in QFUN) or base_numel != t_numel:
        return None
    if t_type in FLOAT_TYPES:
        return "xor"
    if t_type in QFUN and t_nbytes == t_numel // QFUN[t_type][1] * QFUN[t_type][2]:
        return "rq"
    return None


def v0(k, has_imatrix, fitted_set=0, in_fitted_set=False):
    """the variant a tensor is first predicted with (repo3.py:1861-1867)"""
    if k == "rq" and fitted_set and in_fitted_set:
        return fitted_set * RECOV
    return UNIT_W if k == "rq" and not has_imatrix else 0


def n_variants(t_type):
    """the quantizer's code variants besides the current one"""
    return VARIANTS.get(t_type, 1) - 1


def candidates(t_type, first):
    """the other predictions worth trying when `first` leaves a residual (repo3.py:1100-1109)"""
    nv = n_variants(t_type)
    out = [first + j for j in range(1, nv + 1)]
    if first == UNIT_W and t_type < 16:
        out += list(range(nv + 1))
    if first >= RECOV:
        out += list(range(nv + 1))
    return out


def split_variant(v):
    """variant number -> (fitted importance set k, unit weights?, quantizer code variant)
    (repo3.py:849-853)"""
    k, u = divmod(v, RECOV)
    return k, (k == 0 and u >= UNIT_W), u % UNIT_W


_TLS = threading.local()


class _Count:
    """a device u64 counter and its read-back. One counter per thread and device, reused: each use
    ends with the read-back, and freeing a device allocation waits for the whole device (work other
    threads queued on other streams included)."""

    def __init__(self):
        cache = getattr(_TLS, "counters", None)
        if cache is None:
            cache = _TLS.counters = {}
        key = dev.current_device()
        if key not in cache:
            cache[key] = dev.DeviceArray(1, np.uint64)
        self.d = cache[key]

    def value(self, stream=None):
        return int(self.d.to_host(stream=stream)[0])


def xor_into(dst, a, b, stream=None):
    """dst = a ^ b (device arrays of equal byte size) -> non-zero bytes of dst"""
    c = _Count()
    check(lib().spa_xor(dst.ptr, a.ptr, b.ptr, a.nbytes, c.d.ptr, stream))
    return c.value(stream)


def xor3_into(dst, a, b, c_, stream=None):
    c = _Count()
    check(lib().spa_xor3(dst.ptr, a.ptr, b.ptr, c_.ptr, a.nbytes, c.d.ptr, stream))
    return c.value(stream)


def diff_count(a, b=None, stream=None):
    """bytes where a and b differ (b None: non-zero bytes of a)"""
    c = _Count()
    check(lib().spa_diff_count(a.ptr, None if b is None else b.ptr, a.nbytes, c.d.ptr, stream))
    return c.value(stream)


def float_prediction(src, t_type, stream=None):
    """a float file tensor's prediction from the base weights src (DeviceArray of bf16 bits / f16 /
    f32) as the bytes of type t_type (F32, F16 or BF16)"""
    from .gpuquant import _src_kind
    isz = 4 if t_type == F32 else 2
    out = dev.DeviceArray(src.size * isz, np.uint8)
    check(lib().spa_float_pred(src.ptr, _src_kind(src), src.size, t_type, out.ptr, stream))
    return out


class Tensor:
    """a file tensor for the residual stage: its type, weights per row and file region on the device
    (modified in place); `base` the base weights (DeviceArray), `imatrix` the repository's
    importance (numpy float32 per column or None), `fitted` {set k: importance} of fitted sets"""

    def __init__(self, name, t_type, cols, region, base, imatrix=None, fitted=None, base_type=BF16, numel=None):
        self.name, self.type, self.cols, self.region, self.base = name, t_type, cols, region, base
        self.imatrix, self.fitted, self.base_type = imatrix, fitted or {}, base_type
        self.numel = base.size if numel is None else numel      # the file tensor's element count


def predict(gq, t, v, stream=None):
    """prediction of tensor t with variant v (repo3.py:845-855) as a device array"""
    if t.type in FLOAT_TYPES:
        return float_prediction(t.base, t.type, stream)
    k, unit, code_variant = split_variant(v)
    imx = t.fitted[k] if k else (np.ones(t.cols, np.float32) if unit else t.imatrix)
    return gq.quantize_tensors(t.type, [(t.base, t.cols)], [imx], code_variant, device=True)[0]


def _first(t, gq, fitted_set, use_qr, stream, count_ptr):
    """the tensor's kind and first prediction, its differing-byte count written to count_ptr
    (device u64) without waiting -> (kind, first variant, QR?, prediction) or None if not predicted"""
    k = kind(t.base_type, t.base.size, t.type, t.numel, t.region.nbytes)
    if k is None:
        return None
    first = v0(k, t.imatrix is not None, fitted_set, fitted_set in t.fitted)
    isqr = use_qr and k == "rq" and t.type in QR_TYPES and t.base_type in SEED_TYPES
    p0 = predict(gq, t, first, stream)
    if isqr:
        check(lib().spa_diff_count(t.region.ptr, p0.ptr, t.region.nbytes, count_ptr, stream))
    else:
        check(lib().spa_xor(t.region.ptr, t.region.ptr, p0.ptr, t.region.nbytes, count_ptr, stream))
    return k, first, isqr, p0


def _decide(t, gq, k, first, isqr, p0, n0, stream):
    """the candidate variants after a first prediction leaving n0 differing bytes, and the result"""
    choice, best, best_p = first, n0, p0
    cands = candidates(t.type, first) if k == "rq" else []
    if n0 and cands:
        # the region now holds the file (QR) or file ^ p0 (XOR); prediction pv leaves
        # file ^ pv = region ^ p0 ^ pv
        tmp = None if isqr else dev.DeviceArray(t.region.nbytes, np.uint8)
        best_x = None
        for v in sorted(set(cands)):
            pv = predict(gq, t, v, stream)
            if isqr:
                e = diff_count(t.region, pv, stream)
            else:
                e = xor3_into(tmp, t.region, p0, pv, stream)
            if e < best:                          # the first of the fewest differing bytes wins
                choice, best, best_p = v, e, pv
                if not isqr:
                    best_x, tmp = tmp, dev.DeviceArray(t.region.nbytes, np.uint8)
        if best_x is not None:
            check(lib().spa_memcpy_d2d(t.region.ptr, best_x.ptr, t.region.nbytes, stream))
    nonzero = best > 0
    if isqr and not nonzero:                      # exact: the XOR residual, all zero
        check(lib().spa_memset(t.region.ptr, 0, t.region.nbytes, stream))
        isqr = False
    return {"kind": "qr" if isqr else k, "variant": choice, "nonzero": nonzero, "qr": isqr,
            "prediction": best_p if isqr else None, "diff_bytes": best}


_NONE = {"kind": None, "variant": None, "nonzero": True, "qr": False, "prediction": None}


def residual_tensor(t, gq=None, fitted_set=0, use_qr=True, stream=None):
    """the residual of one tensor (the per-tensor decisions of repo3.py:1071-1188) ->
    dict(kind, variant, nonzero, qr, prediction). t.region ends as: the file bytes (QR tensors,
    coded against `prediction`), file ^ prediction (XOR tensors) or zeros (exact predictions)."""
    gq = gq or GPUQuant(stream=stream)
    c = _Count()
    f = _first(t, gq, fitted_set, use_qr, stream, c.d.ptr)
    if f is None:
        return dict(_NONE)
    return _decide(t, gq, *f, c.value(stream), stream)


def _staged(n):
    """a page-locked uint64 array of at least n items for this thread (returned with _unstage)"""
    pool = getattr(_TLS, "staged", None)
    if pool is None:
        pool = _TLS.staged = []
    for k, a in enumerate(pool):
        if a.size >= n:
            return pool.pop(k)
    return dev.pinned(max(64, 2 * n), np.uint64)


def _unstage(a):
    _TLS.staged.append(a)


def _read_counts(counts, n, stream):
    """counts[:n] copied to the host behind the work queued so far -> (host array, event)"""
    host = _staged(n)
    if n:
        check(lib().spa_memcpy_d2h_async(host.ctypes.data, counts.ptr, 8 * n, stream))
    ev = dev.Event()
    ev.record(stream)
    return host, ev


def residual_window_start(ts, gq=None, fitted_set=0, use_qr=True, stream=None):
    """the first predictions of a window of tensors and their byte counts queued back to back (the
    reference's window pipeline defers its comparisons, repo3.py:456-510), the counts' read-back
    queued behind them; nothing is waited for -> the state residual_window_finish completes"""
    gq = gq or GPUQuant(stream=stream)
    counts = dev.DeviceArray(max(64, 2 * len(ts)), np.uint64)
    firsts = [_first(t, gq, fitted_set, use_qr, stream, counts.ptr + 8 * i) for i, t in enumerate(ts)]
    host, ev = _read_counts(counts, len(ts), stream)
    return {"ts": ts, "gq": gq, "stream": stream, "counts": counts, "firsts": firsts, "host": host, "ev": ev}


def residual_window_finish(st):
    """residual_tensor's results for the window residual_window_start queued, in the order of its
    tensors: its counts waited for (one wait), the QR tensors' other candidates predicted and counted
    before one more wait"""
    ts, gq, stream, counts, firsts = st["ts"], st["gq"], st["stream"], st["counts"], st["firsts"]
    st["ev"].synchronize()
    n = st["host"][:len(ts)].copy()
    _unstage(st["host"])
    tried = collections.defaultdict(list)
    for i, (t, f) in enumerate(zip(ts, firsts)):
        if f is not None and f[2] and n[i]:
            tried[i] = [(v, predict(gq, t, v, stream)) for v in sorted(set(candidates(t.type, f[1])))]
    slots = [(i, v, p) for i, vs in tried.items() for v, p in vs]
    if slots:
        if counts.size < len(slots):
            counts = dev.DeviceArray(2 * len(slots), np.uint64)
        for s_, (i, v, p) in enumerate(slots):
            check(lib().spa_diff_count(ts[i].region.ptr, p.ptr, ts[i].region.nbytes, counts.ptr + 8 * s_, stream))
        host, ev = _read_counts(counts, len(slots), stream)
        ev.synchronize()
        e = host[:len(slots)].copy()
        _unstage(host)
        tried = collections.defaultdict(list)
        for s_, (i, v, p) in enumerate(slots):
            tried[i].append((v, p, int(e[s_])))
    out = []
    for i, (t, f) in enumerate(zip(ts, firsts)):
        if f is None:
            out.append(dict(_NONE))
        elif f[2]:
            out.append(_decide_qr(t, f[1], f[3], int(n[i]), tried.get(i, []), stream))
        else:
            out.append(_decide(t, gq, *f, int(n[i]), stream))
    return out


def residual_window(ts, gq=None, fitted_set=0, use_qr=True, stream=None):
    """residual_tensor for a window of tensors with the same decisions -> results in the order of ts"""
    return residual_window_finish(residual_window_start(ts, gq, fitted_set, use_qr, stream))


def _decide_qr(t, first, p0, n0, tried, stream):
    """_decide for a QR tensor whose candidates' differing-byte counts are known: tried [(variant,
    prediction, count)] in variant order"""
    choice, best, best_p = first, n0, p0
    for v, pv, e in tried:
        if e < best:                              # the first of the fewest differing bytes wins
            choice, best, best_p = v, e, pv
    if not best:                                  # exact: the XOR residual, all zero
        check(lib().spa_memset(t.region.ptr, 0, t.region.nbytes, stream))
        return {"kind": "rq", "variant": choice, "nonzero": False, "qr": False, "prediction": None, "diff_bytes": 0}
    return {"kind": "qr", "variant": choice, "nonzero": True, "qr": True, "prediction": best_p, "diff_bytes": best}
