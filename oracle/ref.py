"""ORACLE -- test infrastructure only. ctypes binding of the reference's own llama.cpp quantizers,
compiled from /root/reference/seedpack/ggml by oracle/Makefile into oracle/_ref/.

quantize() follows the reference's CPU entry (seedpack/requant.py:115-134): rows split into
contiguous chunks over a thread pool, each chunk one quantize_<type>(src, dst, nrow, n_per_row,
imatrix) call; IQ tables are initialised first (requant.py:28-29, :48-56). dequantize() runs
dequantize_row_<type> (ggml-quants.c:439-2764) over the whole run of blocks.
"""
import ctypes
import os
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")
LIBS = {0: os.path.join(REF_DIR, "libggmlq_ref.so"), 1: os.path.join(REF_DIR, "libggmlq_ref_v1.so")}

QFUN = {2: "quantize_q4_0", 3: "quantize_q4_1", 6: "quantize_q5_0", 7: "quantize_q5_1", 8: "quantize_q8_0",
        10: "quantize_q2_K", 11: "quantize_q3_K", 12: "quantize_q4_K", 13: "quantize_q5_K", 14: "quantize_q6_K",
        16: "quantize_iq2_xxs", 17: "quantize_iq2_xs", 18: "quantize_iq3_xxs", 19: "quantize_iq1_s",
        20: "quantize_iq4_nl", 21: "quantize_iq3_s", 22: "quantize_iq2_s", 23: "quantize_iq4_xs",
        29: "quantize_iq1_m", 42: "quantize_q2_0"}
QK = {2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 10: 256, 11: 256, 12: 256, 13: 256, 14: 256, 16: 256, 17: 256,
      18: 256, 19: 256, 20: 32, 21: 256, 22: 256, 23: 256, 29: 256, 42: 64}
BS = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 16: 66, 17: 74,
      18: 98, 19: 50, 20: 18, 21: 110, 22: 82, 23: 136, 29: 56, 42: 18}
IQ2_INIT = {16, 17, 19, 22, 29}
IQ3_INIT = {18: 256, 21: 512}

_libs = {}
_inited = set()
_lock = threading.Lock()


def available(variant=0):
    return os.path.exists(LIBS[variant])


def lib(variant=0):
    with _lock:
        if variant not in _libs:
            if not available(variant):
                raise RuntimeError(f"{LIBS[variant]} is missing: run `make -C oracle` where /root/reference exists")
            L = ctypes.CDLL(LIBS[variant])
            for name in QFUN.values():
                f = getattr(L, name)
                f.restype = ctypes.c_size_t
                f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
            L.iq2xs_init_impl.argtypes = [ctypes.c_int]
            L.iq3xs_init_impl.argtypes = [ctypes.c_int]
            _libs[variant] = L
        return _libs[variant]


def _init(t, variant):
    L = lib(variant)
    with _lock:
        if (t, variant) in _inited:
            return
        if t in IQ2_INIT:
            L.iq2xs_init_impl(t)
        if t in IQ3_INIT:
            L.iq3xs_init_impl(IQ3_INIT[t])
        _inited.add((t, variant))


def quantize(ttype, x, imatrix=None, variant=0, threads=None):
    """float32 (nrows, n_per_row) -> quantized bytes (uint8), via the reference C build"""
    _init(ttype, variant)
    if ttype == 42:
        # Q2_0 ignores the imatrix (ggml-quants.c:2114-2127), but the CPU library's stubs.c type table
        # (stubs.c:6-16) has no Q2_0 row size, so its imatrix branch reads past the table. The
        # reference GPU path generates a correct ggml_row_size (gpuquant.py:224-231); the NULL entry
        # runs the same per-block function over the whole tensor.
        imatrix = None
    x = np.ascontiguousarray(x, np.float32)
    nrows, npr = x.shape
    rb = npr // QK[ttype] * BS[ttype]
    out = np.empty(nrows * rb, np.uint8)
    imp = None if imatrix is None else np.ascontiguousarray(imatrix, np.float32)
    f = getattr(lib(variant), QFUN[ttype])
    threads = threads or os.cpu_count() or 1
    chunk = max(1, (nrows + threads * 4 - 1) // (threads * 4))

    def run(r0):
        r1 = min(nrows, r0 + chunk)
        f(x[r0:r1].ctypes.data, out[r0 * rb:r1 * rb].ctypes.data, r1 - r0, npr,
          None if imp is None else imp.ctypes.data)

    if threads == 1:
        for r0 in range(0, nrows, chunk):
            run(r0)
    else:
        with ThreadPoolExecutor(threads) as ex:
            list(ex.map(run, range(0, nrows, chunk)))
    return out


def dequantize(ttype, blocks, n):
    """quantized bytes (a run of blocks holding n weights) -> float32[n], via the reference C build"""
    b = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8))
    assert n % QK[ttype] == 0 and len(b) >= n // QK[ttype] * BS[ttype]
    L = lib(0)
    f = getattr(L, "de" + QFUN[ttype].replace("quantize_", "quantize_row_"))
    f.restype = None
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    out = np.empty(n, np.float32)
    f(b.ctypes.data, out.ctypes.data, n)
    return out
