"""zstd for the archive's parts, through libzstd with ctypes.

The reference uses python-zstandard (seedpack/codecs_gguf.py:72-83, repo3.py:1533-1544,
container.py:106); level-19 output is a function of the library version, so a libzstd 1.5.7 (the
version python-zstandard 0.25 bundles) is preferred when one is installed, else the system libzstd.

compress/decompress: one frame with its content size, as ZstdCompressor(level).compress writes it.
Params + Compressor: a frame from explicit parameters (the level's table entry with overrides: window
log, long-distance matching, worker threads), optionally against a raw-content dictionary, fed in
pieces (the residual of a file). decompress_into: a frame (dictionary optional) into a caller buffer.
"""
import ctypes
import ctypes.util
import glob
import os

import numpy as np

_lib = None

# zstd.h parameter ids (stable API)
C_LEVEL, C_WINDOW_LOG, C_HASH_LOG, C_CHAIN_LOG, C_SEARCH_LOG, C_MIN_MATCH, C_TARGET_LENGTH, C_STRATEGY = \
    100, 101, 102, 103, 104, 105, 106, 107
C_LDM, C_CONTENT_SIZE, C_CHECKSUM, C_DICT_ID, C_WORKERS = 160, 200, 201, 202, 400
D_WINDOW_LOG_MAX = 100
E_CONTINUE, E_END = 0, 2
DLM_BY_COPY, DCT_RAW_CONTENT = 0, 1


class _CParams(ctypes.Structure):
    _fields_ = [("windowLog", ctypes.c_uint), ("chainLog", ctypes.c_uint), ("hashLog", ctypes.c_uint),
                ("searchLog", ctypes.c_uint), ("minMatch", ctypes.c_uint), ("targetLength", ctypes.c_uint),
                ("strategy", ctypes.c_int)]


class _Buf(ctypes.Structure):          # ZSTD_inBuffer / ZSTD_outBuffer: pointer, size, position
    _fields_ = [("ptr", ctypes.c_void_p), ("size", ctypes.c_size_t), ("pos", ctypes.c_size_t)]


def _candidates():
    here = []
    for d in ("/usr/local/lib/python3.10/dist-packages/pillow.libs", "/usr/lib/python3/dist-packages/pillow.libs"):
        here += sorted(glob.glob(os.path.join(d, "libzstd*.so*")))
    sysl = ctypes.util.find_library("zstd")
    return here + ([sysl] if sysl else []) + ["libzstd.so.1"]


def _sig(L, name, res, args):
    f = getattr(L, name)
    f.restype, f.argtypes = res, args


def lib():
    global _lib
    if _lib is None:
        err = None
        for p in _candidates():
            try:
                # a second libzstd may already be in the global scope (profilers and runtimes link
                # the system one): bind this copy's internal calls to itself, or its entry points
                # call into the other version's functions with this version's structures
                L = ctypes.CDLL(p, mode=os.RTLD_LOCAL | getattr(os, "RTLD_DEEPBIND", 0))
                break
            except OSError as e:
                err = e
        else:
            raise RuntimeError(f"no libzstd found: {err}")
        vp, sz, ci = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        _sig(L, "ZSTD_compress", sz, [vp, sz, vp, sz, ci])
        _sig(L, "ZSTD_compressBound", sz, [sz])
        _sig(L, "ZSTD_decompress", sz, [vp, sz, vp, sz])
        _sig(L, "ZSTD_getFrameContentSize", ctypes.c_ulonglong, [vp, sz])
        _sig(L, "ZSTD_isError", ctypes.c_uint, [sz])
        _sig(L, "ZSTD_getErrorName", ctypes.c_char_p, [sz])
        _sig(L, "ZSTD_versionNumber", ctypes.c_uint, [])
        _sig(L, "ZSTD_getCParams", _CParams, [ci, ctypes.c_ulonglong, sz])
        _sig(L, "ZSTD_createCCtx", vp, [])
        _sig(L, "ZSTD_freeCCtx", sz, [vp])
        _sig(L, "ZSTD_CCtx_setParameter", sz, [vp, ci, ci])
        _sig(L, "ZSTD_CCtx_setPledgedSrcSize", sz, [vp, ctypes.c_ulonglong])
        _sig(L, "ZSTD_CCtx_loadDictionary_advanced", sz, [vp, vp, sz, ci, ci])
        _sig(L, "ZSTD_compressStream2", sz, [vp, ctypes.POINTER(_Buf), ctypes.POINTER(_Buf), ci])
        _sig(L, "ZSTD_createDCtx", vp, [])
        _sig(L, "ZSTD_freeDCtx", sz, [vp])
        _sig(L, "ZSTD_DCtx_setParameter", sz, [vp, ci, ci])
        _sig(L, "ZSTD_DCtx_loadDictionary_advanced", sz, [vp, vp, sz, ci, ci])
        _sig(L, "ZSTD_decompressStream", sz, [vp, ctypes.POINTER(_Buf), ctypes.POINTER(_Buf)])
        _sig(L, "ZSTD_decompressDCtx", sz, [vp, vp, sz, vp, sz])
        _lib = L
    return _lib


def _ok(n, what):
    if lib().ZSTD_isError(n):
        raise RuntimeError(f"{what}: {lib().ZSTD_getErrorName(n).decode()}")
    return n


def version():
    v = lib().ZSTD_versionNumber()
    return f"{v // 10000}.{v // 100 % 100}.{v % 100}"


def _addr(buf):
    """(address, size) of a contiguous bytes-like object (read only is fine)"""
    a = np.frombuffer(buf, np.uint8) if not isinstance(buf, np.ndarray) else buf.reshape(-1).view(np.uint8)
    return (a.ctypes.data if a.size else None), a.size, a


def compress(data, level=19):
    """one frame with its content size, the level's parameters (ZstdCompressor(level).compress)"""
    L = lib()
    p, n, keep = _addr(data)
    cap = L.ZSTD_compressBound(n)
    out = np.empty(max(1, cap), np.uint8)
    k = _ok(L.ZSTD_compress(out.ctypes.data, cap, p, n, level), "ZSTD_compress")
    return out[:k].tobytes()


def decompress(data):
    data = bytes(data)
    L = lib()
    size = L.ZSTD_getFrameContentSize(data, len(data))
    if size >= (1 << 63):
        raise RuntimeError("zstd frame without a content size")
    out = ctypes.create_string_buffer(max(1, size))
    n = _ok(L.ZSTD_decompress(out, size, data, len(data)), "ZSTD_decompress")
    if n != size:
        raise RuntimeError("ZSTD_decompress: short frame")
    return out.raw[:n]


class Params:
    """compression parameters: the level's table entry (ZSTD_getCParams), then the overrides, set one
    by one (as ZstdCompressionParameters.from_level(level, window_log=..., threads=...,
    enable_ldm=...) does)"""

    def __init__(self, level, window_log=None, threads=0, ldm=False):
        self.level, self.window_log, self.threads, self.ldm = level, window_log, threads, ldm

    def apply(self, cctx):
        L = lib()
        cp = L.ZSTD_getCParams(self.level, 0, 0)
        vals = [(C_WINDOW_LOG, self.window_log or cp.windowLog), (C_CHAIN_LOG, cp.chainLog), (C_HASH_LOG, cp.hashLog),
                (C_SEARCH_LOG, cp.searchLog), (C_MIN_MATCH, cp.minMatch), (C_TARGET_LENGTH, cp.targetLength),
                (C_STRATEGY, cp.strategy), (C_CONTENT_SIZE, 1), (C_CHECKSUM, 0), (C_DICT_ID, 1)]
        if self.threads:
            vals.append((C_WORKERS, self.threads if self.threads > 0 else os.cpu_count() or 1))
        if self.ldm:
            vals.append((C_LDM, 1))
        for k, v in vals:
            _ok(L.ZSTD_CCtx_setParameter(cctx, k, int(v)), f"ZSTD_CCtx_setParameter({k})")


class Compressor:
    """one frame written in pieces: compress(bytes-like) -> the frame bytes produced so far, finish()
    -> the rest. size: the total input (written into the frame header); dict_data: raw-content
    dictionary (the bytes the frame's matches may also refer to)"""

    OUT = 1 << 22

    def __init__(self, params, dict_data=None, size=None):
        L = lib()
        self.cctx = L.ZSTD_createCCtx()
        if not self.cctx:
            raise MemoryError("ZSTD_createCCtx")
        params.apply(self.cctx)
        if dict_data is not None and len(dict_data):
            self._dict = bytes(dict_data)
            _ok(L.ZSTD_CCtx_loadDictionary_advanced(self.cctx, self._dict, len(self._dict), DLM_BY_COPY,
                                                    DCT_RAW_CONTENT), "load dictionary")
        if size is not None:
            _ok(L.ZSTD_CCtx_setPledgedSrcSize(self.cctx, int(size)), "pledged size")
        self._out = np.empty(self.OUT, np.uint8)

    def _run(self, data, mode):
        L = lib()
        p, n, keep = _addr(data) if data is not None else (None, 0, None)
        inb = _Buf(p, n, 0)
        pieces = []
        while True:
            outb = _Buf(self._out.ctypes.data, self.OUT, 0)
            left = _ok(L.ZSTD_compressStream2(self.cctx, ctypes.byref(outb), ctypes.byref(inb), mode),
                       "ZSTD_compressStream2")
            if outb.pos:
                pieces.append(self._out[:outb.pos].tobytes())
            if mode == E_END:
                if left == 0:
                    break
            elif inb.pos == inb.size:
                break
        return b"".join(pieces)

    def compress(self, data):
        return self._run(data, E_CONTINUE)

    def finish(self):
        out = self._run(None, E_END)
        lib().ZSTD_freeCCtx(self.cctx)
        self.cctx = None
        return out

    def __del__(self):
        if getattr(self, "cctx", None):
            lib().ZSTD_freeCCtx(self.cctx)


def zstd_c(data, level=19):
    """the reference's codecs_gguf.zstd_c (codecs_gguf.py:72-79): small data with the level's
    parameters; above 8 MiB a 2^27 window, long-distance matching and worker threads"""
    if memoryview(data).nbytes <= (8 << 20):
        return compress(data, level)
    return compress_with(data, Params(level, window_log=27, threads=max(1, os.cpu_count() or 1), ldm=True))


def compress_with(data, params, dict_data=None):
    """one frame of `data` with explicit parameters (and dictionary)"""
    c = Compressor(params, dict_data, size=memoryview(data).nbytes)
    return c.compress(data) + c.finish()


def decompress_into(data, out, dict_data=None):
    """the frame in `data` decoded into the writable uint8 array `out` (exactly its size) -> out"""
    L = lib()
    dctx = L.ZSTD_createDCtx()
    if not dctx:
        raise MemoryError("ZSTD_createDCtx")
    try:
        _ok(L.ZSTD_DCtx_setParameter(dctx, D_WINDOW_LOG_MAX, 31), "window log max")
        if dict_data is not None and len(dict_data):
            d = bytes(dict_data)
            _ok(L.ZSTD_DCtx_loadDictionary_advanced(dctx, d, len(d), DLM_BY_COPY, DCT_RAW_CONTENT), "load dictionary")
        p, n, keep = _addr(data)
        if out.size and L.ZSTD_getFrameContentSize(p, n) == out.size:
            # a frame that records its size: decoded in one call straight into `out` (no window
            # buffer, no copy out of it; the loaded dictionary applies)
            r = L.ZSTD_decompressDCtx(dctx, out.ctypes.data, out.size, p, n)
            if L.ZSTD_isError(r):
                raise ValueError(f"zstd frame: {L.ZSTD_getErrorName(r).decode()}")
            if r != out.size:
                raise ValueError(f"zstd frame decodes to {r} bytes, {out.size} expected")
            return out
        inb = _Buf(p, n, 0)
        step = 1 << 28
        o = 0
        while True:
            outb = _Buf(out.ctypes.data + o if out.size else None, min(step, out.size - o), 0)
            before = inb.pos
            r = _ok(L.ZSTD_decompressStream(dctx, ctypes.byref(outb), ctypes.byref(inb)), "ZSTD_decompressStream")
            o += outb.pos
            if r == 0:
                break
            if outb.pos == 0 and inb.pos == before:
                # no progress: the output is full (a longer frame) or the input is used up (truncated)
                if o == out.size:
                    raise ValueError(f"zstd frame decodes to more than {out.size} bytes")
                raise ValueError(f"zstd frame truncated after {o} bytes")
        if o != out.size:
            raise ValueError(f"zstd frame decodes to {o} bytes, {out.size} expected")
        return out
    finally:
        L.ZSTD_freeDCtx(dctx)
