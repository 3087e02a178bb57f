"""zstd framing of the small coded parts (frequency tables, segment lengths), through libzstd with
ctypes. The reference uses python-zstandard (seedpack/codecs_gguf.py:72-83); level-19 output is a
function of the library version, so a libzstd 1.5.7 (the version python-zstandard 0.25 bundles) is
preferred when one is installed, else the system libzstd."""
import ctypes
import ctypes.util
import glob
import os

_lib = None


def _candidates():
    here = []
    for d in ("/usr/local/lib/python3.10/dist-packages/pillow.libs", "/usr/lib/python3/dist-packages/pillow.libs"):
        here += sorted(glob.glob(os.path.join(d, "libzstd*.so*")))
    sysl = ctypes.util.find_library("zstd")
    return here + ([sysl] if sysl else []) + ["libzstd.so.1"]


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
        L.ZSTD_compress.restype = ctypes.c_size_t
        L.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        L.ZSTD_compressBound.restype = ctypes.c_size_t
        L.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        L.ZSTD_decompress.restype = ctypes.c_size_t
        L.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t]
        L.ZSTD_getFrameContentSize.restype = ctypes.c_ulonglong
        L.ZSTD_getFrameContentSize.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        L.ZSTD_isError.restype = ctypes.c_uint
        L.ZSTD_isError.argtypes = [ctypes.c_size_t]
        L.ZSTD_versionNumber.restype = ctypes.c_uint
        _lib = L
    return _lib


def version():
    v = lib().ZSTD_versionNumber()
    return f"{v // 10000}.{v // 100 % 100}.{v % 100}"


def compress(data, level=19):
    data = bytes(data)
    L = lib()
    cap = L.ZSTD_compressBound(len(data))
    out = ctypes.create_string_buffer(cap)
    n = L.ZSTD_compress(out, cap, data, len(data), level)
    if L.ZSTD_isError(n):
        raise RuntimeError("ZSTD_compress failed")
    return out.raw[:n]


def decompress(data):
    data = bytes(data)
    L = lib()
    size = L.ZSTD_getFrameContentSize(data, len(data))
    if size >= (1 << 63):
        raise RuntimeError("zstd frame without a content size")
    out = ctypes.create_string_buffer(max(1, size))
    n = L.ZSTD_decompress(out, size, data, len(data))
    if L.ZSTD_isError(n) or n != size:
        raise RuntimeError("ZSTD_decompress failed")
    return out.raw[:n]
