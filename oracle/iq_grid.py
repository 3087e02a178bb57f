"""ORACLE -- test infrastructure only. Never imported by the product (seedpack_amd/).

ctypes binding of oracle/iq_grid.c, the C restatement of llama.cpp's lattice i-quant quantizers
(IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M; ggml-quants.c:2854-5293), built by
`make -C oracle restatement` into oracle/liboracle_iq.so.

The lattice codebooks (one uint16 per point: 2 or 3 bits per coordinate level) are GGUF format
constants; they are read from the text of seedpack_amd/csrc/iq_grids.h. Everything built from them
here -- points, level-index maps and neighbour lists -- is the restatement's own and is pinned
against the reference fixture's SHA-256 digests (tests/golden/iqtables_sha256.json).
"""
import ctypes
import os
import re
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle_iq.so")
GRIDS_H = os.path.join(os.path.dirname(HERE), "seedpack_amd", "csrc", "iq_grids.h")

TYPES = {16: 0, 17: 1, 22: 3, 18: 4, 21: 5, 19: 2, 29: 2}     # ggml type -> lattice
BS = {16: 66, 17: 74, 22: 82, 18: 98, 21: 110, 19: 50, 29: 56}

_lib = None
_ready = set()
_lock = threading.Lock()


class Planted:
    """A separately built copy of the restatement (oracle/iq_grid.c compiled with -DOG_PLANT=k into
    `path`), for the tests that check a planted mistake fails the golden vectors."""

    def __init__(self, path):
        self.L = ctypes.CDLL(path)
        self.L.og_lattice_init.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        self.L.og_quantize.restype = ctypes.c_int64
        self.L.og_quantize.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_void_p]
        for li, cb in codebooks().items():
            assert self.L.og_lattice_init(li, cb.ctypes.data, cb.size) == 0

    def quantize(self, ttype, x, imatrix=None, variant=0):
        return _run(self.L, ttype, x, imatrix, variant)


def codebooks():
    """{lattice index: uint16 array} parsed from iq_grids.h (IQ_GRID_<i>[n] = { ... };)"""
    text = open(GRIDS_H).read()
    out = {}
    for m in re.finditer(r"IQ_GRID_(\d)\[(\d+)\]\s*=\s*\{([^}]*)\}", text):
        v = np.array([int(t) for t in m.group(3).replace("\n", " ").split(",") if t.strip()], np.uint16)
        assert v.size == int(m.group(2))
        out[int(m.group(1))] = v
    return out


def lib():
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB):
                raise RuntimeError(f"{LIB} is missing: run `make -C oracle restatement`")
            L = ctypes.CDLL(LIB)
            L.og_lattice_init.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
            L.og_lattice_table.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 6
            L.og_quantize.restype = ctypes.c_int64
            L.og_quantize.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_int64, ctypes.c_void_p]
            L.og_half_bits.restype = ctypes.c_uint16
            L.og_half_bits.argtypes = [ctypes.c_float]
            _lib = L
        return _lib


def _init(li):
    L = lib()
    with _lock:
        if li not in _ready:
            cb = codebooks()[li]
            if L.og_lattice_init(li, cb.ctypes.data, cb.size) != 0:
                raise RuntimeError(f"oracle: lattice {li} did not build")
            _ready.add(li)


def table(li):
    """(points uint8 [npts * dim], map int32, neighbour lists uint16) of lattice li"""
    _init(li)
    pt, pn, mp, mn, nb, nn = (ctypes.c_void_p(), ctypes.c_int(), ctypes.c_void_p(), ctypes.c_int(),
                              ctypes.c_void_p(), ctypes.c_int())
    rc = lib().og_lattice_table(li, ctypes.byref(pt), ctypes.byref(pn), ctypes.byref(mp), ctypes.byref(mn),
                                ctypes.byref(nb), ctypes.byref(nn))
    assert rc == 0
    a = np.ctypeslib.as_array(ctypes.cast(pt, ctypes.POINTER(ctypes.c_uint8)), (pn.value,)).copy()
    m = np.ctypeslib.as_array(ctypes.cast(mp, ctypes.POINTER(ctypes.c_int32)), (mn.value,)).copy()
    n = np.ctypeslib.as_array(ctypes.cast(nb, ctypes.POINTER(ctypes.c_uint16)), (nn.value,)).copy()
    return a, m, n


def half_bits(v):
    return lib().og_half_bits(float(v))


def quantize(ttype, x, imatrix=None, variant=0):
    """float32 (nrows, n_per_row) -> quantized bytes (uint8), as quantize_<type>(x, dst, nrows,
    n_per_row, imatrix); raises where the reference aborts"""
    if ttype not in TYPES:
        raise NotImplementedError(f"oracle: type {ttype}")
    _init(TYPES[ttype])
    return _run(lib(), ttype, x, imatrix, variant)


def _run(L, ttype, x, imatrix, variant):
    x = np.ascontiguousarray(x, np.float32)
    assert x.ndim == 2 and x.shape[1] % 256 == 0
    w = None if imatrix is None else np.ascontiguousarray(imatrix, np.float32)
    assert w is None or w.size == x.shape[1]
    out = np.zeros(x.shape[0] * (x.shape[1] // 256) * BS[ttype], np.uint8)
    n = L.og_quantize(ttype, variant, x.ctypes.data, out.ctypes.data, x.shape[0], x.shape[1],
                          None if w is None else w.ctypes.data)
    if n != out.size:
        raise ValueError(f"oracle: quantize type {ttype} variant {variant} aborts (as the reference does)")
    return out
