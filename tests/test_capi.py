"""The C-ABI library loads and exports every symbol include/seedpack_amd.h declares (no GPU calls)."""
import ctypes
import os
import re

import pytest

from seedpack_amd import _lib
from seedpack_amd.requant import QFUN

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(spa_\w+)\s*\(", src, re.M))
    return names


def test_header_and_binding_agree():
    assert declared_symbols() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
        assert ctypes.cast(getattr(L, name), ctypes.c_void_p).value


@pytest.mark.parametrize("t", sorted(QFUN))
def test_row_size_matches_type_table(t):
    _, qk, bs = QFUN[t]
    L = _lib.lib()
    assert L.spa_row_size(t, 4096 // qk * qk * 3) == (4096 // qk * 3) * bs
    assert L.spa_row_size(t, qk + 1) == 0


def test_bad_arguments_fail_before_any_device_call():
    L = _lib.lib()
    assert L.spa_quantize(99, 0, None, 0, 1, 256, None, None, None, None) == -2
    assert b"unknown ggml type" in L.spa_last_error()
    assert L.spa_quantize(12, 0, None, 0, 1, 100, None, None, None, None) == -4
    assert L.spa_quantize(12, 1, None, 0, 1, 256, None, None, None, None) == -2       # no variant 1 for Q4_K
    assert L.spa_quantize(16, 0, None, 0, 1, 256, None, None, None, None) == -4       # null src first
    # scratch: one float per row (256-byte rounded) for the imatrix Q4_0/Q4_1/Q5_0/Q5_1, none otherwise
    assert [L.spa_quantize_work_bytes(t, 100, 4096, 1) for t in (2, 3, 6, 7)] == [512] * 4
    assert [L.spa_quantize_work_bytes(t, 100, 4096, 0) for t in (2, 3, 6, 7)] == [0] * 4
    assert [L.spa_quantize_work_bytes(t, 100, 4096, 1) for t in (8, 12, 16, 20)] == [0] * 4
    assert L.spa_type_variants(29) == 2 and L.spa_type_variants(12) == 1 and L.spa_type_variants(99) == 0


def test_noalloc_encoder_rejects_before_any_device_call():
    """a batch whose workspace exceeds the static scratch is refused from its sizes alone"""
    L = _lib.lib()
    scratch = L.spa_qr_noalloc_scratch_bytes()
    assert scratch == 64 << 20
    nseg = 1
    while L.spa_qr_work_bytes(8, nseg) <= scratch:
        nseg *= 2
    assert L.spa_qr_encode_noalloc(8, None, None, None, None, None, nseg, None, None, None, None, 1 << 16, None, None,
                                   None, 2, None) == -4
    assert b"static scratch" in L.spa_last_error()
    assert L.spa_qr_encode_noalloc(99, None, None, None, None, None, 1, None, None, None, None, 1 << 16, None, None,
                                   None, 2, None) == -2


def test_sync_mode_takes_only_its_two_values():
    L = _lib.lib()
    assert L.spa_set_sync_mode(2) == -4 and b"spa_set_sync_mode" in L.spa_last_error()
    assert L.spa_set_sync_mode(0) == 0


def test_crc32_equals_zlib():
    """the host CRC-32 (512-bit folding from 512 bytes where the CPU has it, 128-bit folding from 64
    bytes, a table below) against zlib.crc32: every length to 300 and around the 512-bit path's
    boundaries, odd offsets, chained calls, zeros and a large buffer"""
    import zlib

    import numpy as np

    from seedpack_amd.container import crc32
    g = np.random.Generator(np.random.PCG64(32))
    for n in list(range(301)) + list(range(500, 800)) + [1023, 1024, 1025, 4096 + 17, 1 << 20]:
        b = g.integers(0, 256, n + 5, dtype=np.uint8).tobytes()
        for o in (0, 1, 5):
            piece = b[o:o + n]
            assert crc32(piece) == zlib.crc32(piece), (n, o)
        assert crc32(b[:n], 0x12345678) == zlib.crc32(b[:n], 0x12345678), n
        assert crc32(b[n // 3:n], crc32(b[:n // 3])) == zlib.crc32(b[:n]), n
    z = bytes(3 << 20)
    assert crc32(z) == zlib.crc32(z)
    big = g.integers(0, 256, 24 << 20, dtype=np.uint8)
    assert crc32(big) == zlib.crc32(big.tobytes())
