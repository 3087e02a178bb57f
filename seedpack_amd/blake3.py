"""BLAKE3 digests on the device and on the host, through the library (spa_blake3, spa_b3h_*).

The reference computes BLAKE3 with the blake3 package: the catalog's file checksums when it is
installed (cli.py:34-53, the normal case) and the keys by which a tensor is found equal to one of an
earlier file (repo3.py:529, :1029, :2018-2022; siblings.py:216-240). Here the tensors and files that
are on the device are hashed there (regions of one buffer in a few launches); host data that is
checked as it is written goes through the incremental host hasher.
"""
import ctypes
import os

import numpy as np

from . import device as dev
from ._lib import check, lib

THREADS = min(16, os.cpu_count() or 1)


def device_digests(base, regions, stream=None):
    """32-byte digests of the byte regions [(offset, length)] of the device array `base`"""
    if not regions:
        return []
    reg = np.ascontiguousarray(np.array(regions, np.uint64).reshape(-1))
    n = len(regions)
    need = lib().spa_blake3_work_bytes(reg.ctypes.data, n)
    work = dev.DeviceArray(max(int(need), 1), np.uint8)
    out = np.empty(32 * n, np.uint8)
    check(lib().spa_blake3(base.ptr if base is not None else None, reg.ctypes.data, n, work.ptr, work.nbytes,
                           out.ctypes.data, stream))
    return [out[32 * i:32 * i + 32].tobytes() for i in range(n)]


def device_hexdigest(d, nbytes=None, stream=None):
    """hex digest of the first `nbytes` bytes (default: all) of the device array d"""
    n = d.nbytes if nbytes is None else int(nbytes)
    return device_digests(d, [(0, n)], stream)[0].hex()


class Hasher:
    """incremental host BLAKE3 (blake3.blake3().update(...).hexdigest() of the reference); pieces are
    fed in order, large ones on several threads"""

    def __init__(self, data=None, threads=THREADS):
        p = ctypes.c_void_p()
        check(lib().spa_b3h_new(ctypes.byref(p)))
        self._h, self.threads = p.value, threads
        if data is not None:
            self.update(data)

    def update(self, data):
        mv = memoryview(data).cast("B")
        if mv.nbytes:
            buf = np.frombuffer(mv, np.uint8)
            check(lib().spa_b3h_update(self._h, buf.ctypes.data, buf.nbytes, self.threads))
        return self

    def digest(self):
        out = np.empty(32, np.uint8)
        check(lib().spa_b3h_final(self._h, out.ctypes.data))
        return out.tobytes()

    def hexdigest(self):
        return self.digest().hex()

    def __del__(self):
        if getattr(self, "_h", None):
            try:
                lib().spa_b3h_free(self._h)
            except Exception:
                pass
            self._h = None


def hexdigest(data, threads=THREADS):
    """hex BLAKE3 of a host buffer"""
    return Hasher(data, threads).hexdigest()
