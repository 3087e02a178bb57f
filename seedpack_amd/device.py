"""Device memory, streams and events over the library's own HIP runtime (no framework needed).

DeviceArray is the minimal device array the host layer passes around: a HIP allocation with a
dtype and a shape. It plays the role CuPy arrays play in the reference (seedpack/xp.py:6-18).
"""
import ctypes

import numpy as np

from ._lib import check, lib


class DeviceArray:
    __slots__ = ("ptr", "nbytes", "dtype", "shape", "_owner")

    def __init__(self, shape, dtype, ptr=None, owner=None):
        self.dtype = np.dtype(dtype)
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        if ptr is None:
            p = ctypes.c_void_p()
            check(lib().spa_malloc(ctypes.byref(p), self.nbytes))
            self.ptr, self._owner = p.value, None
        else:
            self.ptr, self._owner = ptr, owner if owner is not None else self

    @property
    def size(self):
        return self.nbytes // self.dtype.itemsize

    @classmethod
    def from_host(cls, a, stream=None):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(lib().spa_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes, stream))
        return d

    def to_host(self, out=None, stream=None):
        out = np.empty(self.shape, self.dtype) if out is None else out
        if self.nbytes:
            check(lib().spa_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, stream))
        return out

    def view(self, offset_bytes, shape, dtype):
        """a sub-array sharing this allocation (kept alive by the view)"""
        v = DeviceArray(shape, dtype, ptr=self.ptr + offset_bytes, owner=self)
        assert offset_bytes + v.nbytes <= self.nbytes
        return v

    def zero(self, stream=None):
        check(lib().spa_memset(self.ptr, 0, self.nbytes, stream))
        return self

    def __del__(self):
        if getattr(self, "_owner", 1) is None and getattr(self, "ptr", None):
            try:
                lib().spa_free(self.ptr)
            except Exception:
                pass
            self.ptr = None


def empty(shape, dtype):
    return DeviceArray(shape, dtype)


class _Pinned:
    """owner of a page-locked host allocation; freed with the last array that views it"""

    def __init__(self, nbytes):
        p = ctypes.c_void_p()
        check(lib().spa_host_alloc(ctypes.byref(p), nbytes))
        self.ptr = p.value

    def __del__(self):
        if getattr(self, "ptr", None):
            try:
                lib().spa_host_free(self.ptr)
            except Exception:
                pass
            self.ptr = None


def pinned(n, dtype=np.uint8):
    """a numpy array of n elements in page-locked host memory"""
    dtype = np.dtype(dtype)
    owner = _Pinned(max(1, n * dtype.itemsize))
    buf = (ctypes.c_char * max(1, n * dtype.itemsize)).from_address(owner.ptr)
    buf._owner = owner                                # the buffer keeps the allocation alive
    return np.frombuffer(buf, dtype, n)


def synchronize(stream=None):
    check(lib().spa_stream_synchronize(stream) if stream is not None else lib().spa_device_synchronize())


def device_count():
    n = ctypes.c_int()
    check(lib().spa_device_count(ctypes.byref(n)))
    return n.value


def current_device():
    d = ctypes.c_int()
    check(lib().spa_get_device(ctypes.byref(d)))
    return d.value


def set_device(device):
    check(lib().spa_set_device(int(device)))


def mem_info():
    f, t = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib().spa_mem_info(ctypes.byref(f), ctypes.byref(t)))
    return f.value, t.value


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().spa_stream_create(ctypes.byref(p)))
        self.handle = p.value

    def synchronize(self):
        check(lib().spa_stream_synchronize(self.handle))

    def wait(self, event):
        """work queued here from now on waits for the event's last record"""
        check(lib().spa_stream_wait_event(self.handle, event.handle))

    def __del__(self):
        if getattr(self, "handle", None):
            try:
                lib().spa_stream_destroy(self.handle)
            except Exception:
                pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().spa_event_create(ctypes.byref(p)))
        self.handle = p.value

    def record(self, stream=None):
        check(lib().spa_event_record(self.handle, stream))

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        check(lib().spa_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return ms.value

    def __del__(self):
        if getattr(self, "handle", None):
            try:
                lib().spa_event_destroy(self.handle)
            except Exception:
                pass
