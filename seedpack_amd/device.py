"""Device memory, streams and events over the library's own HIP runtime (no framework needed).

DeviceArray is the minimal device array the host layer passes around: a HIP allocation with a
dtype and a shape. It plays the role CuPy arrays play in the reference (seedpack/xp.py:6-18). Freed
allocations go to a per-size cache and are reused (as CuPy's memory pool does), so that short-lived
arrays never reach hipFree, which waits for the whole device.
"""
import bisect
import collections
import ctypes
import threading

import numpy as np

from ._lib import check, lib


class _Free:
    """one thread's freed blocks: a list per (device, size class), and per device the sorted classes
    that hold blocks"""

    def __init__(self):
        self.lists = collections.defaultdict(list)
        self.sizes = collections.defaultdict(list)

    def put(self, dev_id, n, ptr):
        lst = self.lists[(dev_id, n)]
        if not lst:
            bisect.insort(self.sizes[dev_id], n)
        lst.append(ptr)

    def pop(self, dev_id, n, most):
        """a block of the least class in [n, most] -> (class, pointer), or None"""
        sz = self.sizes.get(dev_id)
        if not sz:
            return None
        i = bisect.bisect_left(sz, n)
        if i == len(sz) or sz[i] > most:
            return None
        c = sz[i]
        lst = self.lists[(dev_id, c)]
        p = lst.pop()
        if not lst:
            sz.pop(i)
        return c, p

    def clear(self):
        """-> [(class, pointer)] of every block, the lists emptied"""
        blocks = [(k[1], p) for k, ps in self.lists.items() for p in ps]
        self.lists.clear()
        self.sizes.clear()
        return blocks


class _Cache:
    """freed device allocations kept for reuse, by device and size class: hipFree waits for every
    stream of the device, so freeing a short-lived array (a prediction, a batch's buffers) would stall
    the work other threads have queued, and a new hipMalloc of a large block costs about a millisecond.
    A request takes the least cached block of its class or larger, up to twice its size (a pack's
    files come largest first, so the blocks of one file's predictions serve the next's). A freed
    block goes back to the thread that allocated it and is reused only there: every thread here
    queues its work on one stream of its own, so work still queued on a block precedes, in stream
    order, whatever reuses it (a block dropped by another thread is dropped after that thread waited
    for its own work on it). At most `limit` bytes are held in all; beyond it memory is freed."""

    def __init__(self, limit=48 << 30):
        self.limit, self.bytes, self.lock = limit, 0, threading.Lock()
        self.tls = threading.local()
        self.owners = {}

    @staticmethod
    def size_class(n):
        n = max(int(n), 1)
        step = 4096 if n <= (1 << 20) else 1 << 20
        return -(-n // step) * step

    def mine(self):
        """this thread's free blocks"""
        f = getattr(self.tls, "free", None)
        if f is None:
            f = self.tls.free = _Free()
            with self.lock:
                self.owners[id(f)] = f
        return f

    def take(self, dev_id, n):
        """a cached block for a request of class n -> (its class, pointer), or None"""
        f = self.mine()
        with self.lock:
            got = f.pop(dev_id, n, 2 * n)
            if got is not None:
                self.bytes -= got[0]
            return got

    def give(self, owner, dev_id, ptr, n):
        with self.lock:
            if self.bytes + n > self.limit:
                return False
            self.bytes += n
            owner.put(dev_id, n, ptr)
            return True

    def drain(self, owners):
        """free the blocks the given owners hold"""
        with self.lock:
            blocks = [b for f in owners for b in f.clear()]
            self.bytes -= sum(n for n, _ in blocks)
        for _, p in blocks:
            lib().spa_free(p)

    def alloc(self, n):
        """a new device block of n bytes; when the device is full, this thread's cached blocks are
        freed and, if that is not enough, every thread's after waiting for the whole device"""
        p = ctypes.c_void_p()
        for attempt in range(3):
            if lib().spa_malloc(ctypes.byref(p), n) == 0:
                return p.value
            if attempt == 0:
                self.drain([self.mine()])
            else:
                check(lib().spa_device_synchronize())
                with self.lock:
                    owners = list(self.owners.values())
                self.drain(owners)
        check(lib().spa_malloc(ctypes.byref(p), n))
        return p.value


CACHE = _Cache()


def release_cached():
    """free every cached device block (all threads'; waits for the whole device first)"""
    check(lib().spa_device_synchronize())
    with CACHE.lock:
        owners = list(CACHE.owners.values())
    CACHE.drain(owners)


def _device_id():
    d = ctypes.c_int()
    check(lib().spa_get_device(ctypes.byref(d)))
    return d.value


class DeviceArray:
    __slots__ = ("ptr", "nbytes", "dtype", "shape", "_owner", "_alloc")

    def __init__(self, shape, dtype, ptr=None, owner=None):
        self.dtype = np.dtype(dtype)
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._alloc = None
        if ptr is None:
            dev_id, n = _device_id(), _Cache.size_class(self.nbytes)
            got = CACHE.take(dev_id, n)
            if got is None:
                got = n, CACHE.alloc(n)
            self._alloc = (CACHE.mine(), dev_id, got[0])
            self.ptr, self._owner = got[1], None
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
                owner, dev_id, n = self._alloc
                if not CACHE.give(owner, dev_id, self.ptr, n):
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


_sync_lock = threading.Lock()
_blocking = [0]


def set_blocking_waits(on):
    """the library's waits for the device (stream synchronisation, host copies) poll an event and sleep
    between polls (True) or spin in the runtime's stream synchronisation (False); process-wide -> the
    previous setting"""
    with _sync_lock:
        prev = bool(_blocking[0])
        check(lib().spa_set_sync_mode(1 if on else 0))
        _blocking[0] = 1 if on else 0
        return prev


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

    def synchronize(self):
        """wait for the work before the last record"""
        check(lib().spa_event_synchronize(self.handle))

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
