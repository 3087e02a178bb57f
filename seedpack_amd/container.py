"""The .seedpack container: named chunks written back to back, an index at the end.

Byte layout (seedpack/container.py:1-10, kept as it is so that archives are interchangeable):
    b"SEEDPACK" | u32 format version (1)
    the chunks' bytes, in the order they were put
    index: zstd-19 of json.dumps({"chunks": {name: [offset, length, crc32]}, "meta": meta})
    footer: u64 index offset | u64 index length | b"SEEDEND\\0"

Writer: chunks go to `path`.part through one writer thread (in put order, CRC32 computed on the way);
close() writes the index and footer and renames the file, abort() removes it. put_stream() opens a
chunk written while it is produced, whose first bytes (its head) may be replaced at the end by a
head of the same length. Reader: any chunk or any byte range of one, read with positional reads in
parallel pieces; whole chunks are CRC-checked.
"""
import json
import os
import queue
import struct
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import zstd
from ._lib import lib

MAGIC = b"SEEDPACK"
VERSION = 1
END = b"SEEDEND\0"
FOOTER = struct.Struct("<QQ8s")
PIECE = 32 << 20                  # bytes per parallel read / CRC piece


class FormatError(Exception):
    pass


# ------------------------------------------------------------------ CRC32 of a concatenation
# CRC-32 (reflected, polynomial 0xEDB88320) is linear over GF(2): crc(A || B) = crc(A) * x^(8|B|)
# mod P xor crc(B), with the register read as a polynomial whose bit 31 is x^0. x^(8n) is built from
# the squares x^(2^k) (k = 3.. for a byte count n), so any length costs about 64 products.
_P = 0xEDB88320


def _mulmod(a, b):
    """a(x) * b(x) mod P, both in the reflected representation"""
    p = 0
    m = 1 << 31
    while a:
        if a & m:
            p ^= b
            a ^= m
        m >>= 1
        b = (b >> 1) ^ _P if b & 1 else b >> 1
    return p


_SQ = [1 << 30]                   # x^(2^k) mod P, k = 0..31 (x^1 is bit 30)
for _ in range(31):
    _SQ.append(_mulmod(_SQ[-1], _SQ[-1]))


def _xpow8(n):
    """x^(8 n) mod P"""
    p, k = 1 << 31, 3
    while n:
        if n & 1:
            p = _mulmod(_SQ[k & 31], p)
        n >>= 1
        k += 1
    return p


def crc32_combine(crc1, crc2, len2):
    """crc32(A + B) from crc32(A), crc32(B) and len(B)"""
    if len2 <= 0:
        return crc1
    return _mulmod(_xpow8(len2), crc1) ^ crc2


_POOL = ThreadPoolExecutor(8, "spa-container")


def crc32(buf, crc=0):
    """zlib.crc32(buf, crc), by the library's carry-less-multiplication CRC (the interpreter released)"""
    a = np.frombuffer(buf, np.uint8) if not isinstance(buf, np.ndarray) else buf.reshape(-1).view(np.uint8)
    return lib().spa_crc32(crc, a.ctypes.data if a.size else None, a.size)


def crc32_parallel(buf):
    """CRC32 of a large buffer: pieces on the pool, combined"""
    mv = memoryview(buf).cast("B")
    if len(mv) <= 2 * PIECE:
        return crc32(mv)
    offs = range(0, len(mv), PIECE)
    crcs = list(_POOL.map(lambda o: crc32(mv[o:o + PIECE]), offs))
    crc = 0
    for o, c in zip(offs, crcs):
        crc = crc32_combine(crc, c, min(PIECE, len(mv) - o))
    return crc


def _bytes_of(x):
    return x if isinstance(x, (bytes, bytearray, memoryview)) else memoryview(np.ascontiguousarray(x)).cast("B")


# ------------------------------------------------------------------ writing

class Writer:
    def __init__(self, path):
        self.path = path
        self.f = open(path + ".part", "wb")
        self.f.write(MAGIC + struct.pack("<I", VERSION))
        self.chunks = {}
        self.jobs = queue.Queue()
        self.err = None
        self.streams = []
        self.t = threading.Thread(target=self._run, daemon=True)
        self.t.start()

    # the writer thread: one job at a time, in put order
    def _run(self):
        while True:
            job = self.jobs.get()
            if job is None:
                return
            if self.err is not None:
                continue
            try:
                job()
            except BaseException as e:        # reported by the next put() / close()
                self.err = e

    def _raise(self):
        if self.err is not None:
            raise self.err

    def _claim(self, name):
        self._raise()
        if name in self.chunks:
            raise ValueError(f"duplicate chunk {name}")
        self.chunks[name] = None

    def put(self, name, data):
        """chunk `name` = data (bytes-like, or a list of them written back to back)"""
        self._claim(name)
        parts = data if isinstance(data, list) else [data]
        self.jobs.put(lambda: self._write(name, parts))

    def put_later(self, name, fut):
        """chunk `name` = the result of the future `fut` (bytes-like or a list of them), written in put
        order once it is ready: the chunks put after it wait for it"""
        self._claim(name)
        self.jobs.put(lambda: self._write(name, (lambda d: d if isinstance(d, list) else [d])(fut.result())))

    def _write(self, name, parts):
        off, n, crc = self.f.tell(), 0, 0
        for p in parts:
            b = _bytes_of(p)
            crc = crc32_combine(crc, crc32_parallel(b), len(b)) if len(b) > 2 * PIECE else crc32(b, crc)
            self.f.write(b)
            n += len(b)
        self.chunks[name] = [off, n, crc]

    def put_stream(self, name):
        """a chunk written while it is produced -> ChunkStream (head / write / close / abort)"""
        self._claim(name)
        cs = ChunkStream(self, name)
        self.streams.append(cs)
        self.jobs.put(cs._drain)
        return cs

    def close(self, meta):
        self.jobs.put(None)
        self.t.join()
        self._raise()
        idx = zstd.compress(json.dumps({"chunks": self.chunks, "meta": meta}).encode(), 19)
        off = self.f.tell()
        self.f.write(idx)
        self.f.write(FOOTER.pack(off, len(idx), END))
        self.f.close()
        os.replace(self.path + ".part", self.path)

    def abort(self):
        for cs in self.streams:
            cs.abort()
        self.err = self.err or IOError("archive aborted")
        self.jobs.put(None)
        self.t.join()
        self.f.close()
        try:
            os.remove(self.path + ".part")
        except OSError:
            pass


class ChunkStream:
    """the producer's end of a streamed chunk: head(b) its first bytes (replaceable by close(head) with
    a head of the same length), write(b) the rest in order, close() / abort(). At most `depth` pieces
    wait for the writer (a big model's chunk is gigabytes)."""

    def __init__(self, w, name, depth=4):
        self.w, self.name = w, name
        self.q = queue.Queue(maxsize=depth)

    def _put(self, item):
        while True:                         # (the writer may have failed: then it drains nothing)
            self.w._raise()
            try:
                self.q.put(item, timeout=0.5)
                return
            except queue.Full:
                pass

    def head(self, b):
        self._put(("head", bytes(b)))

    def write(self, b):
        self._put(("data", b))

    def close(self, head=None):
        self._put(("end", head))

    def abort(self):
        try:
            self.q.put_nowait(("abort", None))
        except queue.Full:
            pass

    def _drain(self):
        f = self.w.f
        off, head, n, crc = f.tell(), b"", 0, 0
        while True:
            kind, data = self.q.get()
            if kind == "head":
                head = data
                f.write(head)
                n += len(head)
            elif kind == "data":
                b = _bytes_of(data)
                crc = crc32(b, crc)
                f.write(b)
                n += len(b)
            elif kind == "end":
                if data is not None:
                    if len(data) != len(head):
                        raise ValueError(f"chunk {self.name}: the final head has another length")
                    end = f.tell()
                    f.seek(off)
                    f.write(data)
                    f.seek(end)
                    head = bytes(data)
                self.w.chunks[self.name] = [off, n, crc32_combine(crc32(head), crc, n - len(head))]
                return
            else:
                raise IOError(f"chunk {self.name}: its producer stopped")


# ------------------------------------------------------------------ reading

class Reader:
    def __init__(self, path):
        self.path = path
        self.size = os.path.getsize(path)
        self.fd = os.open(path, os.O_RDONLY)
        head = os.pread(self.fd, len(MAGIC) + 4, 0)
        if head[:len(MAGIC)] != MAGIC:
            raise FormatError(f"{path}: not a .seedpack archive")
        (version,) = struct.unpack_from("<I", head, len(MAGIC))
        if version > VERSION:
            raise FormatError(f"{path}: format version {version} is newer than this reader")
        if self.size < len(head) + FOOTER.size:
            raise FormatError(f"{path}: truncated archive")
        off, n, end = FOOTER.unpack(os.pread(self.fd, FOOTER.size, self.size - FOOTER.size))
        if end != END or off + n > self.size:
            raise FormatError(f"{path}: truncated or damaged archive (no index)")
        idx = json.loads(zstd.decompress(os.pread(self.fd, n, off)))
        self.chunks, self.meta = idx["chunks"], idx["meta"]

    def _read(self, pos, mv):
        got = 0
        while got < len(mv):
            k = os.preadv(self.fd, [mv[got:]], pos + got)
            if k <= 0:
                raise FormatError(f"{self.path}: truncated archive")
            got += k

    def read_at(self, name, rel, n, out=None):
        """n bytes of chunk `name` from its byte `rel` (not CRC-checked: a part of a chunk), into
        `out` (a writable buffer of n bytes) when given"""
        off, size, _ = self.chunks[name]
        if rel < 0 or rel + n > size:
            raise ValueError(f"{name}: bytes {rel}..{rel + n} outside the chunk ({size})")
        out = np.empty(n, np.uint8) if out is None else out
        mv = memoryview(out).cast("B")
        if n <= 2 * PIECE:
            self._read(off + rel, mv)
        else:
            for f in [_POOL.submit(self._read, off + rel + o, mv[o:o + PIECE]) for o in range(0, n, PIECE)]:
                f.result()
        return out

    def get(self, name):
        """the whole chunk (uint8 array), CRC-checked"""
        _, n, crc = self.chunks[name]
        data = self.read_at(name, 0, n)
        if crc32_parallel(data) != crc:
            raise FormatError(f"{self.path}: chunk {name} is damaged (CRC mismatch)")
        return data

    def get_streamed(self, name, on_piece, pool, step=2 * PIECE):
        """the whole chunk as get() returns it, read in pieces of `step` bytes by the threads of `pool`;
        on_piece(offset, piece) runs in the reading thread as each piece arrives (before the chunk's
        CRC is known: a damaged chunk still raises once every piece is in)"""
        _, n, crc = self.chunks[name]
        data = np.empty(n, np.uint8)

        def one(o):
            k = min(step, n - o)
            v = data[o:o + k]
            self.read_at(name, o, k, v)
            on_piece(o, v)
            return crc32(v), k
        c = 0
        for pc, k in pool.map(one, range(0, n, step)):
            c = crc32_combine(c, pc, k)
        if c != crc:
            raise FormatError(f"{self.path}: chunk {name} is damaged (CRC mismatch)")
        return data

    def close(self):
        if self.fd is not None:
            os.close(self.fd)
            self.fd = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
