"""Whole-repository archives on the MI355X: SeedPack's M29 method (seedpack/repo3.py M29RepoGPU and
the pack / unpack / test steps of seedpack/cli.py) with this library's kernels.

An archive holds the BF16 model (the "base", R2-coded) and the repository's other files; every
quantized GGUF is stored as its difference from what the quantizers regrow from the base with the
repository's imatrix: tensors the regrowth reproduces cost nothing, the rest are QR-coded against
their prediction (or XORed, for float tensors).

MI355X design. The reference bounds GPU memory: it streams the base in 1 GB windows and feeds each
file to the GPU a window at a time (repo3.py:1869-2094). Here the whole base stays in HBM (a 9B
model is 16-18 GB of 288 GB) and each quantized file is uploaded whole: its tensors are regrown,
compared, XORed, QR-coded and zeroed on the device, and only the coded residual returns to the host.
The reference's windows still decide bytes of the archive, so they are computed and applied where
they do: a file's QR batches are cut per window and type (repo3.py:1956-1966, :946-979), a tensor
equal to one an earlier file of the same window left a residual becomes a reference
(repo3.py:2006-2030), and the zstd level of a file's residual is judged from its first span
(repo3.py:1935-1944).

Archive layout (the reference's, so that archives are interchangeable): chunks "extras" (lzma-9 of
the packed small files), "x<j>" (zstd of a big extra file), "b<i>" (base i: pack({"r2": R2 chunk})),
"f<i>" (file i's residual: zstd against the base header as raw-content dictionary), "q<i>" (its QR
batches: pack({"meta": zstd(json [[type, names], ...]), "0": batch, ...})), "manifest" (zstd-19 of
its JSON); the container index carries the catalog (names, sizes, SHA-256, roles).

Quantized files without their BF16 model: the senior quant of each group of such files (most bits
per weight) becomes their base, a "seed" (repo3.py:1359-1372), coded by the seed codec (seed.py);
its quantized tensors are dequantized for the others' requantization and seed their QR coding
directly. A file that no base shares a tensor with is coded alone: the Q8_0 codec M22 (q8.Q8Parts)
when at least half of its bytes are Q8_0 tensors (repo3.py:1190-1215), else zstd.

Quant files made with another importance matrix (another chunk count in their metadata) form sets;
the importance of their legacy-quant inputs is fitted back from the first file of a set as it is
coded (fitsets.py over imxfit.py), kept in the archive ("imx" chunk), and the set's files are
predicted with it.

The shards of a split model (llama.cpp's gguf-split names, every shard present) are coded as
bases of their own and predict as one base: the shards one after another in HBM, each tensor at its
shard's start plus its offset there (repo3.py:271-285, :634-647, :1396-1408).
"""
import collections
import dataclasses
import fnmatch
import hashlib
import json
import lzma
import mmap
import os
import re
import resource
import sys
import threading
import time
import types
import warnings
from concurrent.futures import Future, ThreadPoolExecutor, wait as futures_wait

import numpy as np

from . import blake3, container, device as dev, fitsets, gguf, header, imatrix as imx_mod, qr, r2, residual, zstd
from ._lib import check, lib
from .framing import index, nbytes, pack, pack_parts, unpack
from .gpuquant import GPUQuant
from .m24 import M24BF16
from .q8 import Q8Parts
from .requant import QFUN
from .seed import SeedCodec, bits_per_weight

METHOD = "M29 model repo: M28 with the BF16 v2 base codec (R2)"     # repo3.py:2539
METHODS = {"m29": METHOD,                                            # the archive methods built here
           "m28": "M28 model repo: BF16 + quants re-derived on the GPU with llama.cpp quantisers + imatrix",   # repo3.py:585-586
           "m30": "M30 sibling quants: tensor versions coded in chains, no base"}                           # siblings.py:168
TOOL = "seedpack 0.5.0"              # the program whose archives these are byte-for-byte (cli.py:31)
READS = (0, 5, 0)                    # the newest "needs" of a manifest this reader accepts (__init__.py:6)
HASHES = ("sha256", "blake3")        # catalog checksums this reader computes (cli.py:34-39)
WINDOW = 1 << 30                     # base bytes per window (repo3.py:1672)
PRED_WINDOW = 3 << 30                # first predictions per window, bytes (repo3.py:1677)
DUP_MIN = 64 << 10                   # smaller tensors are not made references (repo3.py:1024)
REF_KEEP = 3 << 30                   # bytes of referenced tensors per window (repo3.py:1887)
SWITCH_INTERVAL = 0.0002             # seconds (the interpreter's default is 0.005)
BUNDLE_MAX = 64 << 20                # other files up to this size go into the lzma bundle (repo3.py:1364)
Q8_MIN = 0.5                         # a base-less file with this share of Q8_0 bytes: the Q8_0 codec (repo3.py:1191)
DQ_CACHE = 32 << 30                  # dequantized seed tensors kept in HBM (float32 bytes)
SPARSE = 0.02                        # residuals with fewer non-zero bytes: zstd level >= 9 (repo3.py:45)
SKIP_DIRS = {".git", ".cache", "__pycache__"}
F32, F16, BF16 = 0, 1, 30


def log(verbose, *a):
    if verbose:
        print(*a, flush=True)


# ------------------------------------------------------------------ inputs

def collect(inputs):
    """input paths -> {name in the archive: path}: files by their base name, directories walked (sorted,
    version-control and cache folders skipped) with names relative to them (cli.py:158-175)"""
    out = {}
    for inp in inputs:
        if os.path.isdir(inp):
            for root, dirs, fs in os.walk(inp):
                dirs[:] = sorted(d for d in dirs if d not in SKIP_DIRS)
                for f in sorted(fs):
                    p = os.path.join(root, f)
                    out.setdefault(os.path.relpath(p, inp).replace(os.sep, "/"), []).append(p)
        elif os.path.isfile(inp):
            out.setdefault(os.path.basename(inp), []).append(inp)
        else:
            raise FileNotFoundError(inp)
    dup = [n for n, ps in out.items() if len(ps) > 1]
    if dup:
        raise ValueError(f"several inputs map to the same name in the archive: {', '.join(dup[:5])}")
    return {n: ps[0] for n, ps in out.items()}


def file_role(path, header=None):
    """'base' for a GGUF whose tensor bytes are at least half BF16, 'derived' for another GGUF, None for
    any other file or an imatrix GGUF (cli.py:181-205); header: its (metadata, tensors) if known"""
    if not path.lower().endswith(".gguf"):
        return None
    meta, ts = header if header is not None else gguf.header_of(path)
    if not meta and not ts:
        return None
    if meta.get("general.type") == "imatrix":
        return None
    total = sum(t.nbytes for t in ts) or 1
    return "base" if sum(t.nbytes for t in ts if t.type == BF16) / total >= 0.5 else "derived"


def order_groups(orders):
    """the files' tensor orders (tuples of names) -> {a group's order: [its files' indices]}: longest
    orders first, a file whose order is a subsequence of a group's joins it (repo3.py:277-291)"""
    groups = {}
    for k in sorted(range(len(orders)), key=lambda k: -len(orders[k])):
        for g in groups:
            it = iter(g)
            if all(n in it for n in orders[k]):
                groups[g].append(k)
                break
        else:
            groups[orders[k]] = [k]
    return {g: sorted(ks) for g, ks in groups.items()}


_SHARD = re.compile(r"^(.*)-(\d{5})-of-(\d{5})\.gguf$")


def joined_groups(names):
    """the split models among `names`: for each, the indices of its shards in shard order, when every
    shard of it (llama.cpp's gguf-split names <model>-00001-of-0000N.gguf ... -0000N-of-0000N.gguf,
    N > 1) is there (repo3.py:271-285)"""
    models = collections.defaultdict(dict)
    for i, n in enumerate(names):
        m = _SHARD.match(n)
        if m:
            models[(m.group(1), int(m.group(3)))][int(m.group(2))] = i
    return [[shards[k] for k in range(1, count + 1)] for (_, count), shards in models.items()
            if count > 1 and set(shards) == set(range(1, count + 1))]


def windows(nbytes_, window=WINDOW, pred=None, pred_window=PRED_WINDOW):
    """positions 0..n-1 (tensors in order, their base bytes) -> [(start, end)]: a window closes before a
    tensor that would take it past `window` base bytes or `pred_window` prediction bytes; a window
    holds at least one tensor (repo3.py:1689-1706)"""
    pred = pred or [0] * len(nbytes_)
    cuts, base_bytes, pred_bytes = [0], 0, 0
    for p, (nb, pb) in enumerate(zip(nbytes_, pred)):
        if p > cuts[-1] and (base_bytes + nb > window or pred_bytes + pb > pred_window):
            cuts.append(p)
            base_bytes = pred_bytes = 0
        base_bytes += nb
        pred_bytes += pb
    return list(zip(cuts, cuts[1:] + [len(nbytes_)])) if nbytes_ else []


def _nice_thread(inc):
    """raise the calling thread's nice value by inc (Linux keeps one per thread)"""
    if inc > 0 and hasattr(os, "setpriority"):
        try:
            tid = threading.get_native_id()
            os.setpriority(os.PRIO_PROCESS, tid, os.getpriority(os.PRIO_PROCESS, tid) + inc)
        except OSError:
            pass


def _read_into(path, out, off=0, pool=None, cpu=None):
    """bytes [off, off + len(out)) of a file into the writable uint8 array `out`, in parallel pieces;
    cpu(seconds) is told each piece's thread CPU time"""
    n = out.size
    step = 64 << 20
    fd = os.open(path, os.O_RDONLY)
    try:
        def piece(o):
            c0 = time.thread_time()
            try:
                _piece(o)
            finally:
                if cpu is not None:
                    cpu(time.thread_time() - c0)

        def _piece(o):
            mv = memoryview(out[o:o + step])
            got = 0
            while got < len(mv):
                k = os.preadv(fd, [mv[got:]], off + o + got)
                if k <= 0:
                    raise IOError(f"{path}: file shrank while being read")
                got += k
        if pool is None or n <= step:
            for o in range(0, n, step):
                piece(o)
        else:
            for f in [pool.submit(piece, o) for o in range(0, n, step)]:
                f.result()
    finally:
        os.close(fd)
    return out


class _DevBuf:
    """a reusable device buffer (freeing HBM waits for the whole device), grown on demand"""

    def __init__(self):
        self.a = None

    def get(self, n):
        if self.a is None or self.a.nbytes < n:
            self.a = None
            self.a = dev.DeviceArray(max(n, 1 << 20), np.uint8)
        return self.a.view(0, (n,), np.uint8)


class _DevPool:
    """device buffers of the files in flight, under a byte budget and reused (freeing HBM waits for the
    whole device): acquire(n) -> a view of n bytes of the smallest free buffer that holds it, else of a
    new buffer while the budget allows (free buffers too small are freed to make room), else it waits;
    release(view); close() frees every buffer"""

    def __init__(self, budget):
        self.budget, self.total, self.peak, self.free = budget, 0, 0, []
        self.cv = threading.Condition()

    def acquire(self, n):
        n = max(int(n), 1)
        with self.cv:
            while True:
                fit = [k for k, a in enumerate(self.free) if a.nbytes >= n]
                if fit:
                    a = self.free.pop(min(fit, key=lambda k: self.free[k].nbytes))
                    return a.view(0, (n,), np.uint8)
                if self.total + n <= self.budget or self.total == 0:
                    self.total += n
                    self.peak = max(self.peak, self.total)
                    break
                if self.free:
                    a = self.free.pop(max(range(len(self.free)), key=lambda k: self.free[k].nbytes))
                    self.total -= a.nbytes
                    check(lib().spa_free(a.ptr))
                    continue
                self.cv.wait()
        try:
            p = dev.CACHE.alloc(n)
        except BaseException:
            with self.cv:
                self.total -= n
                self.cv.notify_all()
            raise
        return dev.DeviceArray((n,), np.uint8, ptr=p, owner=self).view(0, (n,), np.uint8)

    def release(self, v):
        with self.cv:
            self.free.append(v._owner)
            self.cv.notify_all()

    def close(self):
        with self.cv:
            free, self.free = self.free, []
            self.total -= sum(a.nbytes for a in free)
        for a in free:
            lib().spa_free(a.ptr)


class _PinnedPool:
    """page-locked host buffers handed out under a byte budget and reused: acquire(n) -> a buffer of at
    least n bytes (waits while the budget is spent), release(buffer) hands it back"""

    def __init__(self, budget):
        self.budget, self.total, self.free = budget, 0, []
        self.cv = threading.Condition()

    def acquire(self, n):
        with self.cv:
            while True:
                fit = [k for k, b in enumerate(self.free) if b.size >= n]
                if fit:
                    return self.free.pop(min(fit, key=lambda k: self.free[k].size))
                if self.free and self.total + n > self.budget:
                    # free buffers too small: the largest is dropped
                    big = self.free.pop(max(range(len(self.free)), key=lambda k: self.free[k].size))
                    self.total -= big.size
                    continue
                if self.total + n <= self.budget or self.total == 0:
                    self.total += n
                    break
                self.cv.wait()
        return dev.pinned(n)

    def release(self, b):
        base = b.base if b.base is not None and isinstance(b.base, np.ndarray) else b
        while isinstance(base.base, np.ndarray):
            base = base.base
        with self.cv:
            self.free.append(base)
            self.cv.notify_all()


def _prefault(buf, pool, step=64 << 20):
    """every page of a host buffer written once (zeros), by the threads of `pool`: a freshly allocated
    page-locked buffer takes its pages' first-touch faults at about 3 GB/s in one thread (a single
    zstd stream filling it), and about six times faster from 16 threads at once"""
    a = np.frombuffer(memoryview(buf).cast("B"), np.uint8)

    def one(o):
        a[o:o + step:4096] = 0
    for f in [pool.submit(one, o) for o in range(0, a.size, step)]:
        f.result()


def _preallocate(path, n):
    """the file `path` created with n bytes reserved (posix_fallocate) -> True; False (and no file) where
    the filesystem cannot reserve them. A file whose blocks are reserved can be filled through a shared
    mapping without the risk of a fault on a full disk."""
    fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        if n:
            os.posix_fallocate(fd, 0, n)
        return True
    except OSError:
        os.close(fd)
        fd = None
        os.remove(path)
        return False
    finally:
        if fd is not None:
            os.close(fd)


def _fill_mapped(m, mv, pool, step):
    """mv copied into the mapping m in parallel pieces -> the first error, or None; every copy has
    finished and no view of m is left when it returns, so m can be closed"""
    dst, src = np.frombuffer(m, np.uint8), np.frombuffer(mv, np.uint8)
    futs = [pool.submit(np.copyto, dst[o:o + step], src[o:o + step]) for o in range(0, len(src), step)]
    futures_wait(futs)
    errs = [e for e in (f.exception() for f in futs) if e is not None]
    del dst, src, futs
    return errs[0] if errs else None


def _write_file(path, mv, pool, step=64 << 20, reserved=False):
    """the bytes mv as the file `path`, written in parallel pieces. reserved: the file already has its
    size with its blocks reserved (_preallocate); it is then filled through a shared mapping, whose page
    faults proceed in parallel (buffered writes to one file are serialised by the kernel's per-file
    lock)."""
    n = len(mv)
    if reserved and n > step and os.path.getsize(path) == n:
        fd = os.open(path, os.O_RDWR)
        try:
            m = mmap.mmap(fd, n, mmap.MAP_SHARED, mmap.PROT_READ | mmap.PROT_WRITE)
        finally:
            os.close(fd)
        try:
            err = _fill_mapped(m, mv, pool, step)
        finally:
            m.close()
        if err is not None:
            raise err
        return
    fd = os.open(path, os.O_WRONLY | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        def piece(o):
            v = mv[o:o + step]
            done = 0
            while done < len(v):
                done += os.pwrite(fd, v[done:], o + done)
        if n <= step:
            piece(0)
        else:
            for f in [pool.submit(piece, o) for o in range(0, n, step)]:
                f.result()
    finally:
        os.close(fd)


def file_digest(path, algo="sha256", chunk=64 << 20):
    """the catalog checksum (SHA-256 or BLAKE3) of a file, read in pieces into a buffer of its own"""
    h = _stream_hash(algo)
    buf = np.empty(chunk, np.uint8)
    fd = os.open(path, os.O_RDONLY)
    try:
        off = 0
        while True:
            k = os.preadv(fd, [memoryview(buf)], off)
            if k <= 0:
                break
            h.update(memoryview(buf)[:k])
            off += k
    finally:
        os.close(fd)
    return h.hexdigest()


def process_order(files, groups):
    """the order the derived files are processed in: largest first (a file that a larger one must wait
    for goes with that larger one), except that two files of one group
    sharing a (tensor name, type) pair keep their archive order -- a reference can only point to an
    earlier file with the same tensor (repo3.py:2006-2030), so processing them in any such order makes
    the same archive. A group whose potential references could exceed a window's REF_KEEP budget (then
    the decisions depend on the order of all its files) keeps its archive order throughout; files of
    one fitted-importance set keep their archive order (the first one's tensors are fitted from).
    files: {index: (bytes, {(name, type)}, group, {window: potential reference bytes}[, set])}"""
    ks = sorted(files)
    strict = set()
    for g in set(v[2] for v in files.values()):
        pot = collections.Counter()
        for i in ks:
            if files[i][2] == g:
                for w, nb in files[i][3].items():
                    pot[w] += nb
        if any(v > REF_KEEP for v in pot.values()):
            strict.add(g)

    def before(j, i):                       # must j (archive order j < i) be processed before i?
        gj, gi = files[j][2], files[i][2]
        if len(files[j]) > 4 and files[j][4] and files[j][4] == files[i][4]:
            return True                     # a fitted-importance set: its first file fits for the others
        return gj == gi and (gi in strict or files[j][1] & files[i][1])

    # a file's priority: the largest file that waits for it (itself included), so that a small file
    # holding back a big one goes early
    prio = {i: files[i][0] for i in ks}
    for i in reversed(ks):
        for j in ks:
            if j < i and before(j, i):
                prio[j] = max(prio[j], prio[i])
    todo, out = list(ks), []
    while todo:
        ready = [i for i in todo if not any(j < i and before(j, i) for j in todo)]
        pick = max(ready, key=lambda i: (prio[i], files[i][0], -i))
        out.append(pick)
        todo.remove(pick)
    return out


class _Window:
    """the base tensors one window of a derived file reads, on the device: d holds them packed,
    by_name gives each at its offset in d"""

    def __init__(self, d, by_name):
        self.d, self.by_name = d, by_name

    def view(self, t, stream=None):
        dt = np.uint16 if t.type == BF16 else np.float16 if t.type == F16 else np.float32
        return self.d.view(t.offset, (t.numel,), dt)


class _Base:
    """a base model resident in HBM: the whole file (header included) at its file offsets; or, for
    a base bigger than HBM holds beside its derived files, in host memory (`src`, d None), its
    tensors uploaded window by window (window()). A seed's quantized tensors are dequantized
    (llama.cpp's dequantize_row_*) when first used and kept, the least recently used dropped beyond
    DQ_CACHE bytes"""

    def __init__(self, index, name, host, d, g, seed=False):
        self.index, self.name, self.d, self.g, self.seed = index, name, d, g, seed
        self.header = bytes(host[:g.data_start])
        self.by_name = {t.name: t for t in g.tensors}
        self.dq, self.dq_bytes = collections.OrderedDict(), 0
        self.src, self.parts, self.rt = host, None, None

    def _source(self, off):
        """(the base holding file offset `off`, the offset there): itself, or a split model's shard"""
        if self.parts is None:
            return self, off
        start, sb = [p for p in self.parts if p[0] <= off][-1]
        return sb, off - start

    def window(self, names, stream):
        """the base itself when resident, else a _Window of the tensors `names`, each at a 256-byte
        boundary: uploaded from host memory (a base being packed), or decoded from the archive's
        coded stream (`rt`, an R2Tensors; the file's other bytes from its rest part)"""
        if self.d is not None:
            return self
        ts = [self.by_name[n] for n in dict.fromkeys(names) if n in self.by_name]
        offs, o = [], 0
        for t in ts:
            offs.append(o)
            o += -(-t.nbytes // 256) * 256
        d = dev.DeviceArray(max(o, 1), np.uint8)
        coded = collections.defaultdict(list)          # source -> [(tensor index there, offset in d, bytes)]
        for t, at in zip(ts, offs):
            sb, so = self._source(t.offset)
            rt = getattr(sb, "rt", None)
            if rt is not None and so in rt.index:
                coded[sb].append((rt.index[so], at, t.nbytes))
                continue
            src = np.ascontiguousarray(rt.outside(so, so + t.nbytes) if rt is not None else sb.src[so:so + t.nbytes])
            check(lib().spa_memcpy_h2d(d.ptr + at, src.ctypes.data, t.nbytes, stream))
        for sb, items in coded.items():
            dd, outs = sb.rt.decode([k for k, _, _ in items])
            for (_, at, nb), o_ in zip(items, outs):
                check(lib().spa_memcpy_d2d(d.ptr + at, dd.ptr + o_, nb, stream))
            dev.synchronize(stream)
            del dd
        return _Window(d, {t.name: dataclasses.replace(t, offset=at) for t, at in zip(ts, offs)})

    @classmethod
    def joined(cls, index, parts, d=None):
        """a split model as one base (repo3.py:634-647): parts [(start, shard base)], shard k's bytes from
        byte start_k of `d` on, every tensor at start_k plus its offset in the shard; the residuals'
        dictionary is the first shard's header"""
        b = cls.__new__(cls)
        first = parts[0][1]
        b.index, b.name, b.d, b.g, b.seed = index, f"{first.name} + {len(parts) - 1} more shard(s)", d, None, False
        b.header = first.header
        b.by_name = {n: dataclasses.replace(t, offset=t.offset + start)
                     for start, sb in parts for n, t in sb.by_name.items()}
        b.dq, b.dq_bytes = collections.OrderedDict(), 0
        b.src, b.parts, b.rt = None, list(parts), None
        return b

    def view(self, t, stream=None):
        """base tensor t as the quantizers take it (bf16 bits / f16 / f32; a quantized tensor as f32)"""
        if t.type in QFUN:
            a = self.dq.get(t.name)
            if a is not None:
                self.dq.move_to_end(t.name)
                return a
            cols = t.shape[0]
            a = dev.DeviceArray(t.numel, np.float32)
            check(lib().spa_dequantize(t.type, self.d.ptr + t.offset, t.numel // cols, cols, a.ptr, stream))
            self.dq[t.name] = a
            self.dq_bytes += a.nbytes
            while self.dq_bytes > DQ_CACHE and len(self.dq) > 1:
                _, old = self.dq.popitem(last=False)
                self.dq_bytes -= old.nbytes
            return a
        dt = np.uint16 if t.type == BF16 else np.float16 if t.type == F16 else np.float32
        return self.d.view(t.offset, (t.numel,), dt)


def pick_seeds(base_tensors, derived_tensors):
    """the seeds of the derived files that share no tensor name with any base (repo3.py:1359-1372):
    the senior quant left (most bits per weight, then the larger name) is a seed, and every file left
    that shares at least half of its tensor names with it is of its model; until none is left.
    base_tensors: [tensor lists]; derived_tensors: {name: tensor list} in input order"""
    in_bases = set().union(*({t.name for t in ts} for ts in base_tensors))
    left = {n: {t.name for t in ts} for n, ts in derived_tensors.items()}
    left = {n: tn for n, tn in left.items() if tn and not tn & in_bases}
    seeds = []
    while left:
        seed = max(left, key=lambda n: (bits_per_weight(derived_tensors[n]), n))
        model = left[seed]
        seeds.append(seed)
        left = {n: tn for n, tn in left.items() if 2 * len(tn & model) < len(tn)}
    return seeds


def _row_bytes(t):
    """bytes per row of a block-quantized tensor"""
    _, qk, bs = QFUN[t.type]
    return int(t.shape[0]) // qk * bs


def _zc_params(level, data):
    """the zstd parameters of a file stored alone: level >= 9 for an almost all-zero one (repo3.py:1533-1544)"""
    v = np.frombuffer(data, np.uint8)
    sparse = np.count_nonzero(v[::61]) * 61 < SPARSE * len(v)
    return zstd.Params(max(level, 9) if sparse else level, window_log=25, threads=4)


def _ws(n):
    """sha256 of a buffer"""
    return hashlib.sha256(memoryview(n).cast("B")).hexdigest()


def _done(v):
    """a finished future holding v"""
    f = Future()
    f.set_result(v)
    return f


def _digest_fn(algo):
    """the catalog's checksum of a host buffer (cli.py:34-39): SHA-256, or BLAKE3 on host threads"""
    if algo == "blake3":
        return lambda n: blake3.hexdigest(memoryview(n).cast("B"))
    return _ws


def _stream_hash(algo):
    """an incremental hasher (update / hexdigest) of the catalog's algorithm"""
    return blake3.Hasher() if algo == "blake3" else hashlib.sha256()


def check_archive(meta, manifest, verify=True):
    """what the reader refuses before it decodes anything -> the catalog's hash algorithm, or None
    (files extracted unchecked: only with verify=False and a warning).

    An archive whose manifest needs a newer reader than the version whose archives these are is
    refused (repo3.py:2285-2289); so is a catalog whose hash is neither SHA-256 nor BLAKE3, the two
    the reference writes (cli.py:34-53), unless the caller opts out of verification."""
    needs = manifest.get("needs")
    if needs:
        try:
            want = tuple(int(x) for x in str(needs).split("."))
        except ValueError:
            raise container.FormatError(f"the archive's manifest needs version {needs!r}, which is not a version number")
        if want > READS:
            raise container.FormatError(f"this archive needs SeedPack {needs} or newer (this reader reads the archives "
                                        f"of {'.'.join(map(str, READS))})")
    algo = meta.get("hash")
    if algo in HASHES:
        return algo
    if verify:
        raise container.FormatError(f"the archive's catalog hash is {algo!r}; this reader checks files with "
                                    f"{' or '.join(HASHES)} (pass verify=False to extract without checking)")
    warnings.warn(f"catalog hash {algo!r} is not one this reader computes: files are extracted unchecked")
    return None


def open_archive(path, verify=True):
    """the archive's reader, catalog (meta), manifest and checksum algorithm, after the checks of
    check_archive (nothing is decoded or written before they pass)"""
    r = container.Reader(path)
    try:
        manifest = json.loads(zstd.decompress(r.get("manifest")))
        return r, r.meta, manifest, check_archive(r.meta, manifest, verify)
    except Exception:
        r.close()
        raise


# ------------------------------------------------------------------ packing

class Packer:
    """pack(inputs, output) -> stats; the M29 pipeline of repo3.M28RepoGPU.compress (repo3.py:1374-1662)
    for a repository with BF16 base model(s), quantized GGUFs derived from them, an imatrix and other
    files"""

    def __init__(self, level=7, verbose=False, coders=8, zstd_lanes=24, staging_bytes=24 << 30, device_bytes=None,
                 method="m29", m30_slice=None, bases_in_hbm=None, hash_algo="blake3", blocking_waits=True,
                 io_threads=16, read_threads=8, lane_nice=5, switch_interval=SWITCH_INTERVAL):
        self.m30_slice = m30_slice
        # the host side (zstd frames, the read, the hashes) is what bounds a pack: the library's waits
        # for the device sleep instead of spinning a core while a pack runs
        self.blocking_waits = blocking_waits
        # the interpreter's thread switch interval while a pack runs: the device thread re-acquires the
        # interpreter lock after each wait, behind the coder and lane threads' Python slices
        self.switch_interval = switch_interval
        # the catalog's checksum: BLAKE3, the reference's whenever its blake3 requirement is installed
        # (cli.py:48-53), or SHA-256, its fallback; derived files and bases in HBM are hashed there
        if hash_algo not in HASHES:
            raise ValueError(f"catalog hash {hash_algo!r} (one of {', '.join(HASHES)})")
        self.hash_algo, self._digest = hash_algo, _digest_fn(hash_algo)
        # the BF16 bases in HBM (True), read window by window from host memory (False), or in HBM
        # when they fit beside the largest derived file and RESERVE (None)
        self.bases_in_hbm = bases_in_hbm
        if method not in METHODS:
            raise NotImplementedError(f"archive method {method!r} (built: {', '.join(METHODS)})")
        self.level, self.verbose, self.method = level, verbose, method
        self.stream = dev.Stream()
        self.gq = GPUQuant(stream=self.stream.handle)
        # the bases and the first derived file are read (in pieces) by io_threads while nothing else runs;
        # the later files, read ahead of the device while the host codes, by read_threads
        self.io = ThreadPoolExecutor(io_threads, "spa-read")
        self.io_ahead = ThreadPoolExecutor(read_threads, "spa-read-ahead")
        self.hasher = ThreadPoolExecutor(8, "spa-hash")      # file checksums
        # stage 2 of a file: its residual frame (one thread each). The host's cores bound a pack, so the
        # lanes run at a lower scheduling priority (nice + lane_nice, Linux keeps one per thread) than
        # the device thread and the QR coders that feed them, except the lane of the first file
        # processed, the largest, whose frame is the longest single-threaded job
        self.zpool = ThreadPoolExecutor(zstd_lanes, "spa-zstd", initializer=_nice_thread, initargs=(lane_nice,))
        self.zfirst = ThreadPoolExecutor(1, "spa-zstd-first")
        self.reader = ThreadPoolExecutor(1, "spa-ahead")      # the next file read ahead
        self.coders = ThreadPoolExecutor(coders, "spa-qr")
        self.pool = _PinnedPool(staging_bytes)   # page-locked: file reads
        # residuals wait in HBM for their zstd lane, within what the bases leave (set once they are
        # resident unless given)
        self.auto_budget = device_bytes is None
        self.fpool = _DevPool(device_bytes if device_bytes is not None else 8 << 30)
        self.tls = threading.local()
        self.cpu, self.cpu_lock = collections.Counter(), threading.Lock()
        self.timing = []
        self.stats = collections.Counter()
        self.sizes = {}
        self.fits = fitsets.FitSets()

    # ---------------------------------------------------------------- bases
    def _load_base(self, path, piece=1 << 30, into=None):
        """the base file uploaded whole into HBM (into `into`, a split model's place for the shard, if
        given), read through two page-locked pieces (the next piece is read, on a thread of its own,
        while the current one is copied)"""
        size = os.path.getsize(path)
        if into is not None and into.nbytes != size:
            raise ValueError(f"{path}: {size} bytes for a place of {into.nbytes}")
        d = into if into is not None else dev.DeviceArray(size, np.uint8)
        bufs = [self.pool.acquire(min(piece, max(size, 1))) for _ in range(2)]
        try:
            with ThreadPoolExecutor(1) as rd:
                offs = list(range(0, size, piece))
                nxt = rd.submit(_read_into, path, bufs[0][:min(piece, size)], 0, self.io) if offs else None
                for k, o in enumerate(offs):
                    n = min(piece, size - o)
                    nxt.result()
                    if k + 1 < len(offs):
                        o2 = offs[k + 1]
                        nxt = rd.submit(_read_into, path, bufs[(k + 1) % 2][:min(piece, size - o2)], o2, self.io)
                    check(lib().spa_memcpy_h2d(d.ptr + o, bufs[k % 2].ctypes.data, n, self.stream.handle))
        finally:
            for x in bufs:
                self.pool.release(x)
        return d

    def _code_alone(self, entry, data, ts):
        """(a zstd lane) a file no base predicts: the Q8_0 codec when at least half its bytes are Q8_0
        tensors, else zstd alone (repo3.py:1199-1215, :1633-1638)"""
        if data and sum(t.nbytes for t in ts if t.type == 8) >= Q8_MIN * len(data):
            s = dev.Stream()
            c = Q8Parts(stream=s.handle).compress(data)
            s.synchronize()
            entry["codec"] = "q8"
            self.stats["q8 files"] += 1
            return entry, None, c
        return entry, None, zstd.compress_with(data, _zc_params(self.level, data))

    def _code_base(self, b, host, order):
        """the base's chunk: pack({"r2": R2 chunk}) with the reference's part order (m29), or the M24
        chunk's parts (m28, repo3.py:1470-1475), or a seed's chunk (seed.py), coded on its own stream
        from the resident copy"""
        s = dev.Stream()
        g = gguf.GGUF(host) if b.g.light else b.g     # the whole header, tokenizer arrays included
        if b.seed:
            c = SeedCodec(stream=s.handle).compress(host, g=g, d=b.d)
            s.synchronize()
            return c
        if self.method == "m28":
            if b.d is None:
                raise NotImplementedError("archive method m28 codes its base in HBM: a base bigger than HBM needs m29")
            parts = M24BF16(stream=s.handle).compress_dev(host, d=b.d, g=g)
            s.synchronize()
            return pack_parts(parts)
        lay = r2.layout_of([(t.name, t.offset, t.nbytes, t.shape[0]) for t in g.tensors
                            if t.type == BF16 and len(t.shape) == 2], len(host))
        with ThreadPoolExecutor(1) as hp:
            rest = hp.submit(header.header_c, host, g, lay)
            # a base in host memory is coded in groups of BASE_GROUP bytes (read twice)
            codec = r2.BF16v2(stream=s.handle, stream_bytes=self.BASE_GROUP)
            inner = codec.compress_parts(b.d if b.d is not None else host, lay, rest=rest.result(), order=order) \
                if lay["t"] else \
                pack_parts({"meta": zstd.compress(json.dumps({"layout": lay, "dups": [], "nrows_c": []}).encode(), 19),
                            "side": zstd.compress(b"", 19), "tables": r2.store_tables(np.zeros((0, 256), np.uint16), []),
                            "lens": zstd.compress(b"", 19), "stream": b"", "rest": rest.result()})
        s.synchronize()
        return pack_parts({"r2": inner})

    # ---------------------------------------------------------------- QR coding on worker streams
    def _qr_job(self, T, items, seed, imx):
        if not hasattr(self.tls, "stream"):
            self.tls.stream = dev.Stream()
        c0 = time.thread_time()
        parts = qr.encode_parts(T, items, seed, imx, stream=self.tls.stream.handle)
        c1 = time.thread_time()
        out = qr.frame(parts)
        self._cpu(("qr batches", 1), ("qr coder cpu_s", c1 - c0), ("qr tables+lens zstd-19 cpu_s", time.thread_time() - c1))
        return out

    def _checksum(self, buf):
        c0 = time.thread_time()
        h = self._digest(buf)
        self._cpu(("checksum cpu_s", time.thread_time() - c0))
        return h

    def _cpu(self, *items):
        with self.cpu_lock:
            for k, v in items:
                self.cpu[k] += v

    def _timed(self, name, fn, *args):
        """fn(*args) with its thread CPU time added to the stage `name`"""
        c0 = time.thread_time()
        try:
            return fn(*args)
        finally:
            self._cpu((f"stage {name} cpu_s", time.thread_time() - c0))

    # ---------------------------------------------------------------- one derived file
    def _read_file(self, job, first=False):
        """(reader thread) the file's bytes into a page-locked buffer and its checksum started on them"""
        t0 = time.perf_counter()
        size = os.path.getsize(job["path"])
        host = self.pool.acquire(size)[:size]
        t1 = time.perf_counter()
        _read_into(job["path"], host, pool=self.io if first else self.io_ahead,
                   cpu=lambda dt: self._cpu(("file read pieces cpu_s", dt)))
        t2 = time.perf_counter()
        self._cpu(("file reads wall_s", t2 - t1))
        job["host"] = host
        # SHA-256 on a host thread from the staged bytes; BLAKE3 on the device once they are uploaded
        job["sum"] = self.hasher.submit(self._checksum, host) if self.hash_algo == "sha256" else None
        job["read"] = {"staging": round(t1 - t0, 3), "read": round(t2 - t1, 3)}
        return job

    def _device_file(self, job, b, imx_dev, imx_off, imx_map):
        """(device thread, stage 1) file job["fi"] against base b: uploaded, regrown and compared, its QR
        batches handed to the coders -> the state stage 2 finishes"""
        fi, host, tens = job["fi"], job["host"], job["tens"]
        wins_of, wstate = job["wins_of"], job["wstate"]
        tm = {"t0": time.perf_counter()}
        tm.update(job["read"])
        size = host.size
        pred = [(t, k) for t, k in tens if k]
        by_name = {t.name: t for t, _ in tens}
        F = self.fpool.acquire(size)
        tm["hbm wait"] = time.perf_counter() - tm["t0"]   # for residuals still waiting for their frames
        st = self.stream.handle
        check(lib().spa_memcpy_h2d(F.ptr, host.ctypes.data, size, st))
        tm["upload"] = time.perf_counter()
        if job["sum"] is None:
            job["sum"] = _done(blake3.device_digests(F, [(0, size)], st)[0].hex())
        # the predicted tensors' keys, their BLAKE3 digests as the reference keys them (repo3.py:2018-2022),
        # hashed on the device before anything changes them
        thash = dict(zip([t.name for t, _ in pred],
                         blake3.device_digests(F, [(t.offset, t.nbytes) for t, _ in pred], st)))
        # references: equal to a tensor an earlier file of the same window left a residual in
        refs, mine = {}, []
        for t, k in pred:
            ws = wstate[wins_of[t.name]]
            key = (t.name, t.type, thash[t.name])
            src = ws["first"].get(key)
            if src is not None and ws["memo"].get(key, False) and t.nbytes >= DUP_MIN:
                if (src, t.name) not in ws["kept"]:
                    if ws["kept_bytes"] + t.nbytes > REF_KEEP:
                        mine.append((t, k))
                        continue
                    ws["kept"].add((src, t.name))
                    ws["kept_bytes"] += t.nbytes
                refs[t.name] = [src, t.name]
                check(lib().spa_memset(F.ptr + t.offset, 0, t.nbytes, st))
                continue
            mine.append((t, k))
        self.stats["ref"] += len(refs)
        kset = self.fits.set_of.get(fi, 0)
        kind_of = {t.name: k for t, k in mine}
        # window by window (repo3.py:2041-2053): the set's importance fitted from this window's
        # tensors, then the window's residuals, its plan entries and its QR batches (each window's QR
        # tensors by type in order of appearance, repo3.py:946-979), handed to the coders at once; the
        # predictions that queued batches hold are bounded (QR_HOLD), the oldest batches waited for
        plan, qmeta, qjobs, qregs, held = [], [], [], [], collections.deque()
        by_w, mine_w = collections.defaultdict(list), collections.defaultdict(list)
        for t, _ in pred:
            by_w[wins_of[t.name]].append(t)
        for t, _ in mine:
            mine_w[wins_of[t.name]].append(t)
        out = {}

        def start(w):
            """window w's importance fit, then its first predictions and counts queued (not waited for)"""
            ts_w = mine_w.get(w, [])
            bw = b.window([t.name for t in ts_w], st)     # (the base itself when it is in HBM)
            if self.fits.waiting(kset):
                self.fits.fit_window(kset, [t for t in ts_w if kind_of[t.name] == "rq"], bw.by_name.get,
                                     lambda bt, r0, r1: self._f32_rows(bw, bt, r0, r1),
                                     lambda t, r0, r1: F.view(t.offset + r0 * _row_bytes(t), ((r1 - r0) * _row_bytes(t),), np.uint8),
                                     self.gq, st)
            fitted = self.fits.importance(kset)
            rts = [residual.Tensor(t.name, t.type, t.shape[0], F.view(t.offset, (t.nbytes,), np.uint8),
                                   bw.view(bw.by_name[t.name], st), imatrix=imx_map.get(t.name),
                                   fitted={kset: fitted[t.name]} if t.name in fitted else None,
                                   base_type=bw.by_name[t.name].type, numel=t.numel) for t in ts_w]
            return ts_w, bw, residual.residual_window_start(rts, self.gq, fitted_set=kset, stream=st) if rts else None

        # one window ahead: the next window's first predictions are queued before this one's decisions
        # wait, so the device works while the host decides and hands batches to the coders
        wins = sorted(by_w)
        ahead = start(wins[0]) if wins else None
        for wk, w in enumerate(wins):
            ts_w, bw, pending = ahead
            ahead = start(wins[wk + 1]) if wk + 1 < len(wins) else None
            w0 = time.perf_counter()
            for t, r in zip(ts_w, residual.residual_window_finish(pending) if pending is not None else []):
                out[t.name] = r
            tm["residual windows"] = tm.get("residual windows", 0.0) + time.perf_counter() - w0
            qitems = collections.defaultdict(list)
            for t in by_w[w]:
                if t.name in refs:
                    continue
                r = out[t.name]
                plan.append([t.name, "qr" if r["qr"] else r["kind"], r["variant"], t.type])
                self.stats["xor" if r["kind"] == "xor" else "requant_diff" if r["nonzero"] else "requant_exact"] += 1
                if r["qr"]:
                    qitems[t.type].append(t)
            plan += [[n, "ref", refs[n], by_name[n].type] for n in refs if wins_of[n] == w]
            for T, ts in qitems.items():
                for batch in qr.batches(T, [t.nbytes for t in ts]):
                    its = [ts[i] for i in batch]
                    grid = T in qr.GRID_TYPES
                    items = [(F.view(t.offset, (t.nbytes,), np.uint8), out[t.name]["prediction"], bw.by_name[t.name].offset,
                              bw.by_name[t.name].type, bw.by_name[t.name].shape[0], imx_off.get(t.name, -1) if grid else -1)
                             for t in its]
                    self.stats["qr_grid"] += len(its) if grid else 0
                    qmeta.append([T, [t.name for t in its]])
                    qregs.append([(t.offset, t.nbytes) for t in its])
                    qjobs.append(self.coders.submit(self._timed, "qr", self._qr_job, T, items, bw.d, imx_dev if grid else None))
                    held.append((qjobs[-1], [t.name for t in its], sum(out[t.name]["prediction"].nbytes for t in its)))
                    del items
            while held and sum(h[2] for h in held) > self.QR_HOLD:
                qj, names, _ = held.popleft()
                w0 = time.perf_counter()
                qj.result()
                tm["coder wait"] = tm.get("coder wait", 0.0) + time.perf_counter() - w0
                for n in names:                   # the batch is coded: its predictions go
                    out[n]["prediction"] = None
        tm["regrow"] = time.perf_counter()
        for t, _ in mine:
            ws = wstate[wins_of[t.name]]
            key = (t.name, t.type, thash[t.name])
            ws["first"].setdefault(key, fi)
            ws["memo"][key] = bool(out[t.name]["nonzero"])
        self.stats["qr"] += sum(len(m[1]) for m in qmeta)
        self.stream.synchronize()
        # the staged bytes go back once the checksum has read them too
        job["sum"].add_done_callback(lambda _, h=job.pop("host"): self.pool.release(h))
        entry = {"name": job["name"], "size": size, "base": b.index, "plan": plan}
        return {"fi": fi, "F": F, "qjobs": qjobs, "qmeta": qmeta, "qregs": qregs,
                "span": self._zspan(pred, wins_of, job["last_window"], size), "entry": entry, "zdict": b.header,
                "tm": tm}

    # ---------------------------------------------------------------- fitted importance (fitsets.py)
    def _f32_rows(self, b, bt, r0, r1):
        """rows r0:r1 of base tensor bt as float32 (rows, cols) on the device"""
        cols = int(bt.shape[0])
        n = (r1 - r0) * cols
        if bt.type == F32:
            return b.d.view(bt.offset + 4 * r0 * cols, (r1 - r0, cols), np.float32)
        isz, dt = 2, (np.uint16 if bt.type == BF16 else np.float16)
        src = b.d.view(bt.offset + isz * r0 * cols, (n,), dt)
        return residual.float_prediction(src, F32, self.stream.handle).view(0, (r1 - r0, cols), np.float32)

    def _lane(self):
        """this zstd lane's stream, page-locked piece and device counter"""
        if not hasattr(self.tls, "stream"):
            self.tls.stream = dev.Stream()
            self.tls.piece = dev.pinned(self.PIECE)
            self.tls.count = dev.DeviceArray(1, np.uint64)
        return self.tls.stream, self.tls.piece, self.tls.count

    PIECE = 64 << 20
    QR_HOLD = 24 << 30                   # predictions held by a file's queued QR batches (bytes)
    BASE_GROUP = 8 << 30                 # a base in host memory: bytes per group of its coding
    RESERVE = 48 << 30                   # HBM kept beside the bases and the files in flight

    def _finish_file(self, state):
        """(a zstd lane, stage 2) the zstd level judged on the device, then the residual streamed out of
        HBM into its zstd frame piece by piece, each piece once the QR batches whose tensors start in
        it or before are coded and their tensors zeroed -> (manifest entry, QR chunk or None,
        residual frame)"""
        s, piece, count = self._lane()
        st = s.handle
        F, size = state["F"], state["entry"]["size"]
        tm = state["tm"]
        try:
            # the level rule on the residual with the QR tensors still holding the file's bytes (the
            # coders only read them)
            start, span = state["span"]
            check(lib().spa_count_every(F.ptr + start, span, 61, count.ptr, st))
            nz = int(count.to_host(stream=st)[0])
            sparse = nz * 61 < SPARSE * span
            prm = zstd.Params(max(self.level, 9) if sparse else self.level, window_log=25)
            z = zstd.Compressor(prm, state["zdict"], size=size)
            qjobs, qregs = state["qjobs"], state["qregs"]
            first = [min(o for o, _ in r) for r in qregs]
            pending = sorted(range(len(qjobs)), key=lambda k: first[k])
            qparts, pi, frame = [None] * len(qjobs), 0, []
            c0, waited = time.thread_time(), 0.0
            for o in range(0, size, self.PIECE):
                m = min(self.PIECE, size - o)
                while pi < len(pending) and first[pending[pi]] < o + m:
                    k = pending[pi]
                    w0 = time.perf_counter()
                    qparts[k] = qjobs[k].result()
                    waited += time.perf_counter() - w0
                    for off, nb in qregs[k]:
                        check(lib().spa_memset(F.ptr + off, 0, nb, st))
                    pi += 1
                check(lib().spa_memcpy_d2h(piece.ctypes.data, F.ptr + o, m, st))
                frame.append(z.compress(piece[:m]))
            frame.append(z.finish())
            self._cpu(("residual zstd cpu_s", time.thread_time() - c0))
            tm["qr wait"] = waited
        finally:
            futures_wait(state["qjobs"])          # (after an error too: no coder still reads F)
            self.fpool.release(F)
        tm["zstd"] = time.perf_counter()
        qchunk = None
        if state["qmeta"]:
            qchunk = pack_parts({"meta": zstd.compress(json.dumps(state["qmeta"]).encode(), 19),
                                 **{str(k): p for k, p in enumerate(qparts)}})
        t0 = tm.pop("t0")
        self.timing.append({"file": state["entry"]["name"], "level": prm.level, "start": round(t0 - self._t_pack, 3),
                            **{k: (round(v, 3) if k in ("staging", "read", "qr wait", "hbm wait", "coder wait", "residual windows") else round(v - t0, 3))
                               for k, v in tm.items()}})
        return state["entry"], qchunk, b"".join(frame)

    @staticmethod
    def _zspan(pred, wins_of, last_window, size):
        """the bytes the zstd level is judged from: the file's first span that holds a predicted tensor,
        from that tensor on (the last window's span runs to the end of the file) -> (start, length)"""
        pred = [t for t, _ in pred]
        start = min(t.offset for t in pred)
        first_w = min(wins_of[t.name] for t in pred)
        end = max(t.offset + t.nbytes for t in pred if wins_of[t.name] == first_w)
        if first_w == last_window:
            end = size
        return start, end - start

    # ---------------------------------------------------------------- the repository
    def pack(self, inputs, output, tool=TOOL, created=None, force=False):
        # device blocks that earlier work left cached are released first: blocks of other sizes would
        # fill the cache, and each later free beyond its limit waits for the whole device
        dev.release_cached()
        prev = dev.set_blocking_waits(self.blocking_waits)
        prev_si = sys.getswitchinterval()
        if self.switch_interval:
            sys.setswitchinterval(self.switch_interval)
        try:
            return self._pack(inputs, output, tool, created, force)
        finally:
            sys.setswitchinterval(prev_si)
            dev.set_blocking_waits(prev)

    def _pack(self, inputs, output, tool, created, force):
        t0 = self._t_pack = time.perf_counter()
        ru0 = resource.getrusage(resource.RUSAGE_SELF)
        phases = {}

        def phase(name):
            phases[name] = round(time.perf_counter() - t0, 3)
        files = collect(inputs)
        if not files:
            raise ValueError("nothing to archive")
        if os.path.exists(output) and not force:
            raise FileExistsError(output)
        ggufs = [(n, p) for n, p in files.items() if p.lower().endswith(".gguf")]
        heads = dict(zip([n for n, _ in ggufs], self.io.map(gguf.header_of, [p for _, p in ggufs])))
        roles = {n: file_role(p, heads.get(n)) for n, p in files.items()}
        bases = {n: p for n, p in files.items() if roles[n] == "base"}
        derived = {n: p for n, p in files.items() if roles[n] == "derived"}
        extras = {n: p for n, p in files.items() if roles[n] is None}
        seeds = []
        if self.method != "m30":
            # quants without their BF16 model: the senior quant of each group is coded like a base and
            # the others are derived from it (repo3.py:1388-1394)
            seeds = pick_seeds([heads[n][1] for n in bases], {n: heads[n][1] for n in derived})
            bases = {**bases, **{n: derived[n] for n in seeds}}
            derived = {n: p for n, p in derived.items() if n not in seeds}
        # the shards of a split model: bases of their own, and one more base joining them (base index
        # len(bases) + k for split model k; repo3.py:1396-1408)
        bnames = list(bases)
        bsize = [os.path.getsize(bases[n]) for n in bnames]
        joined = []
        for grp in (joined_groups(bnames) if self.method != "m30" else []):
            if not any(bnames[i] in seeds for i in grp):
                starts = np.cumsum([0] + [bsize[i] for i in grp[:-1]]).tolist()
                joined.append({"parts": [[i, s_] for i, s_ in zip(grp, starts)], "size": sum(bsize[i] for i in grp)})
        base_names = [{t.name for t in heads[n][1]} for n in bases]
        base_names += [set().union(*(base_names[i] for i, _ in j["parts"])) for j in joined]
        total = sum(os.path.getsize(p) for p in files.values())
        hashes = {}
        w = container.Writer(output)
        try:
            # other files: the small ones in one lzma bundle, the big ones zstd'd one by one
            small = {n: p for n, p in extras.items() if os.path.getsize(p) <= BUNDLE_MAX}
            # (coded on a side thread; the writer takes them in chunk order when they are ready)
            aux = ThreadPoolExecutor(1, "spa-aux")
            ex = {n: open(p, "rb").read() for n, p in small.items()}
            for n, data in ex.items():
                hashes[n] = self.hasher.submit(self._digest, data)
            later = {"other files": aux.submit(lambda: lzma.compress(pack(ex), preset=9))}
            w.put_later("extras", later["other files"])
            big = {}
            for j, (n, p) in enumerate((n, p) for n, p in extras.items() if n not in small):
                data = open(p, "rb").read()
                hashes[n] = self.hasher.submit(self._digest, data)
                later[n] = aux.submit(zstd.compress_with, data, zstd.Params(self.level, threads=8, ldm=True))
                w.put_later(f"x{j}", later[n])
                big[n] = [f"x{j}", len(data)]
            phase("other files")
            if self.method == "m30":
                self._pack_m30({**bases, **derived}, w, later, hashes, {"bundle": list(ex), "single": big})
                phase("tensor chains")
                self._close(w, files, roles, hashes, later, total, tool, created)
                aux.shutdown()
                dt = time.perf_counter() - t0
                return {"input_bytes": total, "archive_bytes": os.path.getsize(output), "seconds": dt,
                        "GB_s": total / dt / 1e9, "phases": phases}
            imx_name = next((n for n in ex if n.startswith("imatrix")), None)
            imx_all = imx_mod.load(ex[imx_name]) if imx_name else {}
            # bases: their headers now (the files' plans need them), their bytes uploaded below
            loaded = []
            for i, (n, p) in enumerate(bases.items()):
                host = np.memmap(p, np.uint8, "r") if os.path.getsize(p) else np.zeros(0, np.uint8)
                # (the tokenizer's arrays are parsed later, by the base's coder on its side thread)
                loaded.append((host, _Base(i, n, host, None, gguf.GGUF(host, light=True), seed=n in seeds)))
            allb = [b for _, b in loaded] + [_Base.joined(len(bnames) + k, [(s_, loaded[i][1]) for i, s_ in j["parts"]])
                                             for k, j in enumerate(joined)]
            # the repository's importance per tensor on the device (the grid QR types read it)
            imx_vecs = {k: np.asarray(v, np.float32) for k, v in imx_all.items()}
            flat = np.concatenate(list(imx_vecs.values())) if imx_vecs else np.zeros(1, np.float32)
            imx_dev = dev.DeviceArray.from_host(flat, self.stream.handle)
            imx_off, o = {}, 0
            for k, v in imx_vecs.items():
                imx_off[k] = o
                o += v.size
            imx_map = {k: imx_dev.view(4 * imx_off[k], (v.size,), np.float32) for k, v in imx_vecs.items()}
            # derived files, per base, grouped by tensor order; windows over the base's tensor order
            names = list(derived)
            entries, chunks = [None] * len(names), {}
            per_base = collections.defaultdict(list)
            alone = []                                 # files no base shares a tensor with
            for fi, n in enumerate(names):
                ts = heads[n][1]
                common = [len({t.name for t in ts} & s) for s in base_names]
                if not common or max(common) == 0:
                    alone.append((fi, n, ts))
                    continue
                # the base sharing most tensor names; on a tie a split model rather than one of its
                # shards (repo3.py:649-657)
                best = [k for k, c in enumerate(common) if c == max(common)]
                per_base[best[-1] if best[-1] >= len(bnames) else best[0]].append((fi, n, ts))
            self.fits = fitsets.FitSets.plan(names, heads, imx_all, imx_mod.chunks(ex[imx_name]) if imx_name else None)
            # derived files: per base, grouped by tensor order; windows over each group's order
            jobs, plain, order_done = {}, [], []
            for bi, items in per_base.items():
                b = allb[bi]
                found = []
                for fi, n, ts in items:
                    tk = [(t, self._kind(b, t, imx_all)) for t in ts]
                    self.stats["raw"] += sum(k is None for _, k in tk)
                    order = tuple(t.name for t, k in sorted(tk, key=lambda x: x[0].offset) if k)
                    if order:
                        found.append((order, fi, n, tk))
                    else:
                        plain.append((bi, fi, n))
                for gk, (order, ks) in enumerate(order_groups([f[0] for f in found]).items()):
                    sts = [found[k] for k in ks]
                    # the windows' prediction bytes: per tensor, its distinct first predictions over the files
                    pred = [sum({(t.type, residual.v0(k_, imx_all.get(t.name) is not None)): t.nbytes
                                 for _, _, _, tk in sts for t, k_ in tk if t.name == nm and k_}.values()) for nm in order]
                    wins = windows([b.by_name[nm].nbytes for nm in order], WINDOW, pred)
                    wins_of = {nm: w_ for w_, (a_, z_) in enumerate(wins) for nm in order[a_:z_]}
                    wstate = [{"first": {}, "memo": {}, "kept": set(), "kept_bytes": 0} for _ in wins]
                    for _, fi, n, tk in sts:
                        jobs[fi] = {"fi": fi, "name": n, "path": derived[n], "tens": tk, "wins_of": wins_of,
                                    "wstate": wstate, "last_window": len(wins) - 1, "base": bi, "group": (bi, gk)}
                        order_done.append(fi)
            # processing order: largest first where that cannot change the archive (process_order)
            info, seen_keys = {}, {}
            for fi in sorted(jobs):
                j = jobs[fi]
                keys = {(t.name, t.type) for t, k in j["tens"] if k and t.nbytes >= DUP_MIN}
                prev = seen_keys.setdefault(j["group"], set())
                pot = collections.Counter()
                for t, k in j["tens"]:
                    if k and (t.name, t.type) in prev and t.nbytes >= DUP_MIN:
                        pot[j["wins_of"][t.name]] += t.nbytes
                prev |= keys
                info[fi] = (os.path.getsize(j["path"]), keys, j["group"], pot, self.fits.set_of.get(fi, 0))
            porder = process_order(info, None)
            # the first file read while the bases are uploaded, their checksums and codecs started
            # (one stream each)
            ahead = self.reader.submit(self._timed, "read", self._read_file, jobs[porder[0]], True) if porder else None
            side = ThreadPoolExecutor(1, "spa-base")
            base_jobs = []
            # the BF16 bases in HBM when they fit beside the largest derived file and RESERVE, else
            # read window by window from host memory (seeds are always in HBM)
            in_hbm = self.bases_in_hbm
            if in_hbm is None:
                free, _ = dev.mem_info()
                need = sum(bsize[b.index] for _, b in loaded if not b.seed)
                largest = max((os.path.getsize(p) for p in derived.values()), default=0)
                in_hbm = need + largest + self.RESERVE <= free
            if not in_hbm and self.method == "m28":
                raise NotImplementedError("archive method m28 codes its base in HBM: a base bigger than HBM needs m29")
            place = {}                                 # a split model's shards: one after another in HBM
            for k, j in enumerate(joined):
                if in_hbm:
                    allb[len(bnames) + k].d = d = dev.DeviceArray(j["size"], np.uint8)
                    for i, s_ in j["parts"]:
                        place[i] = d.view(s_, (bsize[i],), np.uint8)
            for (host, b), (n, p) in zip(loaded, bases.items()):
                b.d = self._load_base(p, into=place.get(b.index)) if in_hbm or b.seed else None
                if b.d is not None and self.hash_algo == "blake3":
                    hashes[n] = blake3.device_hexdigest(b.d, stream=self.stream.handle)
                else:
                    hashes[n] = self.hasher.submit(file_digest, p, self.hash_algo)
                base_jobs.append(side.submit(self._timed, "base", self._code_base, b, host, "stream" if b.index == 0 else "parts"))
                later[n] = base_jobs[-1]
            if base_jobs:
                # chunk order of the reference: the first base (written while the files are coded),
                # the files derived from the bases, then the other bases
                w.put_later("b0", base_jobs[0])
            self.stream.synchronize()
            if self.auto_budget:
                free, _ = dev.mem_info()
                self.fpool.budget = max(free - self.RESERVE, 8 << 30)
            phase("bases resident")
            log(self.verbose, f"  {len(bases)} base(s) resident in HBM, {time.perf_counter() - t0:.1f} s")
            # the pipeline: the next file read ahead, one file at a time on the device, the residual
            # frames on the zstd lanes
            zjobs = {}
            for k, fi in enumerate(porder):
                job = ahead.result()
                ahead = self.reader.submit(self._timed, "read", self._read_file, jobs[porder[k + 1]]) if k + 1 < len(porder) else None
                b = allb[job["base"]]
                state = self._timed("device", self._device_file, job, b, imx_dev, imx_off, imx_map)
                hashes[names[fi]] = job["sum"]            # (BLAKE3: computed on the device by _device_file)
                lanes = self.zfirst if k == 0 else self.zpool
                zjobs[fi] = lanes.submit(self._timed, "residual frame", self._finish_file, state)
                log(self.verbose, f"  {state['entry']['name']}: {state['entry']['size']:,} B regrown and compared in "
                                  f"{state['tm']['regrow'] - state['tm']['t0']:.2f} s")
            phase("derived files on the device")
            for bi, fi, n in plain:
                # nothing to predict: the file zstd'd against the base header (repo3.py:2062-2076)
                b = allb[bi]
                data = open(derived[n], "rb").read()
                hashes[n] = self.hasher.submit(self._digest, data)
                entries[fi] = {"name": n, "size": len(data), "base": b.index, "plan": []}
                zjobs[fi] = self.zpool.submit(lambda e, d, h: (e, None, zstd.compress_with(
                    d, _zc_params(self.level, d), h)), entries[fi], data, b.header)
                order_done.append(fi)
            for fi, n, ts in alone:
                data = open(derived[n], "rb").read()
                hashes[n] = self.hasher.submit(self._digest, data)
                entries[fi] = {"name": n, "size": len(data), "base": None, "plan": []}
                zjobs[fi] = self.zpool.submit(self._code_alone, entries[fi], data, ts)
                order_done.append(fi)
            for fi in order_done:
                entries[fi], qchunk, fchunk = zjobs[fi].result()
                w.put(f"f{fi}", fchunk)
                self.sizes[names[fi]] = len(fchunk)
                if qchunk is not None:
                    w.put(f"q{fi}", qchunk)
                    self.sizes[names[fi] + " (QR)"] = nbytes(qchunk)
            phase("residual frames")
            for i in range(1, len(base_jobs)):
                w.put_later(f"b{i}", base_jobs[i])
            for n, f in later.items():
                self.sizes[n] = nbytes(f.result())
            side.shutdown()
            aux.shutdown()
            phase("bases and other files coded")
            manifest = {"method": METHODS[self.method], "bases": list(bases), "seeds": seeds, "files": entries,
                        "extras": {"bundle": list(ex), "single": big}}
            if joined:
                manifest["joined"] = joined            # base len(bases) + k: split model k
                manifest["needs"] = "0.3.0"
            if self.stats["qr_grid"] or self.stats["ref"]:
                manifest["needs"] = "0.3.0"
            fitted = self.fits.chunk()
            self.stats["imx_fit"] = self.fits.fitted_inputs()
            self._cpu(("importance fit wall_s", self.fits.seconds))
            if fitted:
                w.put(fitted[1]["chunk"], fitted[0])
                self.sizes["fitted importance"] = len(fitted[0])
                manifest["imx_fit"] = fitted[1]
                manifest["needs"] = "0.3.0"
            w.put("manifest", zstd.compress(json.dumps(manifest).encode(), 19))
            hashes = {n: (h.result() if hasattr(h, "result") else h) for n, h in hashes.items()}
            missing = [n for n in files if not hashes.get(n)]
            if missing:
                raise RuntimeError(f"no checksum for {missing[:3]}")
            phase("checksums")
            q8_files = {e["name"] for e in entries if e and e.get("codec") == "q8"}
            catalog = [{"name": n, "size": os.path.getsize(p), "hash": hashes[n],
                        "role": "derived, M21" if n in q8_files else roles[n] or "file",
                        "stored": self.sizes.get(n)} for n, p in files.items()]
            w.close({"tool": tool, "method": METHODS[self.method], "created": created or _created(), "hash": self.hash_algo,
                     "files": catalog, "total": total})
        except BaseException:
            w.abort()
            raise
        finally:
            self.fpool.close()
        dt = time.perf_counter() - t0
        ru1 = resource.getrusage(resource.RUSAGE_SELF)
        cpu_s = ru1.ru_utime + ru1.ru_stime - ru0.ru_utime - ru0.ru_stime
        size = os.path.getsize(output)
        log(self.verbose, f"{output}: {total:,} B -> {size:,} B in {dt:.1f} s ({total / dt / 1e9:.2f} GB/s)")
        phase("closed")
        return {"input_bytes": total, "archive_bytes": size, "seconds": dt, "GB_s": total / dt / 1e9,
                "stats": dict(self.stats), "phases": phases, "files": self.timing,
                "clock_start_s": t0,             # perf_counter (CLOCK_MONOTONIC): lines the phases up with a trace
                "cpu": {"process cpu_s": round(cpu_s, 1), **{k: round(v, 1) for k, v in self.cpu.items()},
                        "outside the stages cpu_s": round(cpu_s - sum(v for k, v in self.cpu.items()
                                                                      if k.startswith("stage ") or k == "file read pieces cpu_s"), 1)},
                "residuals_in_hbm_peak": self.fpool.peak}

    def _pack_m30(self, ggufs, w, later, hashes, exm):
        """method m30 (siblings.M30Siblings): every GGUF's tensors as version chains"""
        from .siblings import M30Siblings
        for n, p in ggufs.items():
            hashes[n] = self.hasher.submit(file_digest, p, self.hash_algo)
        from .siblings import SLICE
        m = M30Siblings(slice_weights=self.m30_slice or SLICE, stream=self.stream.handle, verbose=self.verbose)
        man = m.compress(ggufs, w.put)
        man["extras"] = exm
        w.put("manifest", zstd.compress(json.dumps(man).encode(), 19))
        self.sizes.update(m.sizes)

    def _close(self, w, files, roles, hashes, later, total, tool, created):
        for n, f in later.items():
            self.sizes[n] = nbytes(f.result())
        hashes = {n: (h.result() if hasattr(h, "result") else h) for n, h in hashes.items()}
        catalog = [{"name": n, "size": os.path.getsize(p), "hash": hashes[n], "role": roles[n] or "file",
                    "stored": self.sizes.get(n)} for n, p in files.items()]
        w.close({"tool": tool, "method": METHODS[self.method], "created": created or _created(), "hash": self.hash_algo,
                 "files": catalog, "total": total})

    @staticmethod
    def _kind(b, t, imx_all):
        """how tensor t of a quantized file is predicted from base b: 'rq', 'xor' or None (repo3.py:691-700)"""
        bt = b.by_name.get(t.name)
        if bt is None:
            return None
        k = residual.kind(bt.type, bt.numel, t.type, t.numel, t.nbytes)
        e = imx_all.get(t.name)
        if k == "rq" and e is not None and len(e) != bt.shape[0]:
            raise NotImplementedError(f"{t.name}: an importance vector of {len(e)} values for rows of {bt.shape[0]}")
        return k


def _created():
    """the archive's creation time: now, or $SOURCE_DATE_EPOCH (UTC) for reproducible archives (cli.py:209-215)"""
    epoch = os.environ.get("SOURCE_DATE_EPOCH")
    if epoch:
        return time.strftime("%Y-%m-%dT%H:%M:%S", time.gmtime(int(epoch)))
    return time.strftime("%Y-%m-%dT%H:%M:%S")


def pack_repo(inputs, output, **kw):
    """pack the files / directories `inputs` into the archive `output` -> stats (method "m29", the
    reference's default, or "m28")"""
    return Packer(level=kw.pop("level", 7), verbose=kw.pop("verbose", False), method=kw.pop("method", "m29"),
                  m30_slice=kw.pop("m30_slice", None)).pack(inputs, output, **kw)


# ------------------------------------------------------------------ unpacking / testing

def select_names(catalog, patterns):
    """the catalog's names matching the patterns (exact, glob or base name), in catalog order
    (cli.py:296-306); all of them without patterns"""
    names = [f["name"] for f in catalog]
    if not patterns:
        return names
    chosen = []
    for pat in patterns:
        hit = [n for n in names if fnmatch.fnmatchcase(n, pat) or n == pat or os.path.basename(n) == pat]
        if not hit:
            raise KeyError(f"{pat}: no such file in the archive")
        chosen += [n for n in hit if n not in chosen]
    return chosen


class _QRAhead:
    """a file's QR batches regrown and decoded on the main stream before its residual is in, each once
    the base tensors it predicts from are decoded (Unpacker._qr_ahead)"""

    def __init__(self, u, ch, batches, var, ttype, b, imx_map, imx_dev, imx_off):
        self.u, self.ch, self.batches, self.var, self.ttype, self.b = u, ch, batches, var, ttype, b
        self.imx_map, self.imx_dev, self.imx_off = imx_map, imx_dev, imx_off
        self.decoded = {}

    def step(self, ready):
        """the batches not decoded yet whose tensors are all in `ready` (None: every batch)"""
        u, b, st = self.u, self.b, self.u.stream.handle
        for k, (T, ns) in enumerate(self.batches):
            if k in self.decoded or (ready is not None and not all(n in ready for n in ns)):
                continue
            preds = []
            for n in ns:
                bt = b.by_name[n]
                t = residual.Tensor(n, self.ttype[n], bt.shape[0], None, b.view(bt, st), imatrix=self.imx_map.get(n),
                                    fitted={k_: s_[n] for k_, s_ in u.imx_sets.items() if n in s_}, base_type=bt.type,
                                    numel=bt.numel)
                preds.append(residual.predict(u.gq, t, self.var[n], stream=st))
            items = [(p, b.by_name[n].offset, b.by_name[n].type, b.by_name[n].shape[0],
                      self.imx_off.get(n, -1) if T in qr.GRID_TYPES else -1) for p, n in zip(preds, ns)]
            self.decoded[k] = qr.decode(T, bytes(self.ch[str(k)]), items, b.d,
                                        self.imx_dev if T in qr.GRID_TYPES else None, stream=st)
            del items, preds

    def result(self):
        return self.ch, self.batches, self.decoded


class Unpacker:
    """the files of an archive rebuilt and checked against their SHA-256 (repo3.py:2277-2509,
    cli.py:309-441): each base decoded into HBM once; each quantized file's residual decompressed on
    the host, uploaded, its predictions regrown and XORed in and its QR batches decoded on the device,
    then read back, checked and written"""

    def __init__(self, verbose=False, staging_bytes=64 << 30, bases_in_hbm=None, verify=True, blocking_waits=True,
                 switch_interval=SWITCH_INTERVAL):
        self.verbose = verbose
        self.blocking_waits = blocking_waits      # the library's waits for the device sleep (as the Packer's)
        self.switch_interval = switch_interval
        self.verify = verify                      # False: a catalog hash not computed here is a warning
        # the bases decoded into HBM (True), decoded window by window from the archive (False), or
        # in HBM when they fit beside the largest file to rebuild and 48 GB (None)
        self.bases_in_hbm = bases_in_hbm
        self.stream = dev.Stream()
        self.gq = GPUQuant(stream=self.stream.handle)
        self.pool = _PinnedPool(staging_bytes)
        self.rbuf = _DevBuf()
        self.files = ThreadPoolExecutor(4)        # a finished file: checked and written
        self.io = ThreadPoolExecutor(16)          # its write, in pieces
        self.readers = ThreadPoolExecutor(16)     # a base chunk read in pieces beside its upload
        self.prealloc = ThreadPoolExecutor(2)     # the output files created and their size reserved
        self.faulters = ThreadPoolExecutor(16)    # a residual's page-locked buffer faulted in before zstd fills it
        self.base_reader = ThreadPoolExecutor(1)  # a base chunk's streamed read, beside its decode
        self.headers = ThreadPoolExecutor(2)      # the bases' headers decoded beside the extras
        self.reserved = {}
        self.hasher = ThreadPoolExecutor(4)       # its checksum, beside the write
        self.ahead = ThreadPoolExecutor(2)        # the next files' residuals decompressed ahead
        self.tls = threading.local()              # an ahead thread's stream for its residual's upload

    def run(self, archive, outdir=None, patterns=None):
        dev.release_cached()                      # (as the packer does)
        prev = dev.set_blocking_waits(self.blocking_waits)
        prev_si = sys.getswitchinterval()
        if self.switch_interval:
            sys.setswitchinterval(self.switch_interval)
        self.reserved = {}                        # .part path -> its preallocation (a future)
        try:
            return self._run(archive, outdir, patterns)
        except BaseException:
            # reserved files not written and renamed are not left behind
            for path, f in self.reserved.items():
                try:
                    if f.result():
                        os.remove(path)
                except Exception:
                    pass
            raise
        finally:
            self.reserved = {}
            sys.setswitchinterval(prev_si)
            dev.set_blocking_waits(prev)

    def _reserve(self, outdir, name, size):
        """the file's .part created and its size reserved on a side thread (the page allocation of a
        memory filesystem then runs beside the rebuild, not in the write)"""
        path = os.path.join(outdir, *name.split("/")) + ".part"

        def job():
            os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
            return _preallocate(path, size)
        self.reserved[path] = self.prealloc.submit(job)

    def _run(self, archive, outdir, patterns):
        t0 = time.perf_counter()
        r, meta, manifest, algo = open_archive(archive, self.verify)
        digest = _digest_fn(algo) if algo else None
        if manifest["method"].startswith("M30"):
            return self._run_m30(r, meta, manifest, outdir, patterns, t0, digest)
        if not manifest["method"].startswith(("M29", "M28")):
            raise NotImplementedError(f"archive method {manifest['method']!r}: only M28 / M29 / M30 archives are read here")
        seeds = set(manifest.get("seeds", []))
        nb, joined = len(manifest["bases"]), manifest.get("joined", [])
        cat = {f["name"]: f for f in meta["files"]}
        want = set(select_names(meta["files"], patterns))
        mf = manifest["files"]
        sel = {i for i, m in enumerate(mf) if m["name"] in want}
        todo = list(sel)
        while todo:                                # files holding the sources of references
            for e in mf[todo.pop()]["plan"]:
                if e[1] in ("ref", "dup") and e[2][0] not in sel:
                    sel.add(e[2][0])
                    todo.append(e[2][0])
        users = collections.defaultdict(set)      # (source file, tensor) -> the files copying it
        for i in sorted(sel):
            for e in mf[i]["plan"]:
                if e[1] in ("ref", "dup"):
                    users[tuple(e[2])].add(i)
        need_b = {i for i, n in enumerate(manifest["bases"]) if n in want} | \
                 {mf[i]["base"] for i in sel if mf[i]["base"] is not None}
        results, jobs = {}, []

        def base_header(i):
            """(side thread) a coded base's header: only the chunk's framing and its "rest" part are
            read (the whole chunk, CRC-checked, later): the rest part starts with the file's header"""
            def read(o, n, c=f"b{i}"):
                return bytes(r.read_at(c, o, n))
            parts = index(read, r.chunks[f"b{i}"][1])
            if "r2" in parts:
                parts = index(read, parts["r2"][1], parts["r2"][0])
            elif not ("side" in parts and "stream" in parts):   # else an M24 chunk (method m28)
                raise ValueError(f"base {manifest['bases'][i]}: a base chunk of an unknown kind")
            rest = np.frombuffer(header.header_d(read(*parts["rest"])), np.uint8)
            return rest, gguf.GGUF(rest.tobytes(), light=True), parts
        # the coded bases' headers decoded beside the reading of the extras and the importance
        headers = {i: self.headers.submit(base_header, i) for i in sorted(
            {i for i in need_b if i < nb} | {i for k, j in enumerate(joined) if nb + k in need_b for i, _ in j["parts"]})
            if manifest["bases"][i] not in seeds}
        # a single R2 base that will be decoded whole: its chunk's read starts now, beside the reading
        # of the extras, the importance and its header
        early_read = {}
        if len(need_b) == 1 and not joined and self.bases_in_hbm is not False:
            i = next(iter(need_b))
            name = manifest["bases"][i]
            fits = self.bases_in_hbm or cat[name]["size"] <= dev.mem_info()[0] - max(
                (mf[f]["size"] for f in sel), default=0) - (48 << 30)
            if i < nb and name not in seeds and fits:
                def read_(o, n, c=f"b{i}"):
                    return bytes(r.read_at(c, o, n))
                pp = index(read_, r.chunks[f"b{i}"][1])
                if "r2" in pp:
                    pp = index(read_, pp["r2"][1], pp["r2"][0])
                    if "stream" in pp:
                        early_read[i] = (pp, self._base_read(r, f"b{i}", pp))
        if outdir is not None:
            for m in mf:
                if m["name"] in want and m["size"] > (64 << 20):
                    self._reserve(outdir, m["name"], m["size"])

        def check_write(name, buf, release=False, known=None):
            """the file's checksum (`known`: already computed on the device) and its write side by
            side; a file that fails its checksum is not left behind"""
            try:
                mv = memoryview(buf).cast("B")
                h = self.hasher.submit(lambda: known) if known else self.hasher.submit(digest, mv) if digest else None
                path = None
                if outdir is not None:
                    path = os.path.join(outdir, *name.split("/"))
                    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
                    pre = self.reserved.get(path + ".part")
                    _write_file(path + ".part", mv, self.io, reserved=pre is not None and pre.result())
                ok = mv.nbytes == cat[name]["size"] and (h.result() == cat[name]["hash"] if h else None)
                if path is not None:
                    if ok is not False:
                        os.replace(path + ".part", path)
                    else:
                        os.remove(path + ".part")
                    self.reserved.pop(path + ".part", None)
                results[name] = ok
                return ok
            finally:
                if release:
                    self.pool.release(buf)

        def stream_write(name, rt):
            """a base decoded window by window (R2Tensors.write_to) into its file, checksummed on the way"""
            h, n = _stream_hash(algo) if algo else None, [0]
            path = None if outdir is None else os.path.join(outdir, *name.split("/"))
            f = None
            if path is not None:
                os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
                f = open(path + ".part", "wb")
            wpool = ThreadPoolExecutor(1)
            try:
                def write(b_):
                    # the file write beside the checksum (both release the interpreter lock)
                    mv = memoryview(np.ascontiguousarray(b_)).cast("B")
                    fw = wpool.submit(f.write, mv) if f is not None else None
                    if h is not None:
                        h.update(mv)
                    n[0] += mv.nbytes
                    if fw is not None:
                        fw.result()
                rt.write_to(write)
            finally:
                wpool.shutdown()
                if f is not None:
                    f.close()
            ok = n[0] == cat[name]["size"] and (h.hexdigest() == cat[name]["hash"] if h is not None else None)
            if path is not None:
                if ok is not False:
                    os.replace(path + ".part", path)
                else:
                    os.remove(path + ".part")
            results[name] = ok

        # other files
        exm = manifest["extras"]
        if any(n in want for n in exm["bundle"]) or sel:
            ex = {k: bytes(v) for k, v in unpack(lzma.decompress(bytes(r.get("extras")))).items()}
            for n in exm["bundle"]:
                if n in want:
                    jobs.append(self.files.submit(check_write, n, ex[n]))
        else:
            ex = {}
        for n, (c, size) in exm["single"].items():
            if n in want:
                out = np.empty(size, np.uint8)
                jobs.append(self.files.submit(check_write, n, zstd.decompress_into(r.get(c), out)))
        imx_name = next((n for n in ex if n.startswith("imatrix")), None)
        imx_all = {k: np.asarray(v, np.float32) for k, v in (imx_mod.load(ex[imx_name]) if imx_name else {}).items()}
        flat = np.concatenate(list(imx_all.values())) if imx_all else np.zeros(1, np.float32)
        imx_dev = dev.DeviceArray.from_host(flat, self.stream.handle)
        imx_off, o = {}, 0
        for k, v in imx_all.items():
            imx_off[k] = o
            o += v.size
        imx_map = {k: imx_dev.view(4 * imx_off[k], (v.size,), np.float32) for k, v in imx_all.items()}
        self.imx_sets = fitsets.read_chunk(r.get(manifest["imx_fit"]["chunk"]), imx_all) if manifest.get("imx_fit") else {}
        # quantized files, in archive order; tensors that later files copy are kept on the device
        kept, done = {}, set()
        # largest first, a file after the files it copies tensors from (so the checksum of a big
        # file overlaps the rebuild of the smaller ones)
        srcs = {i: {k[0] for k, us in users.items() if i in us} for i in sel}
        order, todo = [], set(sel)
        while todo:
            i = max((i for i in todo if not srcs[i] & todo), key=lambda i: (mf[i]["size"], -i))
            order.append(i)
            todo.remove(i)
        # bases: seeds decoded first (their headers need the whole file); the other bases' headers,
        # the residuals' zstd dictionaries, taken from their chunks' "rest" parts on the host, so the
        # first residuals decompress while the bases decode on the device (repo3.py:2324-2333); the
        # shards of a split model that a file predicts from one after another in one allocation
        # (repo3.py:2307-2313)
        log(self.verbose, f"  extras and importance read, {time.perf_counter() - t0:.2f} s")
        bases, place, jd, zdicts, coded = {}, {}, {}, {}, {}
        phys = sorted({i for i in need_b if i < nb} |
                      {i for k, j in enumerate(joined) if nb + k in need_b for i, _ in j["parts"]})
        for i in phys:
            name = manifest["bases"][i]
            if name in seeds:                               # a seed: its file decoded by parts (seed.py)
                if i in place:
                    raise ValueError(f"seed {name} is a shard of a split model")
                data = SeedCodec(stream=self.stream.handle).decompress(r.get(f"b{i}"))
                d = dev.DeviceArray.from_host(data, self.stream.handle)
                bases[i] = _Base(i, name, data, d, gguf.GGUF(data, light=True), seed=True)
                zdicts[i] = bases[i].header
                if name in want:
                    jobs.append(self.files.submit(check_write, name, data))
                log(self.verbose, f"  seed {name}: decoded, {time.perf_counter() - t0:.1f} s")
                continue
            rest, g, parts = headers[i].result()
            coded[i] = (rest, g, parts)
            zdicts[i] = bytes(rest[:g.data_start])
        for k, j in enumerate(joined):
            if nb + k in need_b:
                zdicts[nb + k] = zdicts[j["parts"][0][0]]
        # each base decoded whole into HBM or window by window, decided per base (repo3.py:2311-2321):
        # an M24 base (method m28) has no random access and is always decoded whole; an R2 base is
        # whole when forced (bases_in_hbm True) or, by default, while the bases so far, the largest
        # file to rebuild and a 48 GB reserve fit; a split model's shards are whole only together
        log(self.verbose, f"  base headers read, {time.perf_counter() - t0:.2f} s")
        whole = {}
        free = dev.mem_info()[0] if self.bases_in_hbm is None else 0
        room = free - max((mf[i]["size"] for i in sel), default=0) - (48 << 30)
        for i in sorted(coded, key=lambda i: "layout" not in coded[i][2]):      # M24 bases first
            size = cat[manifest["bases"][i]]["size"]
            if "layout" in coded[i][2]:
                if self.bases_in_hbm is None and size > free:
                    raise MemoryError(f"base {manifest['bases'][i]}: an M24 base is decoded whole and "
                                      f"{size:,} B do not fit in {free:,} B of free HBM")
                whole[i] = True
            else:
                whole[i] = self.bases_in_hbm if self.bases_in_hbm is not None else size <= room
            if whole[i]:
                room -= size
        for j in joined:
            if not all(whole.get(i, True) for i, _ in j["parts"]):
                for i, _ in j["parts"]:
                    if i in whole and "layout" not in coded[i][2]:
                        whole[i] = False
        for k, j in enumerate(joined):       # a split model's shards one after another in one allocation
            if nb + k in need_b and all(whole.get(i, False) for i, _ in j["parts"]):
                jd[k] = d = dev.DeviceArray(j["size"], np.uint8)
                ends = [s_ for _, s_ in j["parts"][1:]] + [j["size"]]
                for (i, s_), e_ in zip(j["parts"], ends):
                    place[i] = d.view(s_, (e_ - s_,), np.uint8)

        def in_hbm(bi):
            """base bi is decoded whole into HBM (a split model: every shard; a seed always)"""
            if bi >= nb:
                return all(whole.get(k, False) for k, _ in joined[bi - nb]["parts"])
            return whole.get(bi, False) or manifest["bases"][bi] in seeds

        def residual_of(i):
            """file i's residual decompressed -> (host buffer, its copy in HBM or None): a file rebuilt
            from a base in HBM has its residual copied there too, on this thread's stream, while the
            bases still decode, when the copy leaves the 48 GB reserve free"""
            m = mf[i]
            resid = self.pool.acquire(m["size"])[:m["size"]]
            _prefault(resid, self.faulters)
            if m.get("codec") == "q8":                      # a base-less file coded by the Q8_0 codec
                s_ = dev.Stream()
                Q8Parts(stream=s_.handle).decompress(r.get(f"f{i}"), out=resid)
                s_.synchronize()
                return resid, None
            out = zstd.decompress_into(r.get(f"f{i}"), resid, zdicts[m["base"]] if m["base"] is not None else None)
            if not (m["plan"] and m["base"] is not None and in_hbm(m["base"])) or \
                    dev.mem_info()[0] < m["size"] + (48 << 30):
                return out, None
            if not hasattr(self.tls, "up"):
                self.tls.up = dev.Stream()
            d_ = dev.DeviceArray(max(1, m["size"]), np.uint8)
            check(lib().spa_memcpy_h2d(d_.ptr, out.ctypes.data, m["size"], self.tls.up.handle))
            return out, d_

        # the first files' residuals (two threads: each frame is one serial zstd stream), as far as
        # the staging budget holds them beside the host copies of the bases to be written
        room = self.pool.budget - sum(cat[manifest["bases"][i]]["size"] for i in coded if manifest["bases"][i] in want)
        ahead = {}                                          # file index -> its residual, decompressing
        for i in order[:2]:
            room -= mf[i]["size"]
            if room < 0:
                break
            ahead[i] = self.ahead.submit(residual_of, i)
        made_early = {}                                     # file index -> its QR batches decoded during the base read
        for i in phys:
            if i not in coded:
                continue
            name = manifest["bases"][i]
            rest, g, parts = coded.pop(i)
            if not whole[i]:
                # decoded window by window from the archive (repo3.py:2311-2323): random access to
                # the coded stream of its tensors, the file written through it when it is wanted
                if "stream" not in parts or "lens" not in parts or "meta" not in parts or "side" not in parts:
                    raise ValueError(f"base {name}: not an R2 chunk")
                if "layout" in parts:
                    raise NotImplementedError("an M24 base (method m28) is decoded in HBM")
                c = f"b{i}"
                rt = r2.R2Tensors(lambda nm, c=c, pp=parts: bytes(r.read_at(c, *pp[nm])),
                                  lambda o, n, out, c=c, at=parts["stream"][0]: r.read_at(c, at + o, n, out),
                                  stream=self.stream.handle)
                b = _Base(i, name, rest, None, g)
                b.rt = rt
                bases[i] = b
                if name in want:
                    stream_write(name, rt)
                log(self.verbose, f"  base {name}: decoded window by window, {time.perf_counter() - t0:.1f} s")
                continue
            if "layout" not in parts and "stream" in parts and i not in place:
                # an R2 base: decoded tensor by tensor as its coded stream reaches HBM, the QR batches of
                # the files whose residuals decompress ahead regrown as the tensors they need are in
                users_i = [f for f in ahead if mf[f]["base"] == i and mf[f]["plan"]]
                early = {}

                def on_ready(b, ready, users_i=users_i, early=early):
                    for f in users_i:
                        if f not in early:
                            early[f] = self._qr_ahead(r, f, mf[f], b, imx_map, imx_dev, imx_off)
                        if early[f] is not None:
                            early[f].step(ready)
                er = early_read.pop(i, None)
                b = self._base_streamed(r, f"b{i}", parts, rest, g, i, name, on_ready,
                                        er[1] if er is not None and er[0] == parts else None)
                d = b.d
                for f, q in early.items():
                    if q is not None:
                        made_early[f] = q.result()
                log(self.verbose, f"  base {name}: read and decoded, {time.perf_counter() - t0:.1f} s")
            else:
                ch = unpack(memoryview(r.get(f"b{i}")))
                log(self.verbose, f"  base {name}: chunk read, {time.perf_counter() - t0:.1f} s")
                if "r2" in ch:
                    ch = {"r2": unpack(ch["r2"])}
                    d, _ = r2.BF16v2(stream=self.stream.handle).decompress(ch["r2"], device="full", into=place.get(i),
                                                                           rest=rest)
                else:
                    d = M24BF16(stream=self.stream.handle).decompress_dev(ch, into=place.get(i), rest=rest)
                b = _Base(i, name, rest, d, g)
            bases[i] = b
            if name in want:
                host = self.pool.acquire(d.nbytes)[:d.nbytes]
                known = blake3.device_hexdigest(d, stream=self.stream.handle) if algo == "blake3" else None
                check(lib().spa_memcpy_d2h(host.ctypes.data, d.ptr, d.nbytes, self.stream.handle))
                jobs.append(self.files.submit(check_write, name, host, True, known))
            log(self.verbose, f"  base {name}: decoded, {time.perf_counter() - t0:.1f} s")
        for k, j in enumerate(joined):
            if nb + k in need_b:
                bases[nb + k] = _Base.joined(nb + k, [(s_, bases[i]) for i, s_ in j["parts"]], jd.get(k))
        # files in the order their residuals become ready, among those whose sources are rebuilt (the
        # first file left always is one); two residuals decompress ahead
        left = list(order)

        def top_up():
            for i in left:
                if len(ahead) >= 2:
                    break
                if i not in ahead:
                    ahead[i] = self.ahead.submit(residual_of, i)
        top_up()
        # the QR batches of a file whose residual is still decompressing are regrown and decoded
        # meanwhile (the device works while the host's zstd streams run)
        made = made_early
        while left:
            tf = time.perf_counter()
            ready = [i for i in left if i in ahead and not srcs[i] - done]
            for i in sorted(ready, key=lambda i: mf[i]["size"]):      # the frame that ends first first
                if i not in made and not ahead[i].done() and mf[i]["plan"] and mf[i]["base"] is not None:
                    made[i] = self._predict_qr(r, i, mf[i], bases[mf[i]["base"]], imx_map, imx_dev, imx_off)
            futures_wait([ahead[i] for i in ready], return_when="FIRST_COMPLETED")
            i = next(i for i in ready if ahead[i].done())
            m = mf[i]
            resid, resid_d = ahead.pop(i).result()
            tw = time.perf_counter() - tf
            left.remove(i)
            top_up()
            tm, known = {}, None
            if m["plan"]:
                tm, known = self._rebuild(r, i, m, bases[m["base"]], resid, kept, users, done, imx_dev, imx_off,
                                          imx_map, algo == "blake3" and m["name"] in want, made.pop(i, None), resid_d)
            resid_d = None                                  # (its stream's work on it waited for by _rebuild)
            done.add(i)
            if m["name"] in want:
                jobs.append(self.files.submit(check_write, m["name"], resid, True, known))
            else:
                self.pool.release(resid)
            log(self.verbose, f"  {m['name']}: {m['size']:,} B in {time.perf_counter() - tf:.2f} s (residual wait "
                              f"{tw:.2f} s, {tm})")
        for j in jobs:
            j.result()
        r.close()
        dt = time.perf_counter() - t0
        nbytes_ = sum(cat[n]["size"] for n in results)
        return {"files": results, "bad": [n for n, ok in results.items() if ok is False],
                "unchecked": [n for n, ok in results.items() if ok is None],
                "missing": [n for n in want if n not in results], "bytes": nbytes_, "seconds": dt,
                "GB_s": nbytes_ / dt / 1e9}

    def _run_m30(self, r, meta, manifest, outdir, patterns, t0, digest):
        """an M30 archive: the extras, then the GGUF files rebuilt from their tensor chains"""
        from .siblings import M30Siblings
        cat = {f["name"]: f for f in meta["files"]}
        want = set(select_names(meta["files"], patterns))
        results = {}

        def sink(name, buf):
            ok = len(buf) == cat[name]["size"] and (digest(buf) == cat[name]["hash"] if digest else None)
            if ok is not False and outdir is not None:
                path = os.path.join(outdir, *name.split("/"))
                os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
                _write_file(path, memoryview(np.ascontiguousarray(buf)).cast("B"), self.io)
            results[name] = ok

        exm = manifest["extras"]
        if any(n in want for n in exm["bundle"]):
            for n, b in unpack(lzma.decompress(bytes(r.get("extras")))).items():
                if n in want:
                    sink(n, bytes(b))
        for n, (c, size) in exm["single"].items():
            if n in want:
                sink(n, zstd.decompress_into(r.get(c), np.empty(size, np.uint8)))
        M30Siblings(stream=self.stream.handle).decompress(manifest, r.get, want, sink)
        r.close()
        dt = time.perf_counter() - t0
        nbytes_ = sum(cat[n]["size"] for n in results)
        return {"files": results, "bad": [n for n, ok in results.items() if ok is False],
                "unchecked": [n for n, ok in results.items() if ok is None],
                "missing": [n for n in want if n not in results], "bytes": nbytes_, "seconds": dt,
                "GB_s": nbytes_ / dt / 1e9}

    PREDICT_AHEAD = 32 << 30             # bytes of QR predictions a file may have made before its residual

    def _qr_ahead(self, r, i, m, b, imx_map, imx_dev, imx_off):
        """file i's QR batches, to be regrown and decoded on the device before its residual is in (they
        need only the base, the plan, the importance and the QR chunk; the file's header, in the
        residual, is not read) -> a _QRAhead, or None when its base is not in HBM, its plan has no QR
        batch or the predictions would take more than PREDICT_AHEAD bytes"""
        plan = m["plan"]
        if b.d is None or not any(e[1] == "qr" for e in plan):
            return None
        ch = unpack(memoryview(r.get(f"q{i}")))
        batches = json.loads(zstd.decompress(ch["meta"]))
        ttype = {e[0]: e[3] for e in plan if len(e) > 3}
        names = [n for _, ns in batches for n in ns]
        if any(n not in ttype for n in names):
            return None
        need = sum(b.by_name[n].numel // QFUN[ttype[n]][1] * QFUN[ttype[n]][2] if ttype[n] in QFUN else 0 for n in names)
        if need > self.PREDICT_AHEAD:
            return None
        return _QRAhead(self, ch, batches, {e[0]: e[2] for e in plan}, ttype, b, imx_map, imx_dev, imx_off)

    def _predict_qr(self, r, i, m, b, imx_map, imx_dev, imx_off):
        """(before file i's residual is decompressed) its QR batches decoded on the device -> (QR chunk
        parts, batch list, {batch index: its tensors' bytes back to back}), or None (_qr_ahead)"""
        q = self._qr_ahead(r, i, m, b, imx_map, imx_dev, imx_off)
        if q is None:
            return None
        q.step(None)
        return q.result()

    def _base_read(self, r, c, parts):
        """the streamed read of R2 base chunk c started: the chunk read in pieces (CRC-checked once all
        are in) by the reader threads, the bytes of its coded stream copied into HBM piece by piece as
        they arrive (on a stream of its own), and its decoder built meanwhile on a side thread -> the
        read's state for _base_streamed"""
        so, sn = parts["stream"]
        st = types.SimpleNamespace(so=so, sn=sn, s_d=r2.stream_buffer(sn), up=dev.Stream(), step=2 * container.PIECE,
                                   cv=threading.Condition(), began=time.perf_counter(), last=None)
        st.done = np.zeros(-(-r.chunks[c][1] // st.step), bool)

        def to_device(o, piece):
            a, b_ = max(o, so), min(o + len(piece), so + sn)
            if a < b_:
                check(lib().spa_memcpy_h2d(st.s_d.ptr + (a - so), piece[a - o:].ctypes.data, b_ - a, st.up.handle))
            with st.cv:
                st.done[o // st.step] = True
                st.last = time.perf_counter()
                st.cv.notify_all()
        st.fut = self.base_reader.submit(r.get_streamed, c, to_device, self.readers, st.step)
        st.dec = self.headers.submit(self._decoder, r, c, parts)
        return st

    @staticmethod
    def _decoder(r, c, parts):
        """(side thread) the R2 decoder of base chunk c (its side information, tables, segment
        offsets and row maps, from the chunk's small parts) built on a stream of its own and waited for,
        its stream left unset: the caller sets the stream its decoding runs on"""
        s = dev.Stream()
        dec = r2._Decoder(lambda k: bytes(r.read_at(c, *parts[k])), s.handle)
        s.synchronize()
        dec.st = None
        return dec

    def _base_streamed(self, r, c, parts, rest, g, index, name, on_ready, rd=None):
        """an R2 base chunk read as _base_read reads it (rd: that read, already started) and its tensors
        decoded in file order on the main stream as soon as their segments are in HBM; on_ready(base,
        names) runs after each group, names being the base tensors decoded so far (all of them, None,
        once the file is complete) -> the base, whole in HBM"""
        st = self.stream.handle
        tc = time.perf_counter()
        rd = rd or self._base_read(r, c, parts)
        dec = rd.dec.result()
        dec.st = st
        layout = dec.layout
        t = layout["t"]
        t_dec = time.perf_counter()
        d = dev.DeviceArray(max(1, layout["size"]), np.uint8)
        t_alloc = time.perf_counter()
        b = _Base(index, name, rest, d, g)
        so, sn, s_d, step, done, cv, fut = rd.so, rd.sn, rd.s_d, rd.step, rd.done, rd.cv, rd.fut

        def uploaded():
            """bytes of the stream part in HBM from its start (the pieces before the first missing one)"""
            k = len(done) if done.all() else int(np.argmin(done))
            return int(np.clip(k * step - so, 0, sn))
        # a tensor's segments end at soff[seg0[i + 1]]; the decoder's reader looks up to 32 bytes
        # further (bytes it loads but does not use), so those are waited for too
        ends = dec.soff[dec.seg0[1:]].astype(np.int64) + 32
        offs = {x[0]: tn.name for x in t for tn in g.tensors if tn.offset == x[0]}
        ready, j, t0 = set(), 0, time.perf_counter()
        # times from the call (read began: negative when the read was started before it)
        lap = {"read began": round(rd.began - tc, 3), "decoder": round(t_dec - tc, 3), "allocated": round(t_alloc - tc, 3),
               "groups": 0, "decode": 0.0, "batches": 0.0, "stream in": None}
        while j < len(t):
            with cv:
                while True:
                    have = uploaded()
                    k = j
                    while k < len(t) and (ends[k] <= have or have >= sn):
                        k += 1
                    if k > j:
                        break
                    if fut.done():
                        fut.result()                 # a read error
                        raise container.FormatError(f"chunk {c}: the coded stream ended early")
                    cv.wait(0.05)
            if lap["stream in"] is None and have >= sn:
                lap["stream in"] = round(time.perf_counter() - t0, 3)
            idxs = list(range(j, k))
            in_off = np.concatenate([dec.soff[dec.seg0[x]:dec.seg0[x + 1]] for x in idxs])
            t1 = time.perf_counter()
            dec.run(s_d, in_off, d, idxs, [t[x][0] for x in idxs])
            t2 = time.perf_counter()
            ready.update(offs[t[x][0]] for x in idxs if t[x][0] in offs)
            j = k
            on_ready(b, ready)
            t3 = time.perf_counter()
            lap["groups"] += 1
            lap["decode"] += t2 - t1
            lap["batches"] += t3 - t2
            lap.setdefault("group spans", []).append((round(t1 - t0, 3), round(t3 - t0, 3), len(idxs)))
        lap["tensors decoded"] = round(time.perf_counter() - t0, 3)
        fut.result()                                 # the whole chunk read and CRC-checked
        lap["chunk checked"] = round(time.perf_counter() - t0, 3)
        lap["last piece"] = round(rd.last - t0, 3)
        r2.upload_rest(d, layout, rest, st)
        on_ready(b, None)
        lap["complete"] = round(time.perf_counter() - t0, 3)
        lap["decode"], lap["batches"] = round(lap["decode"], 3), round(lap["batches"], 3)
        log(self.verbose, f"  base {name}: streamed decode {lap}")
        return b

    def _rebuild(self, r, i, m, b, resid, kept, users, done, imx_dev, imx_off, imx_map, digest=False, pre=None,
                 resid_d=None):
        """file i's bytes from its residual (in `resid`, rebuilt in place; resid_d: its copy in HBM, if
        made already) on the device -> (phase times, the file's BLAKE3 hex digest computed on the
        device when `digest`, else None)"""
        st = self.stream.handle
        size = m["size"]
        tm, t_ = {}, [time.perf_counter()]

        def lap(name):                       # phase times of the verbose log (the stream waited for)
            if self.verbose:
                self.stream.synchronize()
                t1 = time.perf_counter()
                tm[name] = round(t1 - t_[0], 3)
                t_[0] = t1
        if resid_d is not None:
            R = resid_d.view(0, (size,), np.uint8)
        else:
            R = self.rbuf.get(size)
            check(lib().spa_memcpy_h2d(R.ptr, resid.ctypes.data, size, st))
        lap("upload")
        tens = {t.name: t for t in gguf.GGUF(resid, light=True).tensors}
        plan = m["plan"]
        ttype = {e[0]: (e[3] if len(e) > 3 else tens[e[0]].type) for e in plan}

        fitted = self.imx_sets

        def tensor(name, bw):
            bt = bw.by_name[name]
            return residual.Tensor(name, ttype[name], bt.shape[0], R.view(tens[name].offset, (tens[name].nbytes,), np.uint8),
                                   bw.view(bt, st), imatrix=imx_map.get(name),
                                   fitted={k: s_[name] for k, s_ in fitted.items() if name in s_},
                                   base_type=bt.type, numel=tens[name].numel)

        # the regrown and XORed tensors, in runs of about WINDOW base bytes (a base not in HBM is
        # decoded for each run; b.window is the base itself when it is in HBM)
        runs, cur, acc = [], [], 0
        for e in plan:
            if e[1] in ("rq", "xor"):
                nbb = b.by_name[e[0]].nbytes
                if cur and acc + nbb > WINDOW:
                    runs.append(cur)
                    cur, acc = [], 0
                cur.append(e)
                acc += nbb
        if cur:
            runs.append(cur)
        for run in runs:
            bw = b.window([e[0] for e in run], st)
            for name, kind, v, *_ in run:
                t = tensor(name, bw)
                p = residual.predict(self.gq, t, v, stream=st)
                check(lib().spa_xor(t.region.ptr, t.region.ptr, p.ptr, t.region.nbytes, None, st))
        lap("regrow+xor")
        if any(e[1] == "qr" for e in plan):
            if pre is not None:
                ch, batches, decoded = pre
            else:
                ch = unpack(memoryview(r.get(f"q{i}")))
                batches, decoded = json.loads(zstd.decompress(ch["meta"])), {}
            var = {e[0]: e[2] for e in plan}
            for k, (T, names) in enumerate(batches):
                bw = b.window(names, st)
                ts = [tensor(n, bw) for n in names]
                F = decoded.pop(k, None)
                if F is None:
                    preds = [residual.predict(self.gq, t, var[t.name], stream=st) for t in ts]
                    items = [(p, bw.by_name[t.name].offset, bw.by_name[t.name].type, bw.by_name[t.name].shape[0],
                              imx_off.get(t.name, -1) if T in qr.GRID_TYPES else -1) for t, p in zip(ts, preds)]
                    F = qr.decode(T, bytes(ch[str(k)]), items, bw.d, imx_dev if T in qr.GRID_TYPES else None, stream=st)
                    del preds, items
                o = 0
                for t in ts:
                    check(lib().spa_memcpy_d2d(t.region.ptr, F.ptr + o, t.region.nbytes, st))
                    o += t.region.nbytes
                del F
        lap("qr")
        for e in plan:
            if e[1] in ("ref", "dup"):
                src = kept[tuple(e[2])]
                t = tens[e[0]]
                check(lib().spa_memcpy_d2d(R.ptr + t.offset, src.ptr, t.nbytes, st))
        for key in [key for key in kept if users[key] <= done | {i}]:
            del kept[key]
        for (fi, name), us in users.items():
            if fi == i and not us <= done | {i}:
                t = tens[name]
                a = dev.DeviceArray(t.nbytes, np.uint8)
                check(lib().spa_memcpy_d2d(a.ptr, R.ptr + t.offset, t.nbytes, st))
                kept[(fi, name)] = a
        known = blake3.device_digests(R, [(0, size)], st)[0].hex() if digest else None
        check(lib().spa_memcpy_d2h(resid.ctypes.data, R.ptr, size, st))
        lap("download")
        return tm, known


def unpack_repo(archive, outdir=None, patterns=None, verbose=False):
    """extract (outdir given) or test the archive's files -> stats (the checksum result per file)"""
    return Unpacker(verbose=verbose).run(archive, outdir, patterns)
