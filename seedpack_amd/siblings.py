"""Method M30 (the reference's seedpack/siblings.py): several quantizations of one model without the
model itself, coded tensor by tensor instead of file by file.

Planning. The files are read once (sorted by name): each file's and each tensor's BLAKE3 digest
(the reference's keys), its GGUF header and the bytes between its tensors. A file equal to an
earlier one (digest and size) is stored as a pointer to it. The tensors of the other files are
grouped by (name, shape) in order of first appearance (files in name order, tensors by offset); a
group's versions are its distinct (type, bytes), each coded once, chained most bytes first (ties in
order of first appearance).

Coding. A group whose versions are all below 1 MiB goes raw into the "small" chunk. Any other group
is coded in row slices of at most `slice` weights; in each slice the first version of the chain is
coded alone (QR without a seed where that is smaller than its bytes, else zstd level 3 where smaller,
else raw), every later version against an explicit seed: the precision-weighted mean of the versions
before it (estimate.Est), its blocks predicted by the quantizer run on that mean (QR where smaller
than its bytes, else zstd level 3). GGUF headers and the bytes between tensors go into one zstd
chunk ("heads").

Chunk names and manifest (fixed by the reference's format, siblings.py:267-444): "heads",
"g<group>.<version>.<slice>", "small", then the caller's "manifest" of
  {"method", "needs": "0.4.0", "slice", "files": [{"name", "size", "same" | "head", "gaps",
   "tensors"}], "groups": [{"name", "shape", "cols", "vers": [{"type", "nbytes", "kinds" |
   "small"}]}]}
with the keys in that order: "same" is the index of an identical earlier file (null otherwise);
"head" [position, length] in the heads chunk; "gaps" [[file offset, position, length], ...];
"tensors" [[group, version, offset, bytes], ...] by offset; "kinds" one of "self", "qr", "z", "raw"
per slice; "small" [position, length] in the small chunk.
"""
import dataclasses
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import blake3
from . import device as dev
from . import gguf, qr, zstd
from .estimate import Est, half_step
from .gpuquant import GPUQuant
from .requant import QFUN

NAME = "M30 sibling quants: tensor versions coded in chains, no base"     # siblings.py:168
F32, F16, BF16 = 0, 1, 30
FLOATS = {F32: np.float32, F16: np.float16}
SLICE = 1 << 26                          # weights per coding slice (siblings.py:41)
SMALL = 1 << 20                          # groups whose versions are all smaller go raw into "small"
NEED_IMX = {16, 17, 19}                  # quantizers that assert an importance matrix (siblings.py:43)


def _row_bytes(T, cols):
    qk, bs = gguf.BLOCK[T]
    return cols // qk * bs


def _read(path, off, n):
    out = np.empty(n, np.uint8)
    with open(path, "rb") as f:
        f.seek(off)
        f.readinto(memoryview(out))
    return out


def _qr_alone(T, cols):
    """can the type be QR-coded without a seed at this row length"""
    return T in qr.QR_TYPES and cols % qr.QK[T] == 0


def _qr_seeded(T, cols):
    """can the type be QR-coded against an explicit seed (its quantizer predicts the blocks)"""
    return _qr_alone(T, cols) and T in QFUN


@dataclasses.dataclass
class FileScan:
    path: str
    size: int
    digest: str
    head: bytes
    gaps: list                 # [(file offset, bytes)]
    tensors: list              # [(gguf.Tensor, digest)] by offset


@dataclasses.dataclass
class Version:
    type: int
    digest: str
    nbytes: int
    src: tuple                 # (file index, offset) where its bytes are read
    kinds: list = dataclasses.field(default_factory=list)
    small: list = None

    def manifest(self):
        d = {"type": self.type, "nbytes": self.nbytes}
        if self.small is not None:
            d["small"] = self.small
        else:
            d["kinds"] = self.kinds
        return d


@dataclasses.dataclass
class Group:
    name: str
    shape: list
    versions: list

    @property
    def cols(self):
        return int(self.shape[0])

    def rows(self):
        return int(np.prod(self.shape)) // self.cols

    def manifest(self):
        return {"name": self.name, "shape": self.shape, "cols": self.cols,
                "vers": [v.manifest() for v in self.versions]}


def scan_file(path):
    """one read of a GGUF: its digest, header bytes, the bytes between its tensors and each tensor's digest"""
    size = os.path.getsize(path)
    data = np.memmap(path, np.uint8, "r") if size else np.zeros(0, np.uint8)
    g = gguf.GGUF(data, light=True)
    ts = sorted(g.tensors, key=lambda t: t.offset)
    gaps, at = [], g.data_start
    for t in ts:
        if t.offset > at:
            gaps.append((at, bytes(data[at:t.offset])))
        at = max(at, t.offset + t.nbytes)
    if size > at:
        gaps.append((at, bytes(data[at:size])))
    with ThreadPoolExecutor(4) as ex:
        whole = ex.submit(blake3.hexdigest, data)
        digests = list(ex.map(lambda t: blake3.hexdigest(data[t.offset:t.offset + t.nbytes], threads=4), ts))
        return FileScan(path, size, whole.result(), bytes(data[:g.data_start]), gaps, list(zip(ts, digests)))


def plan(names, scans):
    """files and version chains -> (file entries without head / gaps / tensors, unique file indices,
    groups, {(file index, tensor offset): (group, version)})"""
    entries, first = [], {}
    for i, n in enumerate(names):
        s = scans[n]
        j = first.setdefault((s.digest, s.size), i)
        entries.append({"name": n, "size": s.size, "same": None if j == i else j})
    unique = [i for i, e in enumerate(entries) if e["same"] is None]
    groups, by_key = [], {}
    for i in unique:
        for t, h in scans[names[i]].tensors:
            g = by_key.get((t.name, tuple(t.shape)))
            if g is None:
                g = by_key[(t.name, tuple(t.shape))] = Group(t.name, list(t.shape), [])
                groups.append(g)
            if not any(v.type == t.type and v.digest == h for v in g.versions):
                g.versions.append(Version(t.type, h, t.nbytes, (i, t.offset)))
    for g in groups:                           # most bytes first; sorted() keeps first-seen order on ties
        g.versions = sorted(g.versions, key=lambda v: -v.nbytes)
    where = {}
    gindex = {id(g): k for k, g in enumerate(groups)}
    for i in unique:
        for t, h in scans[names[i]].tensors:
            g = by_key[(t.name, tuple(t.shape))]
            k = next(k for k, v in enumerate(g.versions) if v.type == t.type and v.digest == h)
            where[(i, t.offset)] = (gindex[id(g)], k)
    return entries, unique, groups, where


class M30Siblings:
    name = NAME

    def __init__(self, slice_weights=SLICE, stream=None, verbose=False):
        self.slice, self.stream, self.verbose = slice_weights, stream, verbose
        self.gq = GPUQuant(stream=stream)
        self.sizes = {}

    # ------------------------------------------------------------------ the running estimate
    def _values(self, T, blocks, cols, nw):
        """a version's values and half steps per weight (device float32), or None for a type that
        gives none (siblings.py:98-126)"""
        st = self.stream
        if T in FLOATS or T == BF16:
            raw = blocks.to_host(stream=st)
            x = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32) if T == BF16 else \
                raw.view(FLOATS[T]).astype(np.float32)
            return dev.DeviceArray.from_host(x, st), dev.DeviceArray(nw, np.float32).zero(st)
        if T not in QFUN:
            return None
        x = self.gq.dequantize(T, blocks, cols)
        if T in qr.GRID_TYPES:
            return x, qr.grid_half_steps(T, blocks, nw, st)
        if T in qr.QR_TYPES:
            lo, hi = qr.intervals(T, blocks, nw, st)
            return x, half_step(x, lo, hi, st)
        return None

    def _learn(self, est, T, blocks, cols):
        vh = self._values(T, blocks, cols, est.nw)
        if vh is not None:
            est.add(*vh)

    def _prediction(self, T, seed, cols):
        """the blocks llama.cpp's quantizer makes of the seed's values (its even float32 words)"""
        x = dev.DeviceArray.from_host(seed.to_host(stream=self.stream).reshape(-1, 2)[:, 0].copy(), self.stream)
        imx = np.ones(cols, np.float32) if T in NEED_IMX else None
        return self.gq.quantize_tensors(T, [(x, cols)], [imx], device=True)[0]

    def slices(self, g):
        per = max(1, self.slice // g.cols)
        rows = g.rows()
        return [(r, min(per, rows - r)) for r in range(0, rows, per)]

    # ------------------------------------------------------------------ pack
    def compress(self, paths, put):
        """paths: {name: path} of the GGUF files; put(chunk name, bytes) -> the manifest dict (its
        "extras" entry is the caller's); self.sizes gets the stored bytes per file"""
        names = sorted(paths)
        scans = {n: scan_file(paths[n]) for n in names}
        entries, unique, groups, where = plan(names, scans)
        heads = bytearray()
        for i in unique:
            s, e = scans[names[i]], entries[i]
            e["head"] = [len(heads), len(s.head)]
            heads += s.head
            e["gaps"] = []
            for off, b in s.gaps:
                e["gaps"].append([off, len(heads), len(b)])
                heads += b
            e["tensors"] = [[*where[(i, t.offset)], t.offset, t.nbytes] for t, _ in s.tensors]
        put("heads", zstd.compress_with(bytes(heads), zstd.Params(19, window_log=27, threads=8, ldm=True)))
        self.sizes["headers"] = len(heads)
        small, stored = bytearray(), {}
        for gi, g in enumerate(groups):
            if all(v.nbytes < SMALL for v in g.versions):
                for v in g.versions:
                    v.small = [len(small), v.nbytes]
                    small += _read(scans[names[v.src[0]]].path, v.src[1], v.nbytes).tobytes()
            else:
                self._code_group(gi, g, names, scans, put, stored)
        put("small", zstd.zstd_c(bytes(small), 19))
        counted = set()
        for i, e in enumerate(entries):
            if e["same"] is not None:
                self.sizes[e["name"]] = 0
                continue
            mine = {(gi, k) for gi, k, _, _ in e["tensors"]} - counted
            counted |= mine
            self.sizes[e["name"]] = sum(stored.get(x, 0) for x in mine)
        return {"method": self.name, "needs": "0.4.0", "slice": self.slice, "files": entries,
                "groups": [g.manifest() for g in groups]}

    def _code_group(self, gi, g, names, scans, put, stored):
        st, cols = self.stream, g.cols
        for j, (r0, nr) in enumerate(self.slices(g)):
            est = Est(nr * cols, st) if len(g.versions) > 1 else None
            for k, v in enumerate(g.versions):
                rb = _row_bytes(v.type, cols)
                raw = _read(scans[names[v.src[0]]].path, v.src[1] + r0 * rb, nr * rb)
                kind, data = self._alone(v.type, raw, cols) if k == 0 else self._seeded(v.type, raw, cols, est)
                put(f"g{gi}.{k}.{j}", data)
                stored[(gi, k)] = stored.get((gi, k), 0) + len(data)
                v.kinds.append(kind)
                if est is not None and k + 1 < len(g.versions):
                    self._learn(est, v.type, dev.DeviceArray.from_host(raw, st), cols)

    def _alone(self, T, raw, cols):
        """a chain's first version: QR without a seed (grid types too), zstd level 3 or raw, the first
        of them smaller than the bytes (siblings.py:422-429)"""
        if _qr_alone(T, cols):
            c = qr.self_encode(T, [(raw, cols)], stream=self.stream)
            if len(c) < len(raw):
                return "self", c
        z = zstd.zstd_c(raw.tobytes(), 3)
        return ("z", z) if len(z) < len(raw) else ("raw", raw.tobytes())

    def _seeded(self, T, raw, cols, est):
        """a later version: QR against the estimate of the versions before it where that is smaller
        than the bytes, else zstd level 3"""
        if est is not None and est.x0 is not None and _qr_seeded(T, cols):
            seed = est.seed()
            c = qr.encode(T, [(dev.DeviceArray.from_host(raw, self.stream), self._prediction(T, seed, cols), 0,
                               qr.EXPLICIT, cols)], seed, stream=self.stream)
            if len(c) < len(raw):
                return "qr", c
        return "z", zstd.zstd_c(raw.tobytes(), 3)

    # ------------------------------------------------------------------ unpack
    def decompress(self, man, get, want, sink):
        """the wanted GGUF files of an M30 archive: sink(name, bytes) for each (a chain's versions are
        decoded once and kept for the other files that hold them)"""
        self.slice = man["slice"]
        groups = [Group(g["name"], g["shape"], [dict(v) for v in g["vers"]]) for g in man["groups"]]
        heads = np.frombuffer(zstd.decompress(get("heads")), np.uint8)
        small = zstd.decompress(get("small")) if any("small" in v for g in groups for v in g.versions) else b""
        decoded = {}

        def version(gi, k):
            if (gi, k) not in decoded:
                decoded.update(((gi, kk), a) for kk, a in enumerate(self._decode_chain(get, groups[gi], gi, k, small)))
            return decoded[(gi, k)]

        for e in man["files"]:
            if e["name"] not in want:
                continue
            src = man["files"][e["same"]] if e["same"] is not None else e
            out = np.zeros(src["size"], np.uint8)
            h0, hn = src["head"]
            out[:hn] = heads[h0:h0 + hn]
            for off, at, ln in src["gaps"]:
                out[off:off + ln] = heads[at:at + ln]
            for gi, k, off, nb in src["tensors"]:
                out[off:off + nb] = version(gi, k)
            sink(e["name"], out)

    def _decode_chain(self, get, g, gi, top, small):
        """versions 0..top of group g, whole (slices joined) -> list of host uint8 arrays"""
        vers = g.versions
        if "small" in vers[0]:
            return [np.frombuffer(small, np.uint8, vers[k]["small"][1], vers[k]["small"][0]) for k in range(top + 1)]
        st, cols = self.stream, g.cols
        pieces = [[] for _ in range(top + 1)]
        for j, (r0, nr) in enumerate(self.slices(g)):
            est = Est(nr * cols, st) if top > 0 else None
            for k in range(top + 1):
                T, kind = vers[k]["type"], vers[k]["kinds"][j]
                buf = get(f"g{gi}.{k}.{j}")
                n = nr * _row_bytes(T, cols)
                if kind == "self":
                    d = qr.self_decode(T, buf, stream=st)[0]
                elif kind == "qr":
                    seed = est.seed()
                    d = qr.decode(T, bytes(buf), [(self._prediction(T, seed, cols), 0, qr.EXPLICIT, cols)], seed, stream=st)
                else:
                    raw = zstd.decompress(buf) if kind == "z" else bytes(buf)
                    d = dev.DeviceArray.from_host(np.frombuffer(raw, np.uint8), st)
                pieces[k].append(d.to_host(stream=st)[:n])
                if k < top:
                    self._learn(est, T, d.view(0, (n,), np.uint8), cols)
        return [np.concatenate(p) if p else np.zeros(0, np.uint8) for p in pieces]
