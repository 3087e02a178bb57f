"""Method M30 (the reference's seedpack/siblings.py): several quantizations of one model without the
model itself. The archive is coded tensor by tensor instead of file by file:

  * identical files, and identical tensors in different files, are stored once;
  * the versions of a tensor (same name and shape; distinct type and bytes) form a chain, most bytes
    first. The first is coded on its own (QR without a seed, qr.self_encode, where that is smaller;
    else zstd level 3; else raw); every later version is QR-coded against an explicit seed: the
    precision-weighted mean of the versions before it (estimate.Est), its scales predicted by the
    quantizer run on that mean;
  * each version is coded in row slices of at most `slice` weights;
  * GGUF headers and the bytes between tensors go into one zstd chunk ("heads"), versions under 1 MiB
    into another ("small").

Chunks: "heads", "g<group>.<version>.<slice>", "small", "manifest" (after the extras the caller
writes). The tensors' content keys are SHA-256 digests here (blake3 in the reference); they decide
only which tensors are equal and are not stored.
"""
import hashlib
import json
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import device as dev
from . import gguf, qr, zstd
from .estimate import Est, half_step
from .gpuquant import GPUQuant
from .requant import QFUN

NAME = "M30 sibling quants: tensor versions coded in chains, no base"     # siblings.py:168
F32, F16, BF16 = 0, 1, 30
FLOATS = {F32: np.float32, F16: np.float16}
SLICE = 1 << 26                          # weights per coding slice (siblings.py:41)
SMALL = 1 << 20                          # versions smaller than this go into the "small" chunk, raw
NEED_IMX = {16, 17, 19}                  # quantizers that assert an importance matrix (siblings.py:43)
_PIECE = 64 << 20


def _row_bytes(T, cols):
    qk, bs = gguf.BLOCK[T]
    return cols // qk * bs


def _read(path, off, n):
    out = np.empty(n, np.uint8)
    with open(path, "rb") as f:
        f.seek(off)
        f.readinto(memoryview(out))
    return out


def _codable(T, cols):
    return T in qr.QR_TYPES and T in QFUN and cols % qr.QK[T] == 0


class M30Siblings:
    name = NAME

    def __init__(self, slice_weights=SLICE, stream=None, verbose=False):
        self.slice, self.stream, self.verbose = slice_weights, stream, verbose
        self.gq = GPUQuant(stream=stream)
        self.sizes = {}

    # ------------------------------------------------------------------ the version estimate
    def _values(self, T, blocks, cols, nw):
        """a version's values and half steps per weight (device float32), or None when its type gives
        none (siblings.py:98-126)"""
        st = self.stream
        if T in FLOATS:
            x = np.frombuffer(blocks.to_host(stream=st).tobytes(), FLOATS[T]).astype(np.float32)
            return dev.DeviceArray.from_host(x, st), dev.DeviceArray(nw, np.float32).zero(st)
        if T == BF16:
            u = np.frombuffer(blocks.to_host(stream=st).tobytes(), np.uint16)
            x = (u.astype(np.uint32) << 16).view(np.float32)
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

    def _add(self, est, T, blocks, cols):
        v = self._values(T, blocks, cols, est.nw)
        if v is not None:
            est.add(*v)

    def _predicted(self, T, x, cols):
        """llama.cpp's quantization of the estimate: the prediction of a version's blocks"""
        imx = np.ones(cols, np.float32) if T in NEED_IMX else None
        return self.gq.quantize_tensors(T, [(x, cols)], [imx], device=True)[0]

    def _seed_x(self, seed):
        """the values of an explicit seed (its even float32 words), as a device array"""
        h = seed.to_host(stream=self.stream).reshape(-1, 2)[:, 0].copy()
        return dev.DeviceArray.from_host(h, self.stream)

    # ------------------------------------------------------------------ pack
    def compress(self, paths, put):
        """paths: {name: path} of the GGUF files; put(chunk name, bytes) -> the manifest dict (its
        "extras" entry left to the caller) and the stored bytes per file"""
        names = sorted(paths)
        info = {n: self._scan(paths[n]) for n in names}
        first_of, fman = {}, []
        for i, n in enumerate(names):
            f = info[n]
            same = first_of.setdefault((f["hash"], f["size"]), i)
            fman.append({"name": n, "size": f["size"], "same": None if same == i else same})
        uniq = [i for i, m in enumerate(fman) if m["same"] is None]
        groups, gid_of = [], {}
        for i in uniq:
            for t, h in info[names[i]]["tensors"]:
                key = (t.name, tuple(t.shape))
                if key not in gid_of:
                    gid_of[key] = len(groups)
                    groups.append({"name": t.name, "shape": list(t.shape), "cols": int(t.shape[0]), "vers": [], "at": []})
                g = groups[gid_of[key]]
                if (t.type, h) not in [(v["type"], v["hash"]) for v in g["vers"]]:
                    g["vers"].append({"type": t.type, "hash": h, "nbytes": t.nbytes})
                    g["at"].append((i, t.offset))
        for g in groups:                       # chain order: most bytes first (ties: first seen)
            order = sorted(range(len(g["vers"])), key=lambda k: -g["vers"][k]["nbytes"])
            g["vers"] = [g["vers"][k] for k in order]
            g["at"] = [g["at"][k] for k in order]
        heads = bytearray()
        for i in uniq:
            f = info[names[i]]
            fman[i]["head"] = [len(heads), len(f["head"])]
            heads += f["head"]
            fman[i]["gaps"] = []
            for o, b in f["gaps"]:
                fman[i]["gaps"].append([o, len(heads), len(b)])
                heads += b
            vidx = {}
            for t, h in f["tensors"]:
                gi = gid_of[(t.name, tuple(t.shape))]
                k = [(v["type"], v["hash"]) for v in groups[gi]["vers"]].index((t.type, h))
                vidx[t.offset] = [gi, k, t.offset, t.nbytes]
            fman[i]["tensors"] = [vidx[o] for o in sorted(vidx)]
        put("heads", zstd.compress_with(bytes(heads), zstd.Params(19, window_log=27, threads=8, ldm=True)))
        self.sizes["headers"] = len(heads)
        small, stored = bytearray(), {}
        for gi, g in enumerate(groups):
            self._code_group(gi, g, names, info, put, small, stored)
        put("small", zstd.zstd_c(bytes(small), 19))
        for g in groups:
            del g["at"]
            for v in g["vers"]:
                del v["hash"]
        seen = set()
        for i in uniq:
            s = 0
            for gi, k, _, _ in fman[i]["tensors"]:
                if (gi, k) not in seen:
                    seen.add((gi, k))
                    s += stored.get((gi, k), 0)
            self.sizes[names[i]] = s
        for i, m in enumerate(fman):
            if m["same"] is not None:
                self.sizes[names[i]] = 0
        return {"method": self.name, "needs": "0.4.0", "slice": self.slice, "files": fman, "groups": groups}

    def _scan(self, path):
        """one read of a GGUF: its SHA-256, header bytes, the bytes between tensors, each tensor's key"""
        size = os.path.getsize(path)
        data = np.memmap(path, np.uint8, "r") if size else np.zeros(0, np.uint8)
        g = gguf.GGUF(data, light=True)
        ts = sorted(g.tensors, key=lambda t: t.offset)
        with ThreadPoolExecutor(8) as ex:
            fh = ex.submit(lambda: hashlib.sha256(memoryview(data)).hexdigest())
            th = list(ex.map(lambda t: hashlib.sha256(memoryview(data[t.offset:t.offset + t.nbytes])).hexdigest(), ts))
            gaps, cur = [], g.data_start
            for t in ts + [None]:
                stop = t.offset if t is not None else size
                if stop > cur:
                    gaps.append((cur, bytes(data[cur:stop])))
                if t is not None:
                    cur = max(cur, t.offset + t.nbytes)
            return {"path": path, "size": size, "hash": fh.result(), "head": bytes(data[:g.data_start]),
                    "gaps": gaps, "tensors": list(zip(ts, th))}

    def _slices(self, g):
        rows = int(np.prod(g["shape"])) // g["cols"]
        per = max(1, self.slice // g["cols"])
        return [(r, min(per, rows - r)) for r in range(0, rows, per)]

    def _code_group(self, gi, g, names, info, put, small, stored):
        cols, vers = g["cols"], g["vers"]
        for v in vers:
            v["kinds"] = []
        if all(v["nbytes"] < SMALL for v in vers):
            for k, v in enumerate(vers):
                i, off = g["at"][k]
                v["small"] = [len(small), v["nbytes"]]
                small += _read(info[names[i]]["path"], off, v["nbytes"]).tobytes()
                del v["kinds"]
            return
        st = self.stream
        for j, (r0, nr) in enumerate(self._slices(g)):
            nw = nr * cols
            est = Est(nw, st) if len(vers) > 1 else None
            for k, v in enumerate(vers):
                T = v["type"]
                i, off = g["at"][k]
                rb = _row_bytes(T, cols)
                raw = _read(info[names[i]]["path"], off + r0 * rb, nr * rb)
                if k == 0:
                    kind, data = self._first(T, raw, cols)
                else:
                    kind, data = "z", None
                    if est is not None and est.x0 is not None and _codable(T, cols):
                        d = dev.DeviceArray.from_host(raw, st)
                        seed = est.seed()
                        P = self._predicted(T, self._seed_x(seed), cols)
                        data = qr.encode(T, [(d, P, 0, qr.EXPLICIT, cols)], seed, stream=st)
                        kind = "qr"
                        if len(data) >= len(raw):
                            kind, data = "z", None
                    if data is None:
                        data = zstd.zstd_c(raw.tobytes(), 3)
                put(f"g{gi}.{k}.{j}", data)
                stored[(gi, k)] = stored.get((gi, k), 0) + len(data)
                v["kinds"].append(kind)
                if est is not None and k + 1 < len(vers):
                    self._add(est, T, dev.DeviceArray.from_host(raw, st), cols)

    def _first(self, T, raw, cols):
        """the chain's first version: QR without a seed (grid types too) where smaller, else zstd level
        3 where smaller, else raw (siblings.py:422-429)"""
        if T in qr.QR_TYPES and cols % qr.QK[T] == 0:
            c = qr.self_encode(T, [(raw, cols)], stream=self.stream)
            if len(c) < len(raw):
                return "self", c
        c = zstd.zstd_c(raw.tobytes(), 3)
        return ("z", c) if len(c) < len(raw) else ("raw", raw.tobytes())

    # ------------------------------------------------------------------ unpack
    def decompress(self, man, get, want, sink):
        """the wanted GGUF files of an M30 archive: sink(name, bytes) for each (the versions of a
        chain are decoded once and kept for the other files that hold them)"""
        self.slice = man["slice"]
        fm, groups = man["files"], man["groups"]
        heads = zstd.decompress(get("heads"))
        smallb = zstd.decompress(get("small")) if any("small" in v for g in groups for v in g["vers"]) else b""
        cache = {}

        def version(gi, k):
            if (gi, k) not in cache:
                for kk, piece in self._chain(get, groups[gi], gi, k, smallb):
                    cache[(gi, kk)] = piece
            return cache[(gi, k)]

        for i, m in enumerate(fm):
            if m["name"] not in want:
                continue
            src = fm[m["same"]] if m["same"] is not None else m
            out = np.zeros(src["size"], np.uint8)
            h0, hn = src["head"]
            out[:hn] = np.frombuffer(heads, np.uint8, hn, h0)
            for o, s0, ln in src["gaps"]:
                out[o:o + ln] = np.frombuffer(heads, np.uint8, ln, s0)
            for gi, k, off, nb in src["tensors"]:
                out[off:off + nb] = version(gi, k)
            sink(m["name"], out)

    def _chain(self, get, g, gi, top, smallb):
        """versions 0..top of group g, whole (slices joined): (k, host uint8 array)"""
        vers = g["vers"]
        if "small" in vers[0]:
            for k in range(top + 1):
                a, n = vers[k]["small"]
                yield k, np.frombuffer(smallb, np.uint8, n, a)
            return
        cols, st = g["cols"], self.stream
        parts = {k: [] for k in range(top + 1)}
        for j, (r0, nr) in enumerate(self._slices(g)):
            nw = nr * cols
            est = Est(nw, st) if top > 0 else None
            for kk in range(top + 1):
                v = vers[kk]
                T, kind = v["type"], v["kinds"][j]
                buf = get(f"g{gi}.{kk}.{j}")
                n = nr * _row_bytes(T, cols)
                if kind == "self":
                    d = qr.self_decode(T, buf, stream=st)[0]
                elif kind == "qr":
                    seed = est.seed()
                    P = self._predicted(T, self._seed_x(seed), cols)
                    d = qr.decode(T, bytes(buf), [(P, 0, qr.EXPLICIT, cols)], seed, stream=st)
                elif kind == "z":
                    d = dev.DeviceArray.from_host(np.frombuffer(zstd.decompress(buf), np.uint8), st)
                else:
                    d = dev.DeviceArray.from_host(np.frombuffer(bytes(buf), np.uint8), st)
                host = d.to_host(stream=st)[:n]
                parts[kk].append(host)
                if kk < top:
                    self._add(est, T, d.view(0, (n,), np.uint8), cols)
        for k in range(top + 1):
            yield k, np.concatenate(parts[k]) if parts[k] else np.zeros(0, np.uint8)
