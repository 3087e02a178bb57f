"""Fitted importance sets of a repository pack (the reference's repo3.py:1240-1355 over imxfit.py).

A quant file whose GGUF metadata names an importance matrix other than the repository's (its
`quantize.imatrix.chunks_count` differs from the published imatrix's chunk count) belongs to the set
of files made with that matrix, keyed by (chunk count, dataset); sets are numbered from 1 in order of
their first file. Inputs are the published importance vectors: tensors whose importance has the same
bytes (gate and up, q / k / v) share one input.

Fitting. The importance of each input that a set's legacy-quant tensors (Q4_0, Q4_1, Q5_0, Q5_1) use
is fitted once, from the first file of the set that holds such a tensor, window by window as that
file is coded (the base tensors are then in HBM):
  * the Gram sums of every tensor of the input in the window (imxfit.ls_gram over pieces of FIT_ROWS
    weights, in tensor then row order, added as a running float64 sum that starts at the first piece);
  * the fitted vector is ls_solve of that sum, scaled per block like the published vector;
  * it is checked on the last max(64, FIT_ROWS / 8 / cols) rows of the input's first tensor
    (imxfit.equal_blocks) and kept when it reproduces more than half a percent more blocks than the
    published vector there; either way the input is no longer waiting.
The files of a set are predicted with the kept vectors (fitted variant 1000 k + u).

The "imx" chunk: pack({"meta": zstd JSON [{"chunks", "dataset", "groups": [[names], ...]}, ...] per
set in order, "data": zstd-19 of the fitted vectors' float32 bits XOR the published ones', group by
group}); the archive has none when no set kept a fit.
"""
import dataclasses
import functools
import json
import operator
import time

import numpy as np

from . import imxfit, zstd
from .framing import pack, unpack
from .requant import QFUN

FIT_ROWS = 1 << 24                   # weights per piece of a tensor in the fit (repo3.py:1246)
GAIN = 0.005                         # a fit is kept above this gain in reproduced blocks (repo3.py:1317)
F32, F16, BF16 = 0, 1, 30


@dataclasses.dataclass
class Fit:
    names: list                      # the inputs sharing the importance
    fitted: np.ndarray
    published: np.ndarray
    before: float                    # check share with the published vector
    after: float                     # with the fitted one


@dataclasses.dataclass
class FitSet:
    chunks: int
    dataset: str
    files: list                      # file indices
    waiting: set = dataclasses.field(default_factory=set)
    kept: list = dataclasses.field(default_factory=list)

    def importance(self):
        """{tensor name: fitted importance} of the kept fits"""
        return {n: f.fitted for f in self.kept for n in f.names}


def _key(e):
    return np.asarray(e, np.float32).tobytes()


class FitSets:
    """the pack's fitted sets: plan(), then fit_window() per window of a set's first files, chunk()"""

    def __init__(self):
        self.sets = {}               # k (from 1) -> FitSet
        self.set_of = {}             # file index -> k
        self.inputs = {}             # published importance bytes -> names sharing it, in imatrix order
        self.imx = {}
        self.seconds = 0.0

    @classmethod
    def plan(cls, names, heads, imx_all, published_chunks):
        """names: the derived files in archive order; heads: {name: (metadata, tensors)}; imx_all: the
        published importance {tensor name: vector}; published_chunks: its chunk count (None: no sets)"""
        fs = cls()
        if published_chunks is None or not imx_all:
            return fs
        fs.imx = imx_all
        for n, e in imx_all.items():
            fs.inputs.setdefault(_key(e), []).append(n)
        for fi, n in enumerate(names):
            meta = heads[n][0]
            cc = meta.get("quantize.imatrix.chunks_count")
            if cc is None or int(cc) == published_chunks:
                continue
            sig = (int(cc), str(meta.get("quantize.imatrix.dataset", "")))
            k = next((k for k, s in fs.sets.items() if (s.chunks, s.dataset) == sig), len(fs.sets) + 1)
            fs.sets.setdefault(k, FitSet(*sig, [])).files.append(fi)
            fs.set_of[fi] = k
        for s in fs.sets.values():
            for fi in s.files:
                for t in heads[names[fi]][1]:
                    if t.type in imxfit.LS_TYPES and t.name in imx_all:
                        s.waiting.update(fs.inputs[_key(imx_all[t.name])])
        return fs

    def waiting(self, k):
        return bool(k in self.sets and self.sets[k].waiting)

    def importance(self, k):
        return self.sets[k].importance() if k in self.sets else {}

    def fit_window(self, k, tensors, base_of, rows, blocks, gq, stream=None):
        """fit set k's waiting inputs from a window's legacy-quant tensors of its file.
        base_of(name) -> the base tensor or None; rows(base tensor, r0, r1) -> its rows as float32
        (r1 - r0, cols) on the device; blocks(tensor, r0, r1) -> the file's blocks of those rows"""
        s = self.sets[k]
        t0 = time.perf_counter()
        members = {}
        for t in tensors:
            e, bt = self.imx.get(t.name), base_of(t.name)
            usable = t.name in s.waiting and t.type in imxfit.LS_TYPES and e is not None and bt is not None \
                and bt.type in (F32, F16, BF16) and len(e) == bt.shape[0]
            if usable:
                members.setdefault(_key(e), []).append((t, bt))
        for key, tb in members.items():
            pieces = (imxfit.ls_gram(gq, t.type, rows(bt, r0, r1), blocks(t, r0, r1), stream=stream)
                      for t, bt in tb for r0, r1 in _row_pieces(bt))
            published = np.frombuffer(key, np.float32)
            fitted = imxfit.ls_solve(functools.reduce(operator.add, pieces), published)
            t, bt = tb[0]
            nrow, cols = int(bt.shape[1]), int(bt.shape[0])
            last = min(nrow, max(64, FIT_ROWS // 8 // cols))
            x, f = rows(bt, nrow - last, nrow), blocks(t, nrow - last, nrow)
            before = imxfit.equal_blocks(gq, t.type, x, f, published)
            after = imxfit.equal_blocks(gq, t.type, x, f, fitted)
            names = self.inputs[key]
            s.waiting.difference_update(names)
            if after > before + GAIN:
                s.kept.append(Fit(names, fitted, published, before, after))
        self.seconds += time.perf_counter() - t0

    def fitted_inputs(self):
        return sum(len(s.kept) for s in self.sets.values())

    def chunk(self):
        """-> ("imx" chunk bytes, manifest entry) or None when no fit was kept"""
        if not self.fitted_inputs():
            return None
        meta = [{"chunks": s.chunks, "dataset": s.dataset, "groups": [f.names for f in s.kept]}
                for _, s in sorted(self.sets.items())]
        bits = b"".join((f.fitted.view(np.uint32) ^ f.published.view(np.uint32)).tobytes()
                        for _, s in sorted(self.sets.items()) for f in s.kept)
        body = pack({"meta": zstd.zstd_c(json.dumps(meta).encode()), "data": zstd.zstd_c(bits, 19)})
        return body, {"chunk": "imx", "sets": len(meta)}


def _row_pieces(bt):
    cols, nrow = int(bt.shape[0]), int(bt.shape[1])
    step = max(1, FIT_ROWS // cols)
    return [(r0, min(nrow, r0 + step)) for r0 in range(0, nrow, step)]


def read_chunk(buf, imx_all):
    """an archive's "imx" chunk -> {set k: {tensor name: fitted importance}} (repo3.py:1342-1355)"""
    parts = unpack(memoryview(bytes(buf)))
    meta = json.loads(zstd.decompress(parts["meta"]))
    bits = np.frombuffer(zstd.decompress(parts["data"]), np.uint32)
    out, at = {}, 0
    for k, entry in enumerate(meta, 1):
        out[k] = {}
        for names in entry["groups"]:
            published = np.asarray(imx_all[names[0]], np.float32).view(np.uint32)
            fitted = (bits[at:at + published.size] ^ published).view(np.float32)
            at += published.size
            out[k].update({n: fitted for n in names})
    return out
