"""Writes R2 (BF16 base codec) golden vectors by running the reference's own code on the CPU: its
side-information statistics (bf16v2.BF16v2._stats, with detmath), duplicate-row detection (_dups,
row_hash), table normalisation (gpu2.normalize_gpu) and its v2_hist / v2_enc / v2_dec kernels,
through the reference's --cpu backend (seedpack/cpu.py, seedpack/cpukernels.py). Run in the build
container only:

    python tests/golden/make_r2_golden.py            # r2_vectors.npz
    python tests/golden/make_r2_golden.py --header   # header_vectors.npz: the "rest" part's forms

bf16v2.py and gpu2.py import numba / zstandard (absent here), so the functions and the kernel text
are read with `ast` and executed against the --cpu backend; the driver steps of
BF16v2._analyse / _encode (bf16v2.py:323-411: per group of tensors, statistics, dedup, histogram;
normalisation; encode, gather) are restated below without the GGUF parsing and header coding.
Nothing here runs on the GPU box or at test time: the output is data (r2_vectors.npz).
"""
import argparse
import ast
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, ROOT)

os.environ["SEEDPACK_CPU"] = "1"
# the reference's --cpu backend caches its compiled kernels; a temporary directory keeps them out of
# the repository
os.environ.setdefault("SEEDPACK_CACHE", tempfile.mkdtemp(prefix="seedpack_refcache_"))
sys.path.insert(0, REF)

from tests.golden.r2_cases import CASES, case_file  # noqa: E402

PB = 15


def _source(path):
    src = open(path).read()
    return src, ast.parse(src)


def load():
    from seedpack import cpu as cp
    from seedpack import cpukernels, detmath
    src, tree = _source(os.path.join(REF, "seedpack", "bf16v2.py"))
    ns = {"np": np, "cp": cp, "detmath": detmath, "K": 8, "SEG": 16384, "NE": 512, "NM": 128, "NS": 16,
          "TPT": 656, "PB": PB}
    kernels = None
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "KERNELS" for t in node.targets):
            # KERNELS = r\"\"\"...\"\"\".replace("%(PB)d", str(PB))
            kernels = ast.literal_eval(node.value.func.value).replace("%(PB)d", str(PB))
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) in ("TB_DT", "SG_DT") for t in node.targets):
            exec(ast.get_source_segment(src, node), ns)
        if isinstance(node, ast.ClassDef) and node.name == "BF16v2":
            for fn in node.body:
                if isinstance(fn, ast.FunctionDef) and fn.name in ("_stats", "_dups", "_bases", "_plan", "_groups"):
                    code = ast.get_source_segment(src, fn)
                    code = "\n".join(line[4:] if line.startswith("    ") else line for line in code.splitlines())
                    code = code.replace("@staticmethod\n", "")
                    exec(code, ns)
    gsrc, gtree = _source(os.path.join(REF, "seedpack", "gpu2.py"))
    for node in gtree.body:
        if isinstance(node, ast.FunctionDef) and node.name == "normalize_gpu":
            exec(ast.get_source_segment(gsrc, node), ns)
    mod = cpukernels.RawModule(code=kernels, options=("-std=c++17",))
    ns["kern"] = mod.get_function
    return ns, cp


class _Self:
    """the attributes the extracted methods use"""

    def __init__(self, ns, group_bytes):
        self.group_bytes = group_bytes
        self._bases = lambda layout: ns["_bases"](layout)


def compress(ns, cp, data, layout, group_bytes):
    """bf16v2.py:323-411 (pass 1 and pass 2) without the GGUF layer -> the coded parts"""
    me = _Self(ns, group_bytes)
    groups = ns["_groups"](me, layout)
    rb, cb, nrow, ncol = ns["_bases"](layout)
    rfi = np.zeros(nrow, np.int16); cfi = np.zeros(ncol, np.int16); scl = np.zeros(ncol, np.int8)
    nrows_c, dup_pairs, plans = {}, {}, {}
    counts = np.zeros((layout["nroles"] * 656, 256), np.uint32)
    rmap_all, nrm = [], 0
    host = np.frombuffer(data, np.uint8)
    for gi, grp in enumerate(groups):
        a = layout["t"][grp[0]][0]
        b = layout["t"][grp[-1]][0] + layout["t"][grp[-1]][1]
        dev = cp.asarray(host[a:b].copy())
        rmap_off, mine = {}, []
        for i in grp:
            off, nb, rl, _ = layout["t"][i]
            d = dev[off - a:off - a + nb]
            r_, c_, s_ = ns["_stats"](me, d, rl)
            rfi[rb[i]:rb[i] + len(r_)] = np.asarray(r_); cfi[cb[i]:cb[i] + rl] = np.asarray(c_)
            scl[cb[i]:cb[i] + rl] = np.asarray(s_)
            keep, pairs = ns["_dups"](me, d, rl, host[off:off + nb].view(np.uint16))
            nrows_c[i] = nb // 2 // rl if keep is None else len(keep)
            if keep is not None:
                rmap_off[i] = nrm; nrm += len(keep); rmap_all.append(keep); mine.append(keep)
                dup_pairs[i] = pairs
        plans[gi] = ns["_plan"](me, layout, gi, grp, nrows_c, rmap_off)
        tb, sg = plans[gi]
        if mine:
            tb = tb.copy(); m = tb["rmap"] >= 0; tb["rmap"][m] -= min(rmap_off.values())
            rm = np.concatenate(mine).astype(np.int32)
        else:
            rm = np.zeros(1, np.int32)
        ns["kern"]("v2_hist")(((len(sg) + 63) // 64,), (64,),
                              (dev, tb.view(np.uint8), sg.view(np.uint8), np.int32(len(sg)), rfi, cfi, scl, rm, counts))
    rowmap = np.concatenate(rmap_all).astype(np.int32) if rmap_all else np.zeros(1, np.int32)
    freq, used = ns["normalize_gpu"](cp.asarray(counts), 1 << PB)
    freq, used = np.asarray(freq), np.asarray(used)
    remap = np.full(counts.shape[0], -1, np.int32); remap[used] = np.arange(len(used), dtype=np.int32)
    cum = np.zeros((len(freq), 257), np.uint32); cum[:, 1:] = np.cumsum(freq.astype(np.uint32), axis=1)
    cap = 16384 * 2 + 1024
    streams, lens_all = [], []
    for gi, grp in enumerate(groups):
        a = layout["t"][grp[0]][0]
        b = layout["t"][grp[-1]][0] + layout["t"][grp[-1]][1]
        dev = host[a:b].copy()
        tb, sg = plans[gi]
        out = np.zeros(len(sg) * cap, np.uint8); out_len = np.zeros(len(sg), np.uint32)
        ns["kern"]("v2_enc")(((len(sg) + 63) // 64,), (64,),
                             (dev, tb.view(np.uint8), sg.view(np.uint8), np.int32(len(sg)), rfi, cfi, scl, rowmap,
                              remap, freq, cum, out, np.uint64(cap), out_len))
        assert not (out_len == 0xFFFFFFFF).any()
        streams.append(b"".join(out[(s + 1) * cap - out_len[s]:(s + 1) * cap].tobytes() for s in range(len(sg))))
        lens_all.append(out_len.copy())
    return dict(rfi=rfi, cfi=cfi, scl=scl, counts=counts, freq=freq, used=used.astype(np.int32),
                lens=np.concatenate(lens_all).astype(np.uint32), stream=np.frombuffer(b"".join(streams), np.uint8),
                nrows_c=np.array([nrows_c[i] for i in range(len(layout["t"]))], np.int64),
                dups=np.array([[i, r, s] for i, ps in dup_pairs.items() for r, s in ps], np.int64).reshape(-1, 3),
                rowmap=rowmap, groups=np.array([len(g) for g in groups], np.int64)), (groups, plans, remap, cum)


def decode(ns, data, layout, res, aux):
    """v2_dec of the reference on the coded parts (bf16v2.py:422-486 without the header): round trip"""
    groups, plans, remap, cum = aux
    freq = res["freq"]
    lut = np.zeros((len(freq), 1 << PB), np.uint8)
    ns["kern"]("build_lut")((len(freq),), (256,), (cum, np.int32(len(freq)), lut))
    out = np.frombuffer(data, np.uint8).copy()
    spos, lpos = 0, 0
    stream = res["stream"]
    for gi, grp in enumerate(groups):
        tb, sg = plans[gi]
        gl = res["lens"][lpos:lpos + len(sg)]; lpos += len(sg)
        nb_ = int(gl.sum(dtype=np.uint64))
        offs = np.zeros(len(sg), np.uint64); offs[1:] = np.cumsum(gl.astype(np.uint64))[:-1]
        a = layout["t"][grp[0]][0]; b = layout["t"][grp[-1]][0] + layout["t"][grp[-1]][1]
        dev = np.zeros(b - a, np.uint8)
        ns["kern"]("v2_dec")(((len(sg) + 63) // 64,), (64,),
                             (stream[spos:spos + nb_].copy(), offs, dev, tb.view(np.uint8), sg.view(np.uint8),
                              np.int32(len(sg)), res["rfi"], res["cfi"], res["scl"], res["rowmap"], remap, freq, cum, lut))
        spos += nb_
        for i, r, s in res["dups"]:
            if i in grp:
                off, nb, rl, _ = layout["t"][i]
                u = dev[off - a:off - a + nb].view(np.uint16).reshape(-1, rl)
                u[r] = u[s]
        for i in grp:
            off, nb, _, _ = layout["t"][i]
            out[off:off + nb] = dev[off - a:off - a + nb]
    return out.tobytes()


def load_header_coder():
    """the reference's header coder (gpu2.py:299-431, gpu_bf16.py:421-424), read with `ast`:
    rest_of, xz_chunks_c, _items, _xz, header_pairs_c and M24BF16GPU._header_c"""
    import lzma
    import struct
    from concurrent.futures import ThreadPoolExecutor
    ns = {"np": np, "lzma": lzma, "struct": struct, "ThreadPoolExecutor": ThreadPoolExecutor}
    src, tree = _source(os.path.join(REF, "seedpack", "gpu2.py"))
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "HEADER_CHUNKS" for t in node.targets):
            exec(ast.get_source_segment(src, node), ns)
        if isinstance(node, ast.FunctionDef) and node.name in ("rest_of", "xz_chunks_c", "_items", "_xz",
                                                              "header_pairs_c", "header_tok_c"):
            exec(ast.get_source_segment(src, node), ns)
        if isinstance(node, ast.ClassDef) and node.name == "GPU2":          # the Q8_0 codec's header coder
            for fn in node.body:
                if isinstance(fn, ast.FunctionDef) and fn.name == "_header_c":
                    code = ast.get_source_segment(src, fn)
                    code = "\n".join(line[4:] if line.startswith("    ") else line for line in code.splitlines())
                    exec(code.replace("def _header_c", "def q8_header_c"), ns)
    bsrc, btree = _source(os.path.join(REF, "seedpack", "gpu_bf16.py"))
    for node in btree.body:
        if isinstance(node, ast.ClassDef) and node.name == "M24BF16GPU":
            for fn in node.body:
                if isinstance(fn, ast.FunctionDef) and fn.name == "_header_c":
                    code = ast.get_source_segment(bsrc, fn)
                    code = "\n".join(line[4:] if line.startswith("    ") else line for line in code.splitlines())
                    exec(code.replace("@staticmethod\n", ""), ns)
    return ns


def main_header():
    """header_vectors.npz: per case of header_cases.py, the SHA-256 of the input file and the
    reference's "rest" part for it (P or X form), and the Q8_0 codec's (P, T or X form)"""
    from seedpack_amd import gguf
    from tests.golden.header_cases import NAMES, case_file
    ns = load_header_coder()
    out = {}
    for name in NAMES:
        data, layout = case_file(name)
        g = gguf.GGUF(data)                 # spans / data_start: the reference reader's meaning
        part = ns["_header_c"](data, g, layout)
        out[f"{name}/input_sha256"] = np.frombuffer(hashlib.sha256(data).digest(), np.uint8)
        out[f"{name}/rest"] = np.frombuffer(part, np.uint8)
        # the Q8_0 codec's (M22: TOKPAIRS and TOKZ set, gpu3.py:248, :583-584) on the same file
        q8 = ns["q8_header_c"](type("M22", (), {"TOKPAIRS": True, "TOKZ": True})(), data, g, layout)
        out[f"{name}/rest_q8"] = np.frombuffer(q8, np.uint8)
        print(f"{name}: Q8_0 codec header {q8[:1].decode()} form, {len(q8)} B", flush=True)
        print(f"{name}: {len(data)} B file, {part[:1].decode()} form, {len(part)} B", flush=True)
    np.savez_compressed(os.path.join(HERE, "header_vectors.npz"), **out)


def main():
    ns, cp = load()
    out = {}
    for name, *_ in CASES:
        data, layout, group_bytes = case_file(name)
        res, aux = compress(ns, cp, data, layout, group_bytes)
        assert decode(ns, data, layout, res, aux) == data, "reference R2 does not round-trip"
        for k, v in res.items():
            out[f"{name}/{k}"] = v
        print(f"{name}: {len(layout['t'])} tensors, {len(res['groups'])} groups, {len(res['lens'])} segments, "
              f"{len(res['dups'])} duplicate rows, {len(res['used'])} tables, stream {len(res['stream'])} B "
              f"of {sum(t[1] for t in layout['t'])} B", flush=True)
    np.savez_compressed(os.path.join(HERE, "r2_vectors.npz"), **out)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--header", action="store_true", help="write header_vectors.npz only")
    if ap.parse_args().header:
        main_header()
    else:
        main()
