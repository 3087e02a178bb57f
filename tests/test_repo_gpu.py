"""Whole-repository archives on the GPU (configurations 4 and 5 at reduced sizes): a synthetic
Qwen-shaped repository (BF16 base with a BPE tokenizer, imatrix, 21 quantized GGUFs made from the
base with 1% of their blocks changed, a small extra file) packed into a .seedpack archive and
extracted again.

Checked: every file extracts byte-identical and passes its checksum (so every QR batch of every file
decodes back); the container, manifest and chunks follow the reference's layout; the base's header
part takes the tokenizer-aware form; for every QR type, one batch of the archive equals the oracle's
stream for the same tensors (oracle/qr.py's per-tensor histograms summed into the batch's tables,
each tensor's segments coded with them); windows, references and QR batch cuts follow the
reference's rules (repo3.py:1689-1706, :2006-2030, :946-979)."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import qr as oqr
from seedpack_amd import container, device as dev, gguf, qr, repo, synth, zstd
from seedpack_amd.framing import unpack
from seedpack_amd.requant import NAMES

pytestmark = pytest.mark.gpu
TYPES = [2, 3, 6, 7, 8, 42, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _files():
    f = {f"model-{NAMES[t]}.gguf": (lambda name, t=t: t) for t in TYPES}
    f["model-Q4_K_M.gguf"] = synth.q4_k_m
    return f


@pytest.fixture(scope="module")
def small_repo(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("repo"))
    say("case repo small: writing the synthetic repository")
    tensors = synth.qwen_tensors(layers=2, hidden=256, ffn=512, kv=256, vocab=512)
    sizes = synth.write_repo(root, tensors, _files(), per_million=20000, nmerge=3000)
    arc = os.path.join(str(tmp_path_factory.mktemp("arc")), "small.seedpack")
    say("case repo small: pack")
    stats = repo.pack_repo([root], arc)
    return root, arc, sizes, stats


def test_small_repo_extracts_byte_identical(small_repo, tmp_path):
    root, arc, sizes, stats = small_repo
    say("case repo small: unpack", stats)
    out = str(tmp_path / "out")
    res = repo.unpack_repo(arc, out)
    assert not res["bad"] and not res["missing"], res
    names = sorted(os.listdir(root))
    assert sorted(res["files"]) == names
    for n in names:
        a, b = open(os.path.join(root, n), "rb").read(), open(os.path.join(out, n), "rb").read()
        assert a == b, n
    # selective extraction: one quant file alone
    res = repo.unpack_repo(arc, None, ["model-IQ2_XS.gguf"])
    assert res["files"] == {"model-IQ2_XS.gguf": True}
    assert stats["stats"]["qr"] > 0 and stats["stats"]["requant_diff"] > 0
    # the base not in HBM (a base bigger than HBM): decoded window by window from the archive, its
    # own file written through the same decoder
    out2 = str(tmp_path / "out2")
    res = repo.Unpacker(bases_in_hbm=False).run(arc, out2)
    assert not res["bad"] and not res["missing"], res
    for n in names:
        assert open(os.path.join(root, n), "rb").read() == open(os.path.join(out2, n), "rb").read(), n


def _rewrite(src, dst, meta=None, manifest=None):
    """a copy of archive src with its catalog (meta) and / or manifest replaced"""
    r = container.Reader(src)
    w = container.Writer(dst)
    for name in r.chunks:
        if name == "manifest" and manifest is not None:
            w.put(name, zstd.compress(json.dumps(manifest).encode(), 19))
        else:
            w.put(name, bytes(r.get(name)))
    w.close(meta if meta is not None else r.meta)
    r.close()


def test_small_repo_catalog_hash_and_gates(small_repo, tmp_path):
    """the catalog holds BLAKE3 digests (the reference's checksum when its blake3 requirement is
    installed, cli.py:48-53), computed on the device for the base and the derived files: each equals
    the host hasher's. An archive whose manifest needs a newer reader, or whose catalog names a
    checksum this reader does not compute, is refused before any file is written (with verify=False
    the latter extracts unchecked). A SHA-256 catalog (hash_algo="sha256") has the same chunks and
    extracts checked."""
    import hashlib
    from seedpack_amd import blake3
    root, arc, sizes, stats = small_repo
    say("case repo small: catalog hash and reader gates")
    r = container.Reader(arc)
    meta, man, chunks = r.meta, json.loads(zstd.decompress(r.get("manifest"))), dict(r.chunks)
    r.close()
    assert meta["hash"] == "blake3"
    for f in meta["files"]:
        assert f["hash"] == blake3.hexdigest(open(os.path.join(root, f["name"]), "rb").read()), f["name"]
    newer = str(tmp_path / "newer.seedpack")
    _rewrite(arc, newer, manifest={**man, "needs": "9.0.0"})
    out = tmp_path / "o1"
    with pytest.raises(container.FormatError, match="needs SeedPack 9.0.0"):
        repo.unpack_repo(newer, str(out))
    assert not out.exists() or not any(out.iterdir())
    odd = str(tmp_path / "odd.seedpack")
    _rewrite(arc, odd, meta={**meta, "hash": "xxh3"})
    out = tmp_path / "o2"
    with pytest.raises(container.FormatError, match="catalog hash"):
        repo.unpack_repo(odd, str(out))
    assert not out.exists() or not any(out.iterdir())
    with pytest.warns(UserWarning, match="unchecked"):
        res = repo.Unpacker(verify=False).run(odd, str(out), ["model-Q4_K.gguf", "README.md"])
    assert sorted(res["unchecked"]) == ["README.md", "model-Q4_K.gguf"] and not res["bad"]
    for n in res["files"]:
        assert open(os.path.join(root, n), "rb").read() == (out / n).read_bytes(), n
    sha = str(tmp_path / "sha.seedpack")
    repo.Packer(hash_algo="sha256").pack([root], sha)
    r = container.Reader(sha)
    assert r.meta["hash"] == "sha256"
    for f in r.meta["files"]:
        assert f["hash"] == hashlib.sha256(open(os.path.join(root, f["name"]), "rb").read()).hexdigest()
    assert {k: v[1:] for k, v in r.chunks.items()} == {k: v[1:] for k, v in chunks.items()}
    r.close()
    res = repo.unpack_repo(sha, str(tmp_path / "o3"))
    assert not res["bad"] and not res["missing"] and not res["unchecked"], res


def test_small_repo_damaged_base_chunk(small_repo, tmp_path):
    """a byte flipped inside the base chunk's coded stream: the extract, which decodes the base as its
    stream arrives, stops with a CRC error once the chunk is read, and leaves no base or quant file and
    no .part file behind (the small files of the extras bundle, verified on their own, may be
    written)"""
    from seedpack_amd.framing import index
    root, arc, sizes, stats = small_repo
    say("case repo small: damaged base chunk")
    r = container.Reader(arc)
    off, n, _ = r.chunks["b0"]

    def read(o, k):
        return bytes(r.read_at("b0", o, k))
    parts = index(read, n)
    parts = index(read, parts["r2"][1], parts["r2"][0])
    so, sn = parts["stream"]
    r.close()
    raw = bytearray(open(arc, "rb").read())
    raw[off + so + sn // 2] ^= 0x5A
    bad = str(tmp_path / "bad.seedpack")
    open(bad, "wb").write(bytes(raw))
    out = tmp_path / "out"
    with pytest.raises(container.FormatError, match="CRC"):
        repo.unpack_repo(bad, str(out))
    left = sorted(p.name for p in out.rglob("*")) if out.exists() else []
    assert not any(x.endswith(".part") or x.endswith(".gguf") for x in left), left


def test_small_repo_pack_is_deterministic(small_repo, tmp_path):
    """two packs of the same files with the same creation time give the same archive bytes (the
    pipeline's threads and processing order do not show in the archive), and so does a pack under
    tight memory: one file's residual in HBM at a time, every QR batch waited for as it is queued"""
    root, arc, sizes, stats = small_repo
    a, b, c = (str(tmp_path / f"{k}.seedpack") for k in "abc")
    repo.Packer(zstd_lanes=3, coders=1).pack([root], a, created="2026-01-01T00:00:00")
    repo.Packer().pack([root], b, created="2026-01-01T00:00:00")
    assert open(a, "rb").read() == open(b, "rb").read()
    tight = repo.Packer(zstd_lanes=2, coders=2, device_bytes=1 << 20)
    tight.QR_HOLD = 0
    tight.pack([root], c, created="2026-01-01T00:00:00")
    assert open(a, "rb").read() == open(c, "rb").read()
    # the base in host memory (a base bigger than HBM): coded in groups of 1 MiB, its tensors
    # uploaded window by window for the derived files
    d = str(tmp_path / "d.seedpack")
    host = repo.Packer(bases_in_hbm=False)
    host.BASE_GROUP = 1 << 20
    host.pack([root], d, created="2026-01-01T00:00:00")
    assert open(a, "rb").read() == open(d, "rb").read()


def test_small_repo_method_m28(small_repo, tmp_path):
    """method m28: the base chunk is M24's parts (layout, side, tables, lens, stream, rest); every file
    extracts byte-identical, also when the bases are asked to stay out of HBM"""
    root, arc, sizes, stats = small_repo
    a = str(tmp_path / "m28.seedpack")
    repo.pack_repo([root], a, method="m28")
    r = container.Reader(a)
    man = json.loads(zstd.decompress(r.get("manifest")))
    assert man["method"] == repo.METHODS["m28"]
    assert list(unpack(memoryview(r.get("b0")))) == ["layout", "side", "tables", "lens", "stream", "rest"]
    out = str(tmp_path / "out28")
    res = repo.unpack_repo(a, out)
    assert not res["bad"] and not res["missing"], res
    for n in sorted(os.listdir(root)):
        assert open(os.path.join(root, n), "rb").read() == open(os.path.join(out, n), "rb").read(), n
    # bases kept out of HBM where they can be: an M24 base has no random access and is still decoded
    # whole (the decision is per base, repo3.py:2311-2321)
    res = repo.Unpacker(bases_in_hbm=False).run(a, None, ["model-Q4_K.gguf", "model-BF16.gguf"])
    assert res["files"] == {"model-Q4_K.gguf": True, "model-BF16.gguf": True}, res


@pytest.fixture(scope="module")
def sibling_repo(tmp_path_factory):
    """a BF16 model of 1 MiB+ tensors and five quantizations of it"""
    root = str(tmp_path_factory.mktemp("siblings"))
    say("case m30: writing the synthetic repository")
    tensors = synth.qwen_tensors(layers=1, hidden=1024, ffn=1024, kv=256, vocab=1024)
    files = {f"model-{NAMES[t]}.gguf": (lambda name, t=t: t) for t in (8, 14, 12, 17, 2)}
    synth.write_repo(root, tensors, files, per_million=20000, nmerge=1000)
    return root


@pytest.mark.parametrize("with_base", [True, False])
def test_method_m30(sibling_repo, tmp_path, with_base):
    """method m30 (sibling quants, no base): the repository's GGUFs coded as tensor version chains in
    slices (a slice of 256K weights here, so the 1M-weight tensors take several), identical files
    stored once; every file extracts byte-identical. Without the BF16 file the chains start at the
    Q8_0 versions."""
    import shutil
    root = sibling_repo
    src = str(tmp_path / "src")
    os.makedirs(src)
    for n in os.listdir(root):
        if with_base or n != "model-BF16.gguf":
            shutil.copy(os.path.join(root, n), src)
    shutil.copy(os.path.join(root, "model-Q4_K.gguf"), os.path.join(src, "copy-Q4_K.gguf"))   # identical file
    a = str(tmp_path / "m30.seedpack")
    say(f"case m30: pack (with the BF16 file: {with_base})")
    repo.pack_repo([src], a, method="m30", m30_slice=1 << 18)
    r = container.Reader(a)
    man = json.loads(zstd.decompress(r.get("manifest")))
    assert man["method"] == repo.METHODS["m30"] and man["slice"] == 1 << 18 and man["needs"] == "0.4.0"
    chunks = list(r.chunks)
    assert chunks[:2] == ["extras", "heads"] and chunks[-2:] == ["small", "manifest"]
    same = {m["name"]: m["same"] for m in man["files"]}
    names = [m["name"] for m in man["files"]]
    assert names[same["model-Q4_K.gguf"]] == "copy-Q4_K.gguf" or names[same["copy-Q4_K.gguf"]] == "model-Q4_K.gguf"
    kinds = {k for g in man["groups"] for v in g["vers"] for k in v.get("kinds", [])}
    assert "qr" in kinds and max(len(g["vers"]) for g in man["groups"]) >= 5
    assert any(len(v.get("kinds", [])) > 1 for g in man["groups"] for v in g["vers"])     # several slices
    out = str(tmp_path / "out30")
    res = repo.unpack_repo(a, out)
    assert not res["bad"] and not res["missing"], res
    for n in sorted(os.listdir(src)):
        assert open(os.path.join(src, n), "rb").read() == open(os.path.join(out, n), "rb").read(), n


def _gguf_file(path, kv, tensors):
    """a GGUF of [(name, shape, type, payload bytes)]"""
    head, where, size = gguf.header_bytes(kv, [(n, sh, t) for n, sh, t, _ in tensors])
    out = np.zeros(size, np.uint8)
    out[:len(head)] = np.frombuffer(head, np.uint8)
    for (_, _, _, payload), (off, nb) in zip(tensors, where):
        out[off:off + nb] = np.frombuffer(payload, np.uint8)
    with open(path, "wb") as f:
        f.write(out.tobytes())


def test_seed_repo_without_base(sibling_repo, tmp_path):
    """quantized files without their BF16 model (method m29): the senior quant (Q8_0) becomes the seed,
    coded by the seed codec (its token_embd row-predicted by the Q8_0 codec); the other quants are
    derived from its dequantized tensors and QR-coded with its quantized tensors as seeds. A second
    model's lone quant is a seed of its own; a GGUF without tensors is stored alone. Every file
    extracts byte-identical."""
    import shutil
    from tests.golden.q8_cases import q8_blocks
    src = str(tmp_path / "src")
    os.makedirs(src)
    for n in os.listdir(sibling_repo):
        if n != "model-BF16.gguf":
            shutil.copy(os.path.join(sibling_repo, n), src)
    g = np.random.Generator(np.random.PCG64(77))
    _gguf_file(os.path.join(src, "mmproj-Q8_0.gguf"), {"general.architecture": "clip"},
               [("v.blk.0.attn_q.weight", (256, 64), 8, q8_blocks(g.normal(0, 0.02, (64, 256)).astype(np.float32)).tobytes()),
                ("v.post_ln.weight", (256,), 0, np.ones(256, np.float32).tobytes())])
    _gguf_file(os.path.join(src, "vocab.gguf"), {"general.architecture": "qwen35", "tokenizer.ggml.model": "gpt2"}, [])
    a = str(tmp_path / "seed.seedpack")
    say("case seed repo: pack")
    stats = repo.pack_repo([src], a)
    r = container.Reader(a)
    man = json.loads(zstd.decompress(r.get("manifest")))
    assert sorted(man["seeds"]) == ["mmproj-Q8_0.gguf", "model-Q8_0.gguf"] and man["bases"] == man["seeds"]
    bi = man["bases"].index("model-Q8_0.gguf")
    assert list(unpack(memoryview(r.get(f"b{bi}"))))[:2] == ["layout", "q8"]
    files = {m["name"]: m for m in man["files"]}
    assert files["vocab.gguf"]["base"] is None and files["vocab.gguf"]["plan"] == []
    assert all(files[n]["base"] == bi for n in files if n.startswith("model-"))
    kinds = {e[1] for n in files for e in files[n]["plan"]}
    assert "qr" in kinds, kinds
    assert stats["stats"]["qr"] > 0
    say("case seed repo: unpack", stats["stats"])
    out = str(tmp_path / "out")
    res = repo.unpack_repo(a, out)
    assert not res["bad"] and not res["missing"], res
    for n in sorted(os.listdir(src)):
        assert open(os.path.join(src, n), "rb").read() == open(os.path.join(out, n), "rb").read(), n


def test_fitted_importance_repo(small_repo, tmp_path):
    """quants made with another importance matrix (another chunk count in their metadata): their
    importance is fitted back from the first such file (imxfit), stored in the "imx" chunk, and both
    files of the set are predicted with it -- most tensors become exact requantizations; every file
    extracts byte-identical"""
    import shutil
    from seedpack_amd import imatrix as imx_mod
    from seedpack_amd.gpuquant import GPUQuant
    root = small_repo[0]
    src = str(tmp_path / "src")
    os.makedirs(src)
    for n in ("model-BF16.gguf", "imatrix.dat", "model-Q4_0.gguf"):
        shutil.copy(os.path.join(root, n), src)
    base = np.fromfile(os.path.join(root, "model-BF16.gguf"), np.uint8)
    g = gguf.GGUF(base)
    imx = imx_mod.load(open(os.path.join(root, "imatrix.dat"), "rb").read())
    rng = np.random.Generator(np.random.PCG64(9))
    alt = {n: (np.asarray(v, np.float32) ** 0.5 * np.exp(rng.normal(0, 0.5, len(v)))).astype(np.float32)
           for n, v in imx.items()}
    gq = GPUQuant()
    for fname, T in (("alt-Q4_0.gguf", 2), ("alt-Q5_1.gguf", 7)):
        tensors = []
        for t in g.tensors:
            raw = base[t.offset:t.offset + t.nbytes]
            if len(t.shape) == 2:
                x = dev.DeviceArray.from_host(raw.view(np.uint16))
                y = gq.quantize_tensors(T, [(x, t.shape[0])], [alt[t.name]], device=True)[0].to_host()
                tensors.append((t.name, t.shape, T, y.tobytes()))
            else:
                tensors.append((t.name, t.shape, t.type, raw.tobytes()))
        _gguf_file(os.path.join(src, fname), {"general.architecture": "qwen35", "general.alignment": 32,
                                              "quantize.imatrix.file": "other.dat",
                                              "quantize.imatrix.dataset": "other.txt",
                                              "quantize.imatrix.chunks_count": 64}, tensors)
    a = str(tmp_path / "fit.seedpack")
    say("case fitted importance: pack")
    stats = repo.pack_repo([src], a, created="2026-01-01T00:00:00")
    r = container.Reader(a)
    man = json.loads(zstd.decompress(r.get("manifest")))
    assert man.get("imx_fit") == {"chunk": "imx", "sets": 1} and "imx" in r.chunks
    assert stats["stats"]["imx_fit"] > 0, stats["stats"]
    files = {m["name"]: m for m in man["files"]}
    for fname in ("alt-Q4_0.gguf", "alt-Q5_1.gguf"):
        fitted = [e for e in files[fname]["plan"] if isinstance(e[2], int) and e[2] >= 1000]
        assert len(fitted) >= len(files[fname]["plan"]) // 2, (fname, files[fname]["plan"])
    assert not any(isinstance(e[2], int) and e[2] >= 1000 for e in files["model-Q4_0.gguf"]["plan"])
    say("case fitted importance: unpack", stats["stats"])
    out = str(tmp_path / "out")
    res = repo.unpack_repo(a, out)
    assert not res["bad"] and not res["missing"], res
    for n in sorted(os.listdir(src)):
        assert open(os.path.join(src, n), "rb").read() == open(os.path.join(out, n), "rb").read(), n
    # the base kept out of HBM: the fit and the predictions read window by window give the same
    # archive; extract with the base decoded window by window gives the same files
    say("case fitted importance: base in host memory")
    p = repo.Packer(bases_in_hbm=False)
    p.BASE_GROUP = 1 << 20
    a2 = str(tmp_path / "fit_host.seedpack")
    p.pack([src], a2, created="2026-01-01T00:00:00")
    assert open(a, "rb").read() == open(a2, "rb").read()
    out2 = str(tmp_path / "out2")
    res = repo.Unpacker(bases_in_hbm=False).run(a, out2)
    assert not res["bad"] and not res["missing"], res
    for n in sorted(os.listdir(src)):
        assert open(os.path.join(src, n), "rb").read() == open(os.path.join(out2, n), "rb").read(), n


def _split_file(src, dst_fmt, cuts):
    """llama.cpp gguf-split's layout of the GGUF at `src`: its tensors in len(cuts) + 1 shards (cut
    before the tensors named in `cuts`), each shard a GGUF of its own with the split keys"""
    data = np.fromfile(src, np.uint8)
    g = gguf.GGUF(data)
    names = [t.name for t in g.tensors]
    at = [0] + [names.index(c) for c in cuts] + [len(names)]
    n = len(at) - 1
    for k in range(n):
        kv = {"general.architecture": "qwen35", "general.alignment": 32, "split.no": (2, k), "split.count": (2, n),
              "split.tensors.count": (5, len(names))}
        _gguf_file(dst_fmt.format(k + 1, n), kv, [(t.name, t.shape, t.type, data[t.offset:t.offset + t.nbytes].tobytes())
                                                  for t in g.tensors[at[k]:at[k + 1]]])


@pytest.mark.parametrize("method", ["m29", "m28"])
def test_split_model_repo(small_repo, tmp_path, method):
    """a BF16 model in three gguf-split shards, a quant split in two at other boundaries and two whole
    quants: the shards are coded as bases and joined into one base that every quant predicts from
    (manifest "joined", base index len(bases)); every file extracts byte-identical, a quant shard and
    a base shard alone too"""
    import shutil
    root = small_repo[0]
    src = str(tmp_path / "src")
    os.makedirs(src)
    for n in ("imatrix.dat", "model-Q4_K_M.gguf", "model-IQ2_XS.gguf"):
        shutil.copy(os.path.join(root, n), src)
    _split_file(os.path.join(root, "model-BF16.gguf"), os.path.join(src, "model-BF16-{:05d}-of-{:05d}.gguf"),
                ["blk.1.attn_norm.weight", "output_norm.weight"])
    _split_file(os.path.join(root, "model-Q4_0.gguf"), os.path.join(src, "model-Q4_0-{:05d}-of-{:05d}.gguf"),
                ["blk.0.ffn_down.weight"])
    a = str(tmp_path / "split.seedpack")
    say(f"case split model ({method}): pack")
    stats = repo.pack_repo([src], a, method=method, created="2026-01-01T00:00:00")
    if method == "m29":                       # the shards in host memory: the same archive
        h = str(tmp_path / "split_host.seedpack")
        p = repo.Packer(bases_in_hbm=False)
        p.BASE_GROUP = 1 << 20
        p.pack([src], h, created="2026-01-01T00:00:00")
        assert open(a, "rb").read() == open(h, "rb").read()
    man = json.loads(zstd.decompress(container.Reader(a).get("manifest")))
    shards = [f"model-BF16-{k:05d}-of-00003.gguf" for k in (1, 2, 3)]
    assert man["bases"] == shards and man["needs"] == "0.3.0"
    sizes = [os.path.getsize(os.path.join(src, n)) for n in shards]
    assert man["joined"] == [{"parts": [[0, 0], [1, sizes[0]], [2, sizes[0] + sizes[1]]], "size": sum(sizes)}]
    assert all(f["base"] == 3 for f in man["files"]), [(f["name"], f["base"]) for f in man["files"]]
    assert all(f["plan"] for f in man["files"])
    say(f"case split model ({method}): unpack", stats["stats"])
    out = str(tmp_path / "out")
    res = repo.unpack_repo(a, out)
    assert not res["bad"] and not res["missing"], res
    for n in sorted(os.listdir(src)):
        assert open(os.path.join(src, n), "rb").read() == open(os.path.join(out, n), "rb").read(), n
    for pick in ("model-Q4_0-00002-of-00002.gguf", shards[1]):
        res = repo.unpack_repo(a, None, [pick])
        assert res["files"] == {pick: True}, res
    if method == "m29":                       # the shards decoded window by window
        res = repo.Unpacker(bases_in_hbm=False).run(a, str(tmp_path / "out_w"))
        assert not res["bad"] and not res["missing"], res
        for n in sorted(os.listdir(src)):
            assert open(os.path.join(src, n), "rb").read() == open(os.path.join(tmp_path, "out_w", n), "rb").read(), n


def test_small_repo_archive_layout(small_repo):
    root, arc, sizes, stats = small_repo
    r = container.Reader(arc)
    man = json.loads(zstd.decompress(r.get("manifest")))
    assert man["method"] == repo.METHOD and man["bases"] == ["model-BF16.gguf"] and man["seeds"] == []
    assert man["extras"]["bundle"] == ["README.md", "imatrix.dat"] and man["extras"]["single"] == {}
    assert man.get("needs") == "0.3.0"                        # QR-coded grid types
    chunks = list(r.chunks)
    assert chunks[:2] == ["extras", "b0"] and chunks[-1] == "manifest"
    files = [m["name"] for m in man["files"]]
    fchunks = [c for c in chunks if c[0] in "fq"]
    assert fchunks == [c for i in range(len(files)) for c in (f"f{i}", f"q{i}")]
    # the base chunk: pack({"r2": meta, side, tables, stream, lens, rest}), its rest in the P form
    b0 = unpack(memoryview(r.get("b0")))
    inner = unpack(b0["r2"])
    assert list(inner) == ["meta", "side", "tables", "stream", "lens", "rest"]
    assert bytes(inner["rest"][:1]) == b"P"
    # plan entries: [name, kind, variant, type]; 2-D tensors QR-coded, norms predicted by conversion
    for m in man["files"]:
        kinds = {e[1] for e in m["plan"]}
        assert kinds <= {"qr", "rq", "xor"} and "qr" in kinds and "xor" in kinds, (m["name"], kinds)
        assert all(len(e) == 4 for e in m["plan"])
    cat = {f["name"]: f for f in r.meta["files"]}
    assert cat["model-BF16.gguf"]["role"] == "base" and cat["imatrix.dat"]["role"] == "file"
    assert cat["model-Q8_0.gguf"]["role"] == "derived" and r.meta["hash"] == "blake3"
    assert r.meta["total"] == sum(os.path.getsize(os.path.join(root, n)) for n in os.listdir(root))


def _oracle_batch(T, tens, mv, gk):
    """the oracle's coded batch of several tensors [(F, P, seed, seed_type, cols, imx)]: per-tensor
    symbol histograms summed, one normalisation, each tensor's segments coded with those tables"""
    counts, blocks = None, []
    for F, P, seed, st, cols, imx in tens:
        c, b = oqr.histogram(T, F, P, seed, st, cols, mv, imx, gk)
        counts = c if counts is None else counts + c
        blocks.append(b)
    freq, used = oqr.normalize(counts)
    remap = np.full(oqr.NTAB2, -1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    cum = oqr.cum_of(freq)
    parts = [oqr.rans_encode(oqr.segment_sequence(T, b, b0, n), remap, freq, cum) for b in blocks
             for b0, n in oqr.segments(T, len(b))]
    return freq, used, np.array([len(p) for p in parts], np.uint32), b"".join(parts)


def test_small_repo_one_batch_per_type_equals_oracle(small_repo):
    root, arc, sizes, stats = small_repo
    r = container.Reader(arc)
    man = json.loads(zstd.decompress(r.get("manifest")))
    base = open(os.path.join(root, "model-BF16.gguf"), "rb").read()
    bt = {t.name: t for t in gguf.GGUF(base).tensors}
    from seedpack_amd import imatrix
    imx = imatrix.load(open(os.path.join(root, "imatrix.dat"), "rb").read())
    seen = set()
    for i, m in enumerate(man["files"]):
        data = open(os.path.join(root, m["name"]), "rb").read()
        ft = {t.name: t for t in gguf.GGUF(data).tensors}
        q = unpack(memoryview(r.get(f"q{i}")))
        var = {e[0]: e[2] for e in m["plan"]}
        for k, (T, names) in enumerate(json.loads(zstd.decompress(q["meta"]))):
            if T in seen:
                continue
            seen.add(T)
            say(f"case repo oracle batch: {m['name']} type {T}, {len(names)} tensors")
            assert all(var[n] == 0 for n in names)
            from seedpack_amd.gpuquant import GPUQuant
            gq = GPUQuant()
            tens = []
            for n in names:
                b = bt[n]
                w = np.frombuffer(base, np.uint16, b.numel, b.offset)
                P = gq.quantize_tensors(T, [(w, b.shape[0])], [imx[n]])[0]
                F = np.frombuffer(data, np.uint8, ft[n].nbytes, ft[n].offset)
                seed = np.frombuffer(base, np.uint8, b.nbytes, b.offset)
                tens.append((F.tobytes(), P.tobytes(), seed.tobytes(), 30, b.shape[0],
                             imx[n] if T in qr.GRID_TYPES else None))
            freq, used, lens, stream = _oracle_batch(T, tens, qr.MODEL, qr.grid_keys(T) if T in qr.GRID_TYPES else None)
            ch = unpack(q[str(k)])
            f2, u2 = qr.load_tables(ch["t"])
            assert np.array_equal(u2, used) and np.array_equal(f2, freq), "tables"
            assert np.array_equal(np.frombuffer(zstd.decompress(ch["l"]), np.uint32), lens), "segment lengths"
            assert bytes(ch["s"]) == stream, "stream"
    assert seen == set(TYPES)


def _scratch_dir(tmp_path_factory, name):
    """a directory on tmpfs when the box has room there (the files are tens of GB), else under /tmp"""
    import shutil
    if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > (80 << 30):
        d = os.path.join("/dev/shm", f"spa_test_{os.getpid()}_{name}")
        os.makedirs(d, exist_ok=True)
        return d
    return str(tmp_path_factory.mktemp(name))


def test_cfg4_reduced_full_shapes(tmp_path_factory):
    """configuration 4 at full tensor shapes: token_embd and output 151936x4096 and two Qwen3.5-9B
    blocks (4096 / 12288 / 1024 shapes, F32 norms), a 151,936-token tokenizer, all 21 quant files with
    1% of their blocks changed; packed and extracted byte-identical (configuration 5 is a selection of
    that extract). Every QR batch holds tensors of one window and one type, at most BATCH bytes."""
    import shutil
    root = _scratch_dir(tmp_path_factory, "cfg4")
    try:
        src, out = os.path.join(root, "repo"), os.path.join(root, "out")
        say("case repo cfg4 reduced: writing the synthetic repository")
        tensors = synth.qwen_tensors(layers=2)
        sizes = synth.write_repo(src, tensors, _files(), per_million=10000, nmerge=151936 - 256 - 8)
        arc = os.path.join(root, "cfg4.seedpack")
        say(f"case repo cfg4 reduced: pack {sum(sizes.values()) / 1e9:.1f} GB")
        st = repo.pack_repo([src], arc)
        say(f"case repo cfg4 reduced: packed in {st['seconds']:.1f} s ({st['GB_s']:.2f} GB/s), {st['phases']}")
        res = repo.unpack_repo(arc, out)
        say(f"case repo cfg4 reduced: extracted in {res['seconds']:.1f} s ({res['GB_s']:.2f} GB/s)")
        assert not res["bad"] and not res["missing"], res
        for n in sorted(os.listdir(src)):
            with open(os.path.join(src, n), "rb") as fa, open(os.path.join(out, n), "rb") as fb:
                while True:
                    x, y = fa.read(1 << 28), fb.read(1 << 28)
                    assert x == y, n
                    if not x:
                        break
        # QR batches: one window, one type, within the batch size
        r = container.Reader(arc)
        man = json.loads(zstd.decompress(r.get("manifest")))
        base = {t.name: t for t in gguf.tensors_of(os.path.join(src, "model-BF16.gguf"))}
        order = [n for n, s, t in tensors]
        wins = repo.windows([base[n].nbytes for n in order], repo.WINDOW, None)
        win_of = {n: w for w, (a, z) in enumerate(wins) for n in order[a:z]}
        assert len(wins) >= 3                     # the embedding alone, the blocks, the output
        for i, m in enumerate(man["files"]):
            ft = {t.name: t for t in gguf.tensors_of(os.path.join(src, m["name"]))}
            q = unpack(memoryview(r.get(f"q{i}")))
            for T, names in json.loads(zstd.decompress(q["meta"])):
                assert len({win_of[n] for n in names}) == 1, (m["name"], names)
                assert all(ft[n].type == T for n in names)
                assert len(names) == 1 or sum(ft[n].nbytes for n in names) <= qr.BATCH
    finally:
        if root.startswith("/dev/shm"):
            shutil.rmtree(root, ignore_errors=True)
