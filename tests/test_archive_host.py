"""Host parts of the archive path (no GPU): GGUF reader/writer, the .seedpack container, the imatrix
reader, zstd with parameters and dictionaries, and the base codec's header ("rest") coder against the
reference's own output (tests/golden/header_vectors.npz, written by make_r2_golden.py --header)."""
import hashlib
import json
import os
import struct
import zlib

import numpy as np
import pytest

from seedpack_amd import container, gguf, header, imatrix, qr, repo, zstd
from tests.golden.header_cases import NAMES, case_file

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def header_vectors():
    return np.load(os.path.join(ROOT, "tests", "golden", "header_vectors.npz"))


# ------------------------------------------------------------------ header coder vs the reference

@pytest.mark.parametrize("name", NAMES)
def test_header_part_equals_reference(header_vectors, name):
    data, layout = case_file(name)
    assert hashlib.sha256(data).digest() == header_vectors[f"{name}/input_sha256"].tobytes(), "case input drifted"
    part = header.header_c(data, gguf.GGUF(data), layout)
    want = header_vectors[f"{name}/rest"].tobytes()
    assert part[:1] == want[:1], "form (P / X)"
    assert part == want


@pytest.mark.parametrize("name", NAMES)
def test_header_part_decodes_back(header_vectors, name):
    data, layout = case_file(name)
    rest = header.rest_of(data, layout)
    assert header.header_d(header_vectors[f"{name}/rest"].tobytes()) == rest     # the reference's bytes
    out = np.zeros(len(data), np.uint8)
    for off, nb, *_ in layout["t"]:
        out[off:off + nb] = np.frombuffer(data, np.uint8, nb, off)
    header.fill_rest(out, header.header_d(header.header_c(data, gguf.GGUF(data), layout)), layout)
    assert out.tobytes() == data


@pytest.mark.parametrize("name", NAMES)
def test_q8_header_part_equals_reference(header_vectors, name):
    """the Q8_0 codec's header coder (P, then the split-position T form, then X) against the reference's"""
    data, layout = case_file(name)
    part = header.header_c(data, gguf.GGUF(data), layout, tokz=True)
    want = header_vectors[f"{name}/rest_q8"].tobytes()
    assert part[:1] == want[:1], "form (P / T / X)"
    assert part == want
    assert header.header_d(want) == header.rest_of(data, layout)


def test_split_form_needs_its_structure():
    """the T form applies to bpe_split (whose P form does not) and not to a merge with a second space"""
    data, layout = case_file("bpe_split")
    assert header.pairs_c(data, gguf.GGUF(data), layout) is None
    assert header.tok_c(data, gguf.GGUF(data), layout) is not None
    bad, _ = case_file("bpe_bad_merge")
    assert header.tok_c(bad, gguf.GGUF(bad), layout) is None


def test_pairs_form_needs_the_merge_structure():
    """a planted mistake in the fixture's input (a merged token that is not its pair's concatenation)
    must turn the P form down"""
    data, layout = case_file("bpe")
    g = gguf.GGUF(data)
    assert header.pairs_c(data, g, layout) is not None
    bad, _ = case_file("bpe_bad_token")
    assert header.pairs_c(bad, gguf.GGUF(bad), layout) is None


# ------------------------------------------------------------------ GGUF

def test_gguf_round_trip_and_light_mode():
    kv = {"general.architecture": "qwen35", "general.alignment": 64, "a.u32": 7, "a.i64": -5, "a.f32": 0.25,
          "a.bool": True, "a.ints": [1, -2, 3], "a.floats": [0.5, 1.5], "tokenizer.ggml.tokens": [f"t{i}" for i in range(100)],
          "a.typed": (gguf.T_ARRAY, (10, [1, 2 ** 40]))}
    tensors = [("x", (128, 3), gguf.BF16), ("y", (256, 2), 12), ("z", (5,), gguf.F32), ("w", (64, 4), 42)]
    head, where, size = gguf.header_bytes(kv, tensors, align=64)
    data = head + bytes(size - len(head))
    g = gguf.GGUF(data)
    assert g.version == 3 and g.data_start == len(head) and g.data_start % 64 == 0
    assert g.meta["a.i64"] == -5 and g.meta["a.ints"] == [1, -2, 3] and g.meta["a.typed"] == [1, 2 ** 40]
    assert g.meta["tokenizer.ggml.tokens"][99] == "t99"
    assert [(t.name, t.shape, t.type, t.offset, t.nbytes) for t in g.tensors] == \
        [(n, s, ty, o, nb) for (n, s, ty), (o, nb) in zip(tensors, where)]
    assert [t.nbytes for t in g.tensors] == [768, 288, 20, 72]
    assert all(t.offset % 64 == 0 for t in g.tensors)
    light = gguf.GGUF(data, light=True)
    assert light.meta["tokenizer.ggml.tokens"] is None and light.tensors == g.tensors
    assert light.data_start == g.data_start and light.spans == g.spans and light.meta["a.ints"] == [1, -2, 3]
    # arrays of more than 64 items are stepped over (strings by the library's length scan), and one
    # that runs past the data is an error, not a short read
    kv2 = {"tokenizer.ggml.tokens": [f"tok{i}" * (i % 7) for i in range(3000)], "tokenizer.ggml.token_type": [1] * 3000,
           "general.name": "after the arrays"}
    head2, _, size2 = gguf.header_bytes(kv2, tensors)
    data2 = head2 + bytes(size2 - len(head2))
    full, lite = gguf.GGUF(data2), gguf.GGUF(data2, light=True)
    assert lite.meta["tokenizer.ggml.tokens"] is None and lite.meta["tokenizer.ggml.token_type"] is None
    assert lite.meta["general.name"] == "after the arrays" and lite.tensors == full.tensors
    assert lite.data_start == full.data_start
    a0, a1 = full.spans["tokenizer.ggml.tokens"]
    with pytest.raises(ValueError):
        gguf.GGUF(data2[:a0 + (a1 - a0) // 2], light=True)
    a, b = g.spans["a.u32"]
    assert struct.unpack_from("<I", data, a)[0] == 7 and b - a == 4
    with pytest.raises(ValueError):
        gguf.GGUF(b"GGUX" + data[4:])


# ------------------------------------------------------------------ container

def test_crc32_combine_matches_zlib():
    g = np.random.default_rng(5)
    for la, lb in [(0, 1), (3, 0), (1000, 77777), (5, 1 << 20), (1 << 16, 12345678)]:
        a, b = g.bytes(la), g.bytes(lb)
        assert container.crc32_combine(zlib.crc32(a), zlib.crc32(b), lb) == zlib.crc32(a + b)
    big = g.bytes(70 << 20)
    assert container.crc32_parallel(big) == zlib.crc32(big)


def test_container_round_trip_streams_and_damage(tmp_path):
    p = str(tmp_path / "a.seedpack")
    g = np.random.default_rng(6)
    blob = g.integers(0, 256, 3 << 20, dtype=np.uint8)
    w = container.Writer(p)
    w.put("first", b"hello")
    s = w.put_stream("streamed")
    s.head(bytes(16))
    s.write(blob[:1000])
    s.write(blob[1000:])
    s.close(b"0123456789abcdef")
    w.put("pieces", [b"ab", memoryview(b"cd"), np.arange(3, dtype=np.uint8)])
    w.close({"tool": "test", "files": [1, 2]})
    assert not os.path.exists(p + ".part")
    r = container.Reader(p)
    assert r.meta == {"tool": "test", "files": [1, 2]}
    assert list(r.chunks) == ["first", "streamed", "pieces"]
    assert bytes(r.get("first")) == b"hello"
    got = r.get("streamed")
    assert bytes(got[:16]) == b"0123456789abcdef" and np.array_equal(got[16:], blob)
    assert bytes(r.get("pieces")) == b"abcd\0\1\2"
    assert bytes(r.read_at("streamed", 16 + 5, 4)) == blob[5:9].tobytes()
    with open(p, "rb") as f:
        raw = f.read()
    assert raw[:12] == b"SEEDPACK" + struct.pack("<I", 1) and raw[-8:] == b"SEEDEND\0"
    off, n, _ = struct.unpack("<QQ8s", raw[-24:])
    assert zstd.decompress(raw[off:off + n]).startswith(b'{"chunks": {"first": [12, 5, ')
    r.close()
    bad = bytearray(raw)
    bad[12 + 5 + 20] ^= 1                   # a byte inside "streamed"
    open(p, "wb").write(bytes(bad))
    with pytest.raises(container.FormatError):
        container.Reader(p).get("streamed")
    open(p, "wb").write(raw[:-30])
    with pytest.raises(container.FormatError):
        container.Reader(p)


def test_container_streamed_read_pieces_and_damage(tmp_path):
    """get_streamed: every byte of the chunk reaches on_piece exactly once (pieces of any step,
    several threads), the result equals get(), and a damaged chunk raises after its pieces are in"""
    from concurrent.futures import ThreadPoolExecutor
    p = str(tmp_path / "s.seedpack")
    blob = np.random.default_rng(8).integers(0, 256, (5 << 20) + 333, dtype=np.uint8)
    w = container.Writer(p)
    w.put("a", b"x")
    w.put("big", blob)
    w.put("empty", b"")
    w.close({})
    pool = ThreadPoolExecutor(4)
    r = container.Reader(p)
    for step in (1 << 20, (1 << 20) + 7, 64 << 20):
        seen = np.zeros(blob.size, np.int32)
        copy = np.zeros(blob.size, np.uint8)

        def on_piece(o, v):
            seen[o:o + len(v)] += 1
            copy[o:o + len(v)] = v
        got = r.get_streamed("big", on_piece, pool, step)
        assert np.array_equal(got, blob) and np.array_equal(copy, blob) and (seen == 1).all()
    assert r.get_streamed("empty", lambda o, v: None, pool).size == 0
    r.close()
    raw = bytearray(open(p, "rb").read())
    raw[12 + 1 + 4096] ^= 0x40              # a byte inside "big"
    open(p, "wb").write(bytes(raw))
    with pytest.raises(container.FormatError):
        container.Reader(p).get_streamed("big", lambda o, v: None, pool, 1 << 20)


def test_reserved_file_written_through_its_mapping(tmp_path):
    """_preallocate then _write_file(reserved=True): the bytes land whole (pieces across the mapping,
    a ragged last piece); a file of another size, or none reserved, takes the plain write path"""
    from concurrent.futures import ThreadPoolExecutor
    pool = ThreadPoolExecutor(4)
    data = np.random.default_rng(9).integers(0, 256, (3 << 20) + 1234, dtype=np.uint8)
    p = str(tmp_path / "out" / "f.part")
    os.makedirs(os.path.dirname(p))
    assert repo._preallocate(p, data.size) and os.path.getsize(p) == data.size
    repo._write_file(p, memoryview(data), pool, step=1 << 20, reserved=True)
    assert open(p, "rb").read() == data.tobytes()
    assert repo._preallocate(p, data.size + 5)
    repo._write_file(p, memoryview(data), pool, step=1 << 20, reserved=True)   # size differs: plain path
    assert open(p, "rb").read() == data.tobytes()
    q = str(tmp_path / "g")
    repo._write_file(q, memoryview(data[:100]), pool, reserved=False)
    assert open(q, "rb").read() == data[:100].tobytes()


def test_container_abort_leaves_nothing(tmp_path):
    p = str(tmp_path / "b.seedpack")
    w = container.Writer(p)
    w.put("x", b"1")
    s = w.put_stream("y")
    s.head(b"h")
    w.abort()
    assert not os.path.exists(p) and not os.path.exists(p + ".part")


# ------------------------------------------------------------------ imatrix, zstd

def test_imatrix_legacy_and_gguf():
    g = np.random.default_rng(7)
    e = {"blk.0.attn_q.weight": g.lognormal(0, 1, 64).astype(np.float32), "output.weight": np.ones(32, np.float32)}
    buf = imatrix.write_dat(e, ncall=3, chunk_count=125, dataset="calib.txt")
    got = imatrix.load(buf)
    for k in e:
        np.testing.assert_array_equal(got[k], (e[k] * np.float32(3)) / np.float32(3))
    assert imatrix.chunks(buf) == 125 and imatrix.chunks(imatrix.write_dat(e)) is None
    sums = g.random((2, 16)).astype(np.float32)
    counts = np.array([4, 0], np.float32)
    kv = {"general.type": "imatrix", "imatrix.chunk_count": 9}
    head, where, size = gguf.header_bytes(kv, [("t.in_sum2", (16, 2), gguf.F32), ("t.counts", (2,), gguf.F32)])
    data = bytearray(size)
    data[:len(head)] = head
    data[where[0][0]:where[0][0] + 128] = sums.tobytes()
    data[where[1][0]:where[1][0] + 8] = counts.tobytes()
    v = imatrix.load(bytes(data))["t"]
    np.testing.assert_array_equal(v[:16], sums[0] / np.float32(4))
    np.testing.assert_array_equal(v[16:], np.ones(16, np.float32))
    assert imatrix.chunks(bytes(data)) == 9


def test_zstd_params_dictionary_and_pieces():
    g = np.random.default_rng(8)
    d = (g.integers(0, 8, 4 << 20) == 0).astype(np.uint8) * g.integers(0, 256, 4 << 20).astype(np.uint8)
    dic = g.bytes(50000)
    d[:50000] = np.frombuffer(dic, np.uint8)        # the frame's matches refer to the dictionary
    for p in (zstd.Params(7, 25), zstd.Params(9, 25, threads=4), zstd.Params(7, threads=2, ldm=True)):
        c = zstd.Compressor(p, dic, size=d.size)
        frame = c.compress(d[:1234567]) + c.compress(d[1234567:]) + c.finish()
        assert frame == zstd.compress_with(d, p, dic)          # the split into pieces does not matter
        assert np.array_equal(zstd.decompress_into(frame, np.empty(d.size, np.uint8), dic), d)
        with pytest.raises((ValueError, RuntimeError)):
            zstd.decompress_into(frame, np.empty(d.size, np.uint8))      # the dictionary is needed
    with pytest.raises(ValueError):
        zstd.decompress_into(frame[:len(frame) // 2], np.empty(d.size, np.uint8), dic)
    assert zstd.decompress(zstd.compress(b"abc" * 1000, 19)) == b"abc" * 1000


# ------------------------------------------------------------------ archive rules

def test_window_and_batch_rules():
    """the reference's window rule, its prediction-bytes bound, and the QR batch split"""
    gb = 1 << 30
    assert repo.windows([gb + 5, 100, 200, gb]) == [(0, 1), (1, 3), (3, 4)]
    assert repo.windows([10] * 5, window=25) == [(0, 2), (2, 4), (4, 5)]
    assert repo.windows([1] * 4, pred=[2, 2, 2, 2], pred_window=4) == [(0, 2), (2, 4)]
    assert repo.windows([]) == []
    assert repo.order_groups([("a", "b", "c"), ("a", "c"), ("d",), ("a", "b", "c")]) == \
        {("a", "b", "c"): [0, 1, 3], ("d",): [2]}
    assert qr.batches(12, [300 << 20, 100 << 20, 10]) == [[0], [1, 2]]


def test_pinned_pool_reuses_and_bounds(monkeypatch):
    """the packer's page-locked staging: buffers reused smallest-fitting first, never above the budget
    (a free buffer too small for a request is dropped to make room)"""
    monkeypatch.setattr(repo.dev, "pinned", lambda n: np.empty(n, np.uint8))
    p = repo._PinnedPool(100)
    a = p.acquire(40)[:30]
    b = p.acquire(50)
    p.release(a)                          # a view: its whole buffer comes back
    c = p.acquire(35)
    assert c.size == 40 and p.total == 90
    p.release(b)
    p.release(c)
    d = p.acquire(60)
    assert d.size == 60 and p.total == 100 and [x.size for x in p.free] == [40]


def test_process_order_keeps_dependent_files_in_order():
    # files 0 and 2 share a tensor key: 0 before 2; the rest largest first (0 with the priority of 2)
    files = {0: (5, {("a", 1)}, 0, {}), 1: (9, {("b", 1)}, 0, {}), 2: (7, {("a", 1)}, 0, {}), 3: (8, {("c", 2)}, 1, {})}
    assert repo.process_order(files, None) == [1, 3, 0, 2]
    # a small file that a large one must wait for goes first
    files[0] = (2, {("a", 1)}, 0, {})
    files[2] = (10, {("a", 1)}, 0, {})
    assert repo.process_order(files, None) == [0, 2, 1, 3]
    # a group whose potential references could exceed a window's budget keeps archive order (0 and 1
    # go as early as the largest file waiting for them)
    files[0] = (5, {("a", 1)}, 0, {})
    files[2] = (7, {("a", 1)}, 0, {0: repo.REF_KEEP + 1})
    assert repo.process_order(files, None) == [0, 1, 3, 2]


def test_split_models_are_found_only_whole():
    """the shards of a split GGUF are joined when every shard of it is there, in shard order; a lone
    shard, a single-shard "split" and other names are not (repo3.py:271-285)"""
    names = ["m-BF16-00002-of-00003.gguf", "imatrix.dat", "m-BF16-00001-of-00003.gguf", "x-00001-of-00002.gguf",
             "m-BF16-00003-of-00003.gguf", "one-00001-of-00001.gguf", "sub/m-BF16-00001-of-00002.gguf",
             "sub/m-BF16-00002-of-00002.gguf", "m-BF16-0001-of-0003.gguf"]
    assert sorted(repo.joined_groups(names)) == [[2, 0, 4], [6, 7]]
    assert repo.joined_groups(["a-00001-of-00002.gguf", "a-00002-of-00003.gguf"]) == []
    # a split model's by-name table: each shard's tensors shifted by the shard's start
    T = gguf.Tensor
    s0, s1 = repo._Base.__new__(repo._Base), repo._Base.__new__(repo._Base)
    s0.name, s0.header, s0.by_name = "m-00001", b"H0", {"a": T("a", (4,), 30, 64, 8)}
    s1.name, s1.header, s1.by_name = "m-00002", b"H1", {"b": T("b", (4,), 30, 96, 8)}
    j = repo._Base.joined(5, [(0, s0), (200, s1)])
    assert j.index == 5 and j.header == b"H0" and j.by_name["a"].offset == 64 and j.by_name["b"].offset == 296
    assert s1.by_name["b"].offset == 96


def test_framing_index_reads_only_the_framing():
    """index() finds each part of a packed buffer (nested too) from the framing alone, the same
    slices unpack() gives; a length past the end is rejected"""
    from seedpack_amd import framing
    inner = framing.pack({"meta": b"m" * 5, "stream": b"s" * 1000, "rest": b"RRR"})
    buf = b"\0" * 7 + framing.pack({"x": b"", "r2": inner})
    reads = []

    def read(o, n):
        reads.append(n)
        return buf[o:o + n]
    top = framing.index(read, len(buf) - 7, 7)
    assert top["x"] == (7 + 4 + 2 + 1 + 8, 0)
    sub = framing.index(read, top["r2"][1], top["r2"][0])
    for k, v in framing.unpack(inner).items():
        o, n = sub[k]
        assert buf[o:o + n] == bytes(v)
    assert max(reads) <= 8
    bad = bytearray(framing.pack({"a": b"abc"}))
    bad[-11] = 99                              # the length of "a"
    with pytest.raises(ValueError):
        framing.index(lambda o, n: bytes(bad[o:o + n]), len(bad))


def _container(path, meta, manifest):
    w = container.Writer(path)
    w.put("f0", b"\0" * 16)
    w.put("manifest", zstd.compress(json.dumps(manifest).encode(), 19))
    w.close(meta)


@pytest.mark.parametrize("needs,ok", [(None, True), ("0.3.0", True), ("0.5.0", True), ("0.5.1", False),
                                      ("1.0", False), ("x.y", False)])
def test_reader_refuses_newer_archives(tmp_path, needs, ok):
    """a manifest that needs a newer reader is refused before anything is decoded (repo3.py:2285-2289)"""
    from seedpack_amd import repo
    p = str(tmp_path / "a.seedpack")
    man = {"method": repo.METHOD, "files": [], "bases": []}
    if needs is not None:
        man["needs"] = needs
    _container(p, {"hash": "blake3", "files": []}, man)
    if ok:
        r, meta, m2, algo = repo.open_archive(p)
        r.close()
        assert algo == "blake3" and m2 == man
    else:
        with pytest.raises(container.FormatError, match="needs"):
            repo.open_archive(p)


@pytest.mark.parametrize("algo", ["sha256", "blake3", "md5", None])
def test_reader_checks_the_catalog_hash(tmp_path, algo):
    """a catalog whose checksum this reader cannot compute is refused before decoding, unless the
    caller opts out of verification (then a warning, and files go unchecked)"""
    from seedpack_amd import repo
    p = str(tmp_path / "a.seedpack")
    meta = {"files": []} if algo is None else {"hash": algo, "files": []}
    _container(p, meta, {"method": repo.METHOD, "files": [], "bases": []})
    if algo in repo.HASHES:
        r, _, _, got = repo.open_archive(p)
        r.close()
        assert got == algo
        return
    with pytest.raises(container.FormatError, match="catalog hash"):
        repo.open_archive(p)
    with pytest.warns(UserWarning, match="unchecked"):
        r, _, _, got = repo.open_archive(p, verify=False)
    r.close()
    assert got is None


def test_catalog_digests_of_files(tmp_path):
    """file checksums as the catalog writes them: SHA-256 and BLAKE3 of a file read in pieces equal
    the one-shot digests (BLAKE3 pinned to published vectors by test_blake3.py)"""
    import hashlib
    from oracle import blake3 as ob
    from seedpack_amd import repo
    g = np.random.Generator(np.random.PCG64(9))
    data = g.integers(0, 256, 3 * 1024 + 5, dtype=np.uint8).tobytes()
    p = tmp_path / "f.bin"
    p.write_bytes(data)
    assert repo.file_digest(str(p), "sha256", chunk=1000) == hashlib.sha256(data).hexdigest()
    assert repo.file_digest(str(p), "blake3", chunk=1000) == ob.hexdigest(data)
    assert repo._digest_fn("blake3")(data) == ob.hexdigest(data)


def test_seed_choice_rules():
    """files sharing no tensor name with a base; the senior quant left seeds every file that shares at
    least half of its tensor names with it (repo3.py:1359-1372)"""
    from types import SimpleNamespace as T

    def ts(names, ttype, numel=256, nbytes=None):
        return [T(name=n, type=ttype, numel=numel, nbytes=nbytes if nbytes is not None else numel) for n in names]
    a = ["blk.0.w", "blk.1.w", "blk.2.w", "blk.3.w"]
    b = ["enc.0", "enc.1"]
    derived = {
        "A-Q4.gguf": ts(a, 12, nbytes=144),           # 4.5 bits per weight
        "A-Q8.gguf": ts(a, 8, nbytes=272),            # 8.5: the seed of model A
        "A-half.gguf": ts(a[:2] + ["x.0", "x.1"], 12, nbytes=144),  # half of its names are A's: model A
        "B-Q6.gguf": ts(b, 14, nbytes=210),           # model B's only file
        "C.gguf": ts(["tok", "out"], 8, nbytes=272),  # shares a name with the base: not seeded
        "empty.gguf": [],
    }
    bases = [ts(["tok", "norm"], 30, nbytes=512)]
    assert repo.pick_seeds(bases, derived) == ["A-Q8.gguf", "B-Q6.gguf"]
    # equal bits per weight: the larger name wins
    derived2 = {"m-1.gguf": ts(a, 8, nbytes=272), "m-2.gguf": ts(a, 8, nbytes=272)}
    assert repo.pick_seeds([], derived2) == ["m-2.gguf"]
    # a third of the names shared is another model
    derived3 = {"p.gguf": ts(["u", "v", "w"], 8, nbytes=272), "q.gguf": ts(["u", "y", "z"], 12, nbytes=144)}
    assert repo.pick_seeds([], derived3) == ["p.gguf", "q.gguf"]


def test_fit_sets_plan_and_chunk_round_trip():
    """sets by (chunk count, dataset) in order of their first file; every input a set's legacy-quant
    tensors use waits for its fit; the "imx" chunk holds the fitted vectors as XOR of the published
    bits and reads back; no chunk without a kept fit"""
    from types import SimpleNamespace as T
    from seedpack_amd import fitsets
    e_gate = np.linspace(0.5, 2.0, 64).astype(np.float32)
    e_attn = np.linspace(1.0, 3.0, 64).astype(np.float32)
    imx = {"blk.0.ffn_gate": e_gate, "blk.0.ffn_up": e_gate.copy(), "blk.0.attn_q": e_attn, "blk.0.attn_k": e_attn.copy()}
    heads = {
        "a.gguf": ({"quantize.imatrix.chunks_count": 45, "quantize.imatrix.dataset": "x"},
                   [T(name="blk.0.ffn_gate", type=2), T(name="blk.0.attn_q", type=12)]),
        "b.gguf": ({"quantize.imatrix.chunks_count": 1251}, [T(name="blk.0.ffn_gate", type=2)]),
        "c.gguf": ({"quantize.imatrix.chunks_count": 45, "quantize.imatrix.dataset": "x"},
                   [T(name="blk.0.attn_k", type=7)]),
        "d.gguf": ({"quantize.imatrix.chunks_count": 45, "quantize.imatrix.dataset": "y"}, []),
        "e.gguf": ({}, [T(name="blk.0.ffn_up", type=2)]),
    }
    names = list(heads)
    fs = fitsets.FitSets.plan(names, heads, imx, 1251)
    assert fs.set_of == {0: 1, 2: 1, 3: 2}
    assert (fs.sets[1].chunks, fs.sets[1].dataset, fs.sets[2].dataset) == (45, "x", "y")
    assert fs.sets[1].waiting == {"blk.0.ffn_gate", "blk.0.ffn_up", "blk.0.attn_q", "blk.0.attn_k"}
    assert fs.waiting(1) and not fs.waiting(2) and not fs.waiting(0)
    assert fs.chunk() is None
    fit = (e_gate * np.float32(1.25)).astype(np.float32)
    fs.sets[1].kept.append(fitsets.Fit(["blk.0.ffn_gate", "blk.0.ffn_up"], fit, e_gate, 0.5, 0.9))
    body, entry = fs.chunk()
    assert entry == {"chunk": "imx", "sets": 2}
    back = fitsets.read_chunk(body, imx)
    assert set(back) == {1, 2} and back[2] == {}
    assert set(back[1]) == {"blk.0.ffn_gate", "blk.0.ffn_up"} and np.array_equal(back[1]["blk.0.ffn_up"], fit)
    assert fs.importance(1)["blk.0.ffn_gate"] is fit and fs.importance(3) == {}
    # no published chunk count: no sets
    assert fitsets.FitSets.plan(names, heads, imx, None).sets == {}
