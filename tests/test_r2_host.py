"""Host side of the R2 codec that runs without a GPU: the chunk framing, the file's other bytes
(rest_of / fill_rest) and both header forms (the P form also against the reference's own output in
tests/test_archive_host.py)."""
import lzma
import struct

import numpy as np

from seedpack_amd import framing, header


def _gguf_strings(items):
    """a GGUF string-array value as _items reads it: u32 item type, u64 count, (u64 length, bytes)..."""
    return struct.pack("<IQ", 8, len(items)) + b"".join(struct.pack("<Q", len(x)) + x for x in items)


def test_framing_round_trip():
    ch = {"meta": b"m", "stream": [b"ab", memoryview(b"cd"), b""], "rest": b"xyz"}
    buf = framing.pack(ch)
    assert b"".join(bytes(p) for p in framing.pack_parts(ch)) == buf
    back = framing.unpack(memoryview(buf))
    assert {k: bytes(v) for k, v in back.items()} == {"meta": b"m", "stream": b"abcd", "rest": b"xyz"}
    (n,) = struct.unpack_from("<I", buf)
    assert n == 3 and buf[4:6] == struct.pack("<H", 4) and buf[6:10] == b"meta"


def test_rest_of_and_fill_rest():
    g = np.random.default_rng(3)
    data = g.integers(0, 256, 1000, dtype=np.uint8).tobytes()
    layout = {"size": 1000, "t": [[96, 200, 10, "bf16"], [320, 100, 10, "bf16"], [900, 100, 10, "bf16"]]}
    rest = header.rest_of(data, layout)
    assert rest == data[:96] + data[296:320] + data[420:900]
    out = np.zeros(1000, np.uint8)
    header.fill_rest(out, rest, layout)
    want = np.frombuffer(data, np.uint8).copy()
    for off, nb, _, _ in layout["t"]:
        want[off:off + nb] = 0
    assert np.array_equal(out, want)


def test_header_x_round_trip():
    g = np.random.default_rng(4)
    for n in (0, 3, 4097):
        b = g.integers(0, 4, n, dtype=np.uint8).tobytes()
        h = header.header_x(b)
        assert h[:1] == b"X" and header.header_d(h) == b
        lens = struct.unpack_from("<4I", h, 1)
        assert lzma.decompress(h[17:17 + lens[0]]) == b[:n // 4]


def test_header_pairs_form_rebuilds_the_token_arrays():
    """the tokenizer-aware form: a header whose token array is 256 byte tokens, 40 BPE merges (token
    256+k = the concatenation of merge k's pair) and 3 special tokens; the form stores the header
    without the two arrays, the raw tokens and the pairs' byte planes, and decodes to the header's
    exact bytes"""
    g = np.random.default_rng(5)
    toks = [bytes([i]) for i in range(256)]
    pairs = []
    for k in range(40):
        a, b = int(g.integers(0, len(toks))), int(g.integers(0, len(toks)))
        pairs.append((a, b))
        toks.append(toks[a] + toks[b])
    special = [b"<s>", b"</s>", b"<|pad|>"]
    toks += special
    merges = [toks[a] + b" " + toks[b] for a, b in pairs]
    head = b"GGUF" + g.integers(0, 256, 50, dtype=np.uint8).tobytes()
    tok_val = _gguf_strings(toks)
    mid = g.integers(0, 256, 30, dtype=np.uint8).tobytes()
    mer_val = _gguf_strings(merges)
    tail = g.integers(0, 256, 20, dtype=np.uint8).tobytes()
    rest = head + tok_val + mid + mer_val + tail
    t0 = len(head) + 12
    t1 = len(head) + len(tok_val)
    m0 = t1 + len(mid) + 12
    m1 = m0 - 12 + len(mer_val)
    stripped = rest[:t0] + rest[t1:m0] + rest[m1:]
    raw = toks[:256] + special
    lens = np.array([len(x) for x in raw], np.uint16)
    pr = np.array(pairs, np.uint32)
    planes = np.concatenate([(pr >> (8 * i)).astype(np.uint8).T.ravel() for i in range(3)])
    comp = [lzma.compress(x) for x in (stripped, lens.tobytes(), b"".join(raw), planes.tobytes())]
    buf = b"P" + struct.pack("<6Q", t0, t1, m0, m1, len(toks), len(pairs)) + struct.pack("<4I", *map(len, comp)) + b"".join(comp)
    assert header.header_d(buf) == rest
