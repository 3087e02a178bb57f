"""The base codec's "rest" part: a BF16 GGUF's bytes outside its coded tensors (header, metadata,
1-D tensors, padding), coded on the host with lzma, in one of the two forms the reference writes
(seedpack/gpu_bf16.py:421-428, seedpack/gpu2.py:299-457, gpu2.py:636-649):

  "P" form, for a GGUF with a BPE tokenizer: token k >= 256 made by merge rule k - 256 is the two
      tokens that rule joins, so the merged tokens and the merge strings are dropped and rebuilt from
      the (left id, right id) pairs; stored are the stripped header, the lengths and bytes of the
      tokens no merge makes (the 256 byte tokens, the trailing special tokens) and the pair ids as
      three byte planes. Layout: u64 t0, t1, m0, m1 (the token and merge item spans), u64 token
      count, u64 merge count, u32 x 4 compressed part sizes, then the four lzma parts;
  "T" form (the Q8_0 codec only, when the P form does not apply): merge rule k is token 256 + k split
      at one position, so the tokens are stored with each rule's split position;
  "X" form otherwise: the bytes in four equal parts, each lzma'd, sizes first.

Every lzma stream is preset 9 | extreme (xz container, CRC64). The byte layouts are the format; the
code is this repository's own.
"""
import lzma
import struct
from concurrent.futures import ThreadPoolExecutor

import numpy as np

PARTS = 4
_POOL = ThreadPoolExecutor(PARTS)


def _xz(b):
    return lzma.compress(bytes(b), preset=9 | lzma.PRESET_EXTREME)


def _unxz(b):
    return lzma.decompress(bytes(b))


def rest_of(data, layout):
    """the file's bytes outside the coded tensors (layout["t"]: [offset, bytes, ...] in order)"""
    mv = memoryview(data).cast("B") if not isinstance(data, np.ndarray) else memoryview(data.reshape(-1))
    keep, pos = [], 0
    for off, nb, *_ in layout["t"]:
        keep.append(mv[pos:off])
        pos = off + nb
    keep.append(mv[pos:])
    return b"".join(keep)


def fill_rest(out, rest, layout):
    """rest_of's bytes written back around the coded tensors of `out` (the whole file's buffer)"""
    src = np.frombuffer(rest, np.uint8)
    pos = taken = 0
    for off, nb, *_ in layout["t"]:
        out[pos:off] = src[taken:taken + off - pos]
        taken += off - pos
        pos = off + nb
    out[pos:] = src[taken:]


# ------------------------------------------------------------------ "X": four lzma parts

def parts_c(buf):
    n = len(buf)
    cut = [k * n // PARTS for k in range(PARTS + 1)]
    comp = list(_POOL.map(_xz, [buf[cut[k]:cut[k + 1]] for k in range(PARTS)]))
    return struct.pack(f"<{PARTS}I", *(len(c) for c in comp)) + b"".join(comp)


def parts_d(buf):
    sizes = struct.unpack_from(f"<{PARTS}I", buf)
    at = np.cumsum((4 * PARTS,) + sizes).tolist()
    return b"".join(_POOL.map(_unxz, [buf[at[k]:at[k + 1]] for k in range(PARTS)]))


# ------------------------------------------------------------------ "P": BPE tokenizer by merge pairs

def _string_array(data, value_at):
    """(items as bytes, first item's offset, end offset) of a GGUF string array whose value (after
    the type tag) starts at value_at: u32 item type, u64 count, then u64-length-prefixed items"""
    (n,) = struct.unpack_from("<Q", data, value_at + 4)
    first = pos = value_at + 12
    items = []
    for _ in range(n):
        (ln,) = struct.unpack_from("<Q", data, pos)
        items.append(bytes(data[pos + 8:pos + 8 + ln]))
        pos += 8 + ln
    return items, first, pos


def pairs_c(data, g, layout):
    """the P form's body, or None when the tokenizer does not have the merge structure"""
    if "tokenizer.ggml.tokens" not in g.spans or "tokenizer.ggml.merges" not in g.spans:
        return None
    toks, t0, t1 = _string_array(data, g.spans["tokenizer.ggml.tokens"][0])
    merges, m0, m1 = _string_array(data, g.spans["tokenizer.ggml.merges"][0])
    nm = len(merges)
    if not (t1 <= m0 and m1 <= g.data_start and len(toks) >= 256 + nm):
        return None
    first = {}
    for i, tk in enumerate(toks):
        if tk not in first:
            first[tk] = i
    ids = np.empty((2, nm), np.uint32)
    for k, m in enumerate(merges):
        halves = m.split(b" ")
        if len(halves) != 2:
            return None
        a, b = first.get(halves[0]), first.get(halves[1])
        if a is None or b is None or toks[a] + toks[b] != toks[256 + k]:
            return None
        ids[0, k], ids[1, k] = a, b
    kept = toks[:256] + toks[256 + nm:]
    lens = np.fromiter((len(t) for t in kept), np.int64, len(kept))
    if lens.max() > 0xFFFF:
        return None
    rest = rest_of(data, layout)
    stripped = rest[:t0] + rest[t1:m0] + rest[m1:]
    planes = np.stack([(ids >> (8 * byte)).astype(np.uint8) for byte in range(3)])     # [byte][side][rule]
    comp = list(_POOL.map(_xz, [stripped, lens.astype("<u2").tobytes(), b"".join(kept), planes.tobytes()]))
    return (struct.pack("<6Q", t0, t1, m0, m1, len(toks), nm) + struct.pack("<4I", *(len(c) for c in comp))
            + b"".join(comp))


def pairs_d(buf):
    """the P form's body back to rest_of's bytes"""
    t0, t1, m0, m1, ntok, nm = struct.unpack_from("<6Q", buf)
    sizes = struct.unpack_from("<4I", buf, 48)
    at = np.cumsum((64,) + sizes).tolist()
    stripped, lens, raw, planes = _POOL.map(_unxz, [buf[at[k]:at[k + 1]] for k in range(4)])
    lens = np.frombuffer(lens, "<u2").astype(np.int64)
    ends = np.cumsum(lens)
    kept = [raw[e - n:e] for e, n in zip(ends.tolist(), lens.tolist())]
    pl = np.frombuffer(planes, np.uint8).reshape(3, 2, nm).astype(np.uint32)
    ids = pl[0] | (pl[1] << 8) | (pl[2] << 16)
    toks = kept[:256]
    merge_items = []
    for a, b in zip(ids[0].tolist(), ids[1].tolist()):
        left, right = toks[a], toks[b]
        toks.append(left + right)
        merge_items.append(struct.pack("<Q", len(left) + len(right) + 1) + left + b" " + right)
    toks += kept[256:]
    assert len(toks) == ntok, "P form: token count"
    tok_items = b"".join(struct.pack("<Q", len(t)) + t for t in toks)
    gap = t0 + (m0 - t1)                     # the merges' place in the stripped bytes
    return stripped[:t0] + tok_items + stripped[t0:gap] + b"".join(merge_items) + stripped[gap:]


# ------------------------------------------------------------------ "T": BPE tokenizer by split positions

def tok_c(data, g, layout):
    """the T form's body (the Q8_0 codec's fallback when the P form does not apply), or None: merge
    rule k is token 256 + k with a space inserted, so only the split position of each rule is kept.
    Layout: u64 t0, t1, m0, m1, u64 token count, u32 x 4 compressed part sizes, then the lzma parts of
    the stripped header, the u16 token lengths, the token bytes and the u16 split positions."""
    if "tokenizer.ggml.tokens" not in g.spans or "tokenizer.ggml.merges" not in g.spans:
        return None
    toks, t0, t1 = _string_array(data, g.spans["tokenizer.ggml.tokens"][0])
    merges, m0, m1 = _string_array(data, g.spans["tokenizer.ggml.merges"][0])
    if not (t1 <= m0 and m1 <= g.data_start and len(toks) >= 256 + len(merges)):
        return None
    split = np.empty(len(merges), np.uint16)
    for k, m in enumerate(merges):
        tok = toks[256 + k]
        at = m.find(b" ")
        if at < 0 or len(m) != len(tok) + 1 or m[:at] != tok[:at] or m[at + 1:] != tok[at:]:
            return None
        split[k] = at
    lens = np.fromiter((len(t) for t in toks), np.int64, len(toks))
    if lens.max() > 0xFFFF:
        return None
    rest = rest_of(data, layout)
    stripped = rest[:t0] + rest[t1:m0] + rest[m1:]
    comp = list(_POOL.map(_xz, [stripped, lens.astype("<u2").tobytes(), b"".join(toks), split.astype("<u2").tobytes()]))
    return (struct.pack("<5Q", t0, t1, m0, m1, len(toks)) + struct.pack("<4I", *(len(c) for c in comp))
            + b"".join(comp))


def tok_d(buf):
    """the T form's body back to rest_of's bytes"""
    t0, t1, m0, m1, ntok = struct.unpack_from("<5Q", buf)
    sizes = struct.unpack_from("<4I", buf, 40)
    at = np.cumsum((56,) + sizes).tolist()
    stripped, lens, raw, split = _POOL.map(_unxz, [buf[at[k]:at[k + 1]] for k in range(4)])
    lens = np.frombuffer(lens, "<u2").astype(np.int64)
    ends = np.cumsum(lens)
    toks = [raw[e - n:e] for e, n in zip(ends.tolist(), lens.tolist())]
    assert len(toks) == ntok, "T form: token count"
    tok_items = b"".join(struct.pack("<Q", len(t)) + t for t in toks)
    merge_items = b"".join(struct.pack("<Q", len(toks[256 + k]) + 1) + toks[256 + k][:p] + b" " + toks[256 + k][p:]
                           for k, p in enumerate(np.frombuffer(split, "<u2").tolist()))
    gap = t0 + (m0 - t1)
    return stripped[:t0] + tok_items + stripped[t0:gap] + merge_items + stripped[gap:]


# ------------------------------------------------------------------ the part

def header_c(data, g, layout, tokz=False):
    """the "rest" part of a base: the P form when the GGUF's tokenizer allows it, else the X form
    (gpu_bf16.py:421-424); tokz (the Q8_0 codec's header coder, gpu2.py:636-645): the T form before
    the X form. g: the file's parsed header (spans, data_start)"""
    p = pairs_c(data, g, layout)
    if p is not None:
        return b"P" + p
    t = tok_c(data, g, layout) if tokz else None
    return b"T" + t if t is not None else b"X" + parts_c(rest_of(data, layout))


def header_x(rest):
    """the X form of rest_of's bytes"""
    return b"X" + parts_c(rest)


def header_d(buf):
    """either form back to rest_of's bytes (gpu_bf16.py:426-428)"""
    buf = bytes(buf)
    form = buf[:1]
    return pairs_d(buf[1:]) if form == b"P" else tok_d(buf[1:]) if form == b"T" else parts_d(buf[1:])
