"""GGUF files: the header reader the archive path needs, and a writer for synthetic repositories.

Reading follows the GGUF v2/v3 layout that seedpack/gguf_reader.py:47-121 parses: magic, version,
tensor count, key/value count, the key/value pairs (GGUF value types 0-12), the tensor table (name,
dimensions in ggml order, type, offset from the data start), the data start aligned to
`general.alignment` (default 32). `spans[key]` is the byte span of a value (its type tag excluded),
which the base codec's header coder uses to find the tokenizer arrays. With light=True, arrays of more
than 64 items (vocabularies, merges, token types) are skipped and read as None.
"""
import struct
from dataclasses import dataclass

import numpy as np

from ._lib import lib

F32, F16, Q8_0, BF16 = 0, 1, 8, 30
TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K",
              12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S",
              20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 29: "IQ1_M", 30: "BF16", 42: "Q2_0"}
# ggml type -> (elements per block, bytes per block)
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
         16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110), 22: (256, 82),
         23: (256, 136), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 29: (256, 56), 42: (64, 18)}

# GGUF value type -> struct code of the scalar types
_SCALARS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
T_STRING, T_ARRAY = 8, 9


@dataclass
class Tensor:
    name: str
    shape: tuple          # ggml order: shape[0] is the row length (contiguous)
    type: int
    offset: int           # absolute byte offset in the file
    nbytes: int

    @property
    def numel(self):
        return int(np.prod(self.shape, dtype=np.int64))


class GGUF:
    """parsed header of a GGUF file held in `data` (bytes, mmap, memoryview or uint8 array)"""

    def __init__(self, data, light=False):
        self.data = data
        mv = memoryview(data).cast("B") if not isinstance(data, np.ndarray) else memoryview(data.reshape(-1))
        if bytes(mv[:4]) != b"GGUF":
            raise ValueError("not a GGUF file")
        self._mv, self._pos, self.light = mv, 4, light
        self.version = self._get("I")
        nt, nkv = self._get("Q"), self._get("Q")
        self.meta, self.spans = {}, {}
        for _ in range(nkv):
            key = self._string()
            vt = self._get("I")
            a = self._pos
            self.meta[key] = self._value(vt)
            self.spans[key] = (a, self._pos)
        table = []
        for _ in range(nt):
            name = self._string()
            nd = self._get("I")
            dims = tuple(self._get("Q") for _ in range(nd))
            table.append((name, dims, self._get("I"), self._get("Q")))
        align = int(self.meta.get("general.alignment", 32))
        self.header_end = self._pos
        self.data_start = -(-self._pos // align) * align
        self.tensors = []
        for name, dims, t, off in table:
            be, bb = BLOCK[t]
            n = int(np.prod(dims, dtype=np.int64))
            self.tensors.append(Tensor(name, dims, t, self.data_start + off, n // be * bb))
        del self._mv

    @classmethod
    def from_bytes(cls, data, light=False):
        return cls(data, light)

    def _get(self, code):
        v = struct.unpack_from("<" + code, self._mv, self._pos)[0]
        self._pos += struct.calcsize(code)
        return v

    def _string(self):
        n = self._get("Q")
        s = bytes(self._mv[self._pos:self._pos + n]).decode("utf-8", "replace")
        self._pos += n
        return s

    def _value(self, vt):
        if vt == T_STRING:
            return self._string()
        if vt != T_ARRAY:
            return self._get(_SCALARS[vt])
        it, n = self._get("I"), self._get("Q")
        if it in _SCALARS:
            dt = np.dtype("<" + _SCALARS[it])
            if self.light and n > 64:
                if self._pos + n * dt.itemsize > len(self._mv):
                    raise ValueError("GGUF array runs past the end of the data")
                self._pos += n * dt.itemsize
                return None
            v = np.frombuffer(self._mv, dt, n, self._pos).tolist()
            self._pos += n * dt.itemsize
            return v
        if it == T_STRING:
            if self.light and n > 64:
                at = np.frombuffer(self._mv, np.uint8)
                k = lib().spa_gguf_strings_bytes(at.ctypes.data + self._pos, at.size - self._pos, n)
                if k == 2 ** 64 - 1:
                    raise ValueError("GGUF string array runs past the end of the data")
                self._pos += k
                return None
            return [self._string() for _ in range(n)]
        return [self._value(it) for _ in range(n)]


def tensors_of(path):
    """the tensor table of the GGUF file at `path` ([] if it is not one), from its header only"""
    import mmap
    try:
        with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            return GGUF(mm, light=True).tensors
    except (ValueError, OSError, struct.error, KeyError):
        return []


def header_of(path):
    """(metadata, tensor table) of the GGUF file at `path` (({}, []) if it is not one), from its
    header only, in one pass"""
    import mmap
    try:
        with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            g = GGUF(mm, light=True)
            return g.meta, g.tensors
    except (ValueError, OSError, struct.error, KeyError):
        return {}, []


def meta_of(path):
    """the key/value metadata of a GGUF file ({} if it is not one), from its header only"""
    import mmap
    try:
        with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            return GGUF(mm, light=True).meta
    except (ValueError, OSError, struct.error, KeyError):
        return {}


# ------------------------------------------------------------------ writing (synthetic repositories)

def _enc_string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _enc_value(v):
    """(GGUF value type, encoded value) of a Python value: str, bool, int (u32 / i64), float (f32),
    list of str / int / float, or a (type, value) pair naming the type"""
    if isinstance(v, tuple):
        vt, x = v
        if vt == T_ARRAY:
            it, items = x
            body = b"".join(_enc_value((it, e))[1] for e in items) if it in (T_STRING, T_ARRAY) else \
                np.asarray(items, "<" + _SCALARS[it]).tobytes()
            return T_ARRAY, struct.pack("<IQ", it, len(items)) + body
        if vt == T_STRING:
            return T_STRING, _enc_string(x)
        return vt, struct.pack("<" + _SCALARS[vt], x)
    if isinstance(v, (str, bytes)):
        return T_STRING, _enc_string(v)
    if isinstance(v, bool):
        return 7, struct.pack("<?", v)
    if isinstance(v, int):
        return (4, struct.pack("<I", v)) if 0 <= v < (1 << 32) else (11, struct.pack("<q", v))
    if isinstance(v, float):
        return 6, struct.pack("<f", v)
    if isinstance(v, list):
        if all(isinstance(e, (str, bytes)) for e in v):
            return T_ARRAY, struct.pack("<IQ", T_STRING, len(v)) + b"".join(_enc_string(e) for e in v)
        if all(isinstance(e, int) and not isinstance(e, bool) for e in v):
            return T_ARRAY, struct.pack("<IQ", 5, len(v)) + np.asarray(v, "<i4").tobytes()
        return T_ARRAY, struct.pack("<IQ", 6, len(v)) + np.asarray(v, "<f4").tobytes()
    raise TypeError(f"GGUF value of type {type(v)}")


def header_bytes(kv, tensors, align=32):
    """the header of a GGUF v3 file: kv {key: value}, tensors [(name, shape (ggml order), type)] laid
    out back to back in that order, each at an `align`-byte boundary of the data section (the last
    one padded too). Returns (header bytes padded to the data start, [(offset in the file, nbytes)]
    per tensor, file size)"""
    parts = [b"GGUF", struct.pack("<IQQ", 3, len(tensors), len(kv))]
    for k, v in kv.items():
        vt, body = _enc_value(v)
        parts += [_enc_string(k), struct.pack("<I", vt), body]
    rel, o = [], 0
    for name, shape, t in tensors:
        be, bb = BLOCK[t]
        nb = int(np.prod(shape, dtype=np.int64)) // be * bb
        rel.append((o, nb))
        parts += [_enc_string(name), struct.pack("<I", len(shape)), struct.pack(f"<{len(shape)}Q", *shape),
                  struct.pack("<IQ", t, o)]
        o = -(-(o + nb) // align) * align
    head = b"".join(parts)
    start = -(-len(head) // align) * align
    head += b"\0" * (start - len(head))
    return head, [(start + r, nb) for r, nb in rel], start + o
