"""Seeds: when quantized GGUFs come without their BF16 model, the most precise of them (the "senior"
quant, most bits per weight) takes the BF16 model's place (the reference's seedpack/seed.py). Its
tensors are dequantized for the other files' requantization and its quantized tensors seed their QR
coding; the seed file itself is coded by SeedCodec.

Every tensor of the seed takes one route:
  q8     Q8_0 tensors: the Q8_0 codec M22 (q8.Q8Parts);
  float  2-D F16 / BF16 tensors: the BF16 codec R2 over a minimal GGUF of them as BF16; an F16
         weight whose value BF16 cannot hold is listed with its F16 bits (an exception);
  qr     tensors of 64 KiB and more of a type QR codes without a seed: QR per type, kept where it
         is smaller than zstd-9 of the same bytes, else back to plain;
  plain  the other tensors of 64 KiB and more: zstd-9 of their bytes in file order;
and every other byte (metadata, tokenizer, small tensors) goes to the header coder (P, T or X form).

Chunk format (fixed by the reference, seed.py:57-160): pack() of the parts, in this order and only
those that are not empty:
  layout  zstd of the JSON {"size", "t": [[offset, bytes, row length, group], ...] by offset} of
          the routed tensors;
  q8      the Q8_0 codec's chunk;
  f, fmeta, fexc   R2's whole-file chunk; zstd JSON [[name, type, offset, bytes, exceptions], ...];
          zstd of the exceptions' element indices (u32) then their F16 bits (u16), tensor by tensor;
  s<k>, smeta      QR chunk k; zstd JSON [[type, [[offset, bytes], ...]], ...];
  o, ometa         zstd-9 of the plain tensors' bytes; zstd JSON [[offset, bytes], ...];
  rest    the header coder's output.
"""
import dataclasses
import json
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import device as dev
from . import gguf, header, qr, r2, zstd
from .framing import pack, unpack
from .q8 import Q8Parts, group_of

OTHER_MIN = 1 << 16                  # tensors below this size travel with the header bytes (seed.py:27)
F16, BF16, Q8_0 = 1, 30, 8


def bits_per_weight(tensors):
    """bits per weight over a GGUF's quantized and float tensors: the seed is the file with the most
    (seed.py:30-34)"""
    counted = [t for t in tensors if t.type in gguf.BLOCK]
    weights = sum(t.numel for t in counted)
    return 8 * sum(t.nbytes for t in counted) / max(weights, 1)


def gguf_bytes(tensors, align=32):
    """a GGUF v3 file with no metadata holding tensors [(name, shape, type, payload bytes)], laid out in
    that order at `align`-byte boundaries (the R2 route's input, seed.py:37-53)"""
    head, places, size = gguf.header_bytes({}, [(n, tuple(s), ty) for n, s, ty, _ in tensors], align)
    out = np.zeros(size, np.uint8)
    out[:len(head)] = np.frombuffer(head, np.uint8)
    for (at, _), (_, _, _, payload) in zip(places, tensors):
        out[at:at + len(payload)] = np.frombuffer(payload, np.uint8)
    return out.tobytes()


def f16_from_bf16(u):
    """BF16 bits -> F16 bits, round to nearest even (exact for values F16 holds)"""
    return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)


def bf16_of_f16(u):
    """F16 bits -> the BF16 bits of its value, truncated (seed.py:77)"""
    return (u.view(np.float16).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


@dataclasses.dataclass
class Routes:
    """a seed file's tensors by route; `big` keeps the file order of the tensors of OTHER_MIN bytes and
    more that are neither Q8_0 nor 2-D float (the qr and plain candidates)"""
    q8: list
    floats: list
    big: list

    @property
    def routed(self):
        return self.q8 + self.floats + self.big

    def qr_groups(self):
        """QR-codable tensors of `big` grouped by type, types in order of first appearance"""
        groups = {}
        for t in self.big:
            if t.type in qr.SELF_TYPES and t.shape[0] % qr.QK[t.type] == 0:
                groups.setdefault(t.type, []).append(t)
        return groups


def routes_of(g):
    q8 = [t for t in g.tensors if t.type == Q8_0]
    floats = [t for t in g.tensors if t.type in (F16, BF16) and len(t.shape) == 2]
    skip = {id(t) for t in q8 + floats}
    return Routes(q8, floats, [t for t in g.tensors if id(t) not in skip and t.nbytes >= OTHER_MIN])


def _json_z(obj):
    return zstd.zstd_c(json.dumps(obj).encode())


def _as_bf16(u, ttype):
    """a float tensor's weights (u16 bits of type ttype) as BF16 bits -> (bits, exception indices,
    their F16 bits): an F16 weight is exact in BF16 when converting back gives its bits again"""
    if ttype != F16:
        return u, np.zeros(0, np.uint32), np.zeros(0, np.uint16)
    b = bf16_of_f16(u)
    miss = np.flatnonzero(f16_from_bf16(b) != u)
    return b, miss.astype(np.uint32), u[miss]


class SeedCodec:
    """a quantized GGUF coded by routes; compress(data) -> chunk bytes, decompress(buf) -> numpy uint8"""

    def __init__(self, stream=None):
        self.stream = stream
        self.q8 = Q8Parts(stream=stream)
        self.r2 = r2.BF16v2(stream=stream)

    # ---------------------------------------------------------------- compress
    def compress(self, data, g=None, d=None):
        """data: the file (bytes-like, host); g: its parsed header; d: the file in HBM (optional)"""
        host = data.reshape(-1) if isinstance(data, np.ndarray) else np.frombuffer(data, np.uint8)
        g = g or gguf.GGUF(host)
        ro = routes_of(g)
        layout = {"size": len(host),
                  "t": sorted([t.offset, t.nbytes, t.shape[0], group_of(t.name)] for t in ro.routed)}
        parts = {"layout": _json_z(layout)}
        with ThreadPoolExecutor(1) as side:
            rest = side.submit(header.header_c, host, g, layout, True)
            if ro.q8:
                parts["q8"] = self.q8.compress(host, with_rest=False, g=g, d=d)
            if ro.floats:
                parts.update(self._float_parts(host, ro.floats))
            coded = self._qr_parts(host, ro.qr_groups(), parts)
            plain = [t for t in ro.big if t.offset not in coded]
            if plain:
                parts["o"] = zstd.zstd_c(b"".join(host[t.offset:t.offset + t.nbytes].tobytes() for t in plain), 9)
                parts["ometa"] = _json_z([[t.offset, t.nbytes] for t in plain])
            parts["rest"] = rest.result()
        return pack(parts)

    def _float_parts(self, host, floats):
        """the float route: R2 over the tensors as BF16, their list and the F16 exceptions"""
        payloads, listing, idx, bits = [], [], [], []
        for t in floats:
            b, miss, f16 = _as_bf16(host[t.offset:t.offset + t.nbytes].view(np.uint16), t.type)
            payloads.append((t.name, t.shape, BF16, b.tobytes()))
            listing.append([t.name, t.type, t.offset, t.nbytes, len(miss)])
            idx.append(miss)
            bits.append(f16)
        syn = gguf_bytes(payloads)
        del payloads
        return {"f": self._r2_chunk(syn), "fmeta": _json_z(listing),
                "fexc": zstd.zstd_c(np.concatenate(idx).tobytes() + np.concatenate(bits).tobytes())}

    def _qr_parts(self, host, groups, parts):
        """the qr route: each type's tensors QR-coded without a seed into parts s<k>, where that is
        smaller than zstd-9 of their bytes -> the offsets of the tensors so coded"""
        listing, coded = [], set()
        for T, ts in groups.items():
            blobs = [host[t.offset:t.offset + t.nbytes] for t in ts]
            c = qr.self_encode(T, [(b, t.shape[0]) for b, t in zip(blobs, ts)], stream=self.stream)
            if len(c) >= len(zstd.zstd_c(b"".join(b.tobytes() for b in blobs), 9)):
                continue
            parts[f"s{len(listing)}"] = c
            listing.append([T, [[t.offset, t.nbytes] for t in ts]])
            coded.update(t.offset for t in ts)
        if listing:
            parts["smeta"] = _json_z(listing)
        return coded

    def _r2_chunk(self, syn):
        """R2's whole-file chunk of the float route's GGUF (BF16v2.compress, bf16v2.py:273-289)"""
        h = np.frombuffer(syn, np.uint8)
        g = gguf.GGUF(h)
        lay = r2.layout_of([(t.name, t.offset, t.nbytes, t.shape[0]) for t in g.tensors
                            if t.type == BF16 and len(t.shape) == 2], len(h))
        d = dev.DeviceArray.from_host(h, self.stream)
        return b"".join(bytes(p) for p in self.r2.compress_parts(d, lay, rest=header.header_c(h, g, lay), order="parts"))

    # ---------------------------------------------------------------- decompress
    def decompress(self, buf):
        """-> the file (numpy uint8)"""
        parts = unpack(buf if isinstance(buf, memoryview) else memoryview(buf))
        layout = json.loads(zstd.decompress(parts["layout"]))
        out = np.zeros(layout["size"], np.uint8)
        with ThreadPoolExecutor(1) as side:
            rest = side.submit(header.header_d, bytes(parts["rest"]))
            if "q8" in parts:
                self.q8.decompress(parts["q8"], out=out)
            if "f" in parts:
                self._floats_into(parts, out)
            if "smeta" in parts:
                self._qr_into(parts, out)
            if "o" in parts:
                raw = np.frombuffer(zstd.decompress(parts["o"]), np.uint8)
                at = 0
                for off, nb in json.loads(zstd.decompress(parts["ometa"])):
                    out[off:off + nb] = raw[at:at + nb]
                    at += nb
            header.fill_rest(out, rest.result(), layout)
        return out

    def _floats_into(self, parts, out):
        syn = np.asarray(self.r2.decompress(bytes(parts["f"]))).reshape(-1).view(np.uint8)
        coded = gguf.GGUF(syn, light=True).tensors
        listing = json.loads(zstd.decompress(parts["fmeta"]))
        if len(listing) != len(coded):
            raise ValueError("seed: the float tensor list does not match the coded file")
        exc = zstd.decompress(parts["fexc"])
        total = sum(e[4] for e in listing)
        idx = np.frombuffer(exc, np.uint32, total)
        bits = np.frombuffer(exc, np.uint16, total, 4 * total)
        k = 0
        for (name, ttype, off, nb, nexc), ct in zip(listing, coded):
            u = syn[ct.offset:ct.offset + ct.nbytes].view(np.uint16)
            if ttype == F16:
                u = f16_from_bf16(u)
                u[idx[k:k + nexc]] = bits[k:k + nexc]
                k += nexc
            out[off:off + nb] = u.view(np.uint8)

    def _qr_into(self, parts, out):
        for k, (T, places) in enumerate(json.loads(zstd.decompress(parts["smeta"]))):
            for (off, nb), arr in zip(places, qr.self_decode(T, parts[f"s{k}"], stream=self.stream)):
                a = arr.to_host(stream=self.stream) if isinstance(arr, dev.DeviceArray) else np.asarray(arr)
                out[off:off + nb] = a.reshape(-1).view(np.uint8)[:nb]
