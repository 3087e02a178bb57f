"""Seeds (the reference's seedpack/seed.py): when quantized GGUFs come without their BF16 model, the most
precise of them (the "senior" quant, most bits per weight) takes the BF16 model's place. Its tensors
are dequantized for the other files' requantization and its quantized tensors seed their QR coding;
the seed file itself is coded by parts (SeedCodec):
  * Q8_0 tensors with the Q8_0 codec M22 (q8.Q8Parts);
  * 2-D F16 / BF16 tensors with the BF16 codec R2, as BF16 (F16 weights converted from BF16 hold BF16
    values and convert back exactly; the positions where that fails are stored with their F16 bits);
  * other tensors of at least 64 KiB: QR without a seed per type where that beats zstd-9, else zstd-9;
  * every other byte (metadata, tokenizer, small tensors) with the header coder (P, T or X form).
The chunk is pack({layout, [q8], [f, fmeta, fexc], [s<k>..., smeta], [o, ometa], rest}) with the
reference's names, orders and levels (seed.py:57-121).
"""
import json
import struct
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import device as dev
from . import gguf, header, qr, r2, zstd
from .framing import pack, unpack
from .q8 import Q8Parts, group_of

OTHER_MIN = 1 << 16                  # smaller tensors stay with the header bytes (seed.py:27)
F16, BF16, Q8_0 = 1, 30, 8


def bits_per_weight(tensors):
    """mean bits per weight of a GGUF's tensors (the seed is the file with the most, seed.py:30-34)"""
    n = sum(t.numel for t in tensors if t.type in gguf.BLOCK)
    return 8 * sum(t.nbytes for t in tensors if t.type in gguf.BLOCK) / max(n, 1)


def gguf_bytes(tensors, align=32):
    """a minimal GGUF v3 (no metadata) holding tensors [(name, shape, type, payload bytes)], each at an
    aligned offset (seed.py:37-53)"""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 0))
    offs, off = [], 0
    for name, shape, ty, payload in tensors:
        nb = name.encode()
        head += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(shape))
        head += struct.pack(f"<{len(shape)}Q", *shape) + struct.pack("<IQ", ty, off)
        offs.append(off)
        off += (len(payload) + align - 1) // align * align
    start = (len(head) + align - 1) // align * align
    out = bytearray(start + off)
    out[:len(head)] = head
    for (_, _, _, payload), o in zip(tensors, offs):
        out[start + o:start + o + len(payload)] = payload
    return bytes(out)


def f16_from_bf16(u):
    """BF16 bits -> F16 bits, round to nearest even (exact for values F16 holds)"""
    return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)


def bf16_of_f16(u):
    """F16 bits -> the BF16 bits of its value, truncated (seed.py:77)"""
    return (u.view(np.float16).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


class SeedCodec:
    """a quantized GGUF coded by parts; compress(data) -> chunk bytes, decompress(buf) -> numpy uint8"""

    def __init__(self, stream=None):
        self.stream = stream
        self.q8 = Q8Parts(stream=stream)
        self.r2 = r2.BF16v2(stream=stream)

    def compress(self, data, g=None, d=None):
        """data: the file (bytes-like, host); g: its parsed header; d: the file in HBM (optional)"""
        host = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1)
        g = g or gguf.GGUF(host)
        q8t = [t for t in g.tensors if t.type == Q8_0]
        fl = [t for t in g.tensors if t.type in (F16, BF16) and len(t.shape) == 2]
        taken = {id(t) for t in q8t + fl}
        other = [t for t in g.tensors if id(t) not in taken and t.nbytes >= OTHER_MIN]
        lay = {"size": len(host), "t": sorted([t.offset, t.nbytes, t.shape[0], group_of(t.name)] for t in q8t + fl + other)}
        with ThreadPoolExecutor(1) as ex:
            rest = ex.submit(header.header_c, host, g, lay, True)
            ch = {"layout": zstd.zstd_c(json.dumps(lay).encode())}
            if q8t:
                ch["q8"] = self.q8.compress(host, with_rest=False, g=g, d=d)
            if fl:
                parts, meta, idx, vals = [], [], [], []
                for t in fl:
                    u = host[t.offset:t.offset + t.nbytes].view(np.uint16)
                    nbad = 0
                    if t.type == F16:
                        b = bf16_of_f16(u)
                        bad = np.flatnonzero(f16_from_bf16(b) != u)
                        idx.append(bad.astype(np.uint32))
                        vals.append(u[bad])
                        nbad = len(bad)
                        u = b
                    parts.append((t.name, t.shape, BF16, u.tobytes()))
                    meta.append([t.name, t.type, t.offset, t.nbytes, nbad])
                syn = gguf_bytes(parts)
                del parts
                ch["f"] = self._r2_file(syn)
                ch["fmeta"] = zstd.zstd_c(json.dumps(meta).encode())
                ch["fexc"] = zstd.zstd_c(b"".join(a.tobytes() for a in idx) + b"".join(a.tobytes() for a in vals))
            # other quant types (a Q4_K_M seed's tensors): QR without a seed per type where it beats zstd-9
            selfq = {}
            for t in other:
                if t.type in qr.SELF_TYPES and t.shape[0] % qr.QK[t.type] == 0:
                    selfq.setdefault(t.type, []).append(t)
            sq = []
            for T, ts in selfq.items():
                blobs = [host[t.offset:t.offset + t.nbytes] for t in ts]
                c = qr.self_encode(T, [(b, t.shape[0]) for b, t in zip(blobs, ts)], stream=self.stream)
                if len(c) < len(zstd.zstd_c(b"".join(b.tobytes() for b in blobs), 9)):
                    ch[f"s{len(sq)}"] = c
                    sq.append([T, [[t.offset, t.nbytes] for t in ts]])
            done = {o for _, lst in sq for o, _ in lst}
            other = [t for t in other if t.offset not in done]
            if sq:
                ch["smeta"] = zstd.zstd_c(json.dumps(sq).encode())
            if other:
                ch["o"] = zstd.zstd_c(b"".join(host[t.offset:t.offset + t.nbytes].tobytes() for t in other), 9)
                ch["ometa"] = zstd.zstd_c(json.dumps([[t.offset, t.nbytes] for t in other]).encode())
            ch["rest"] = rest.result()
        return pack(ch)

    def _r2_file(self, syn):
        """the BF16 codec's whole-file chunk (BF16v2.compress, bf16v2.py:273-289) of the synthetic GGUF"""
        h = np.frombuffer(syn, np.uint8)
        g = gguf.GGUF(h)
        lay = r2.layout_of([(t.name, t.offset, t.nbytes, t.shape[0]) for t in g.tensors if t.type == BF16
                            and len(t.shape) == 2], len(h))
        rest = header.header_c(h, g, lay)
        d = dev.DeviceArray.from_host(h, self.stream)
        return b"".join(bytes(p) for p in self.r2.compress_parts(d, lay, rest=rest, order="parts"))

    def decompress(self, buf):
        """-> the file (numpy uint8)"""
        ch = unpack(memoryview(buf) if not isinstance(buf, memoryview) else buf)
        lay = json.loads(zstd.decompress(ch["layout"]))
        out = np.zeros(lay["size"], np.uint8)
        with ThreadPoolExecutor(1) as ex:
            rest = ex.submit(header.header_d, bytes(ch["rest"]))
            if "q8" in ch:
                self.q8.decompress(ch["q8"], out=out)
            if "f" in ch:
                syn = self.r2.decompress(bytes(ch["f"]))
                syn = np.asarray(syn).reshape(-1).view(np.uint8)
                gs = gguf.GGUF(syn, light=True)
                meta = json.loads(zstd.decompress(ch["fmeta"]))
                exc = zstd.decompress(ch["fexc"])
                nexc = sum(m[4] for m in meta)
                idx = np.frombuffer(exc, np.uint32, nexc)
                vals = np.frombuffer(exc, np.uint16, nexc, 4 * nexc)
                e = 0
                if len(meta) != len(gs.tensors):
                    raise ValueError("seed: float tensor list does not match the coded file")
                for (name, ty, off, nb, ne), st in zip(meta, gs.tensors):
                    u = syn[st.offset:st.offset + st.nbytes].view(np.uint16)
                    if ty == F16:
                        u = f16_from_bf16(u)
                        if ne:
                            u[idx[e:e + ne]] = vals[e:e + ne]
                        e += ne
                    out[off:off + nb] = u.view(np.uint8)
                del syn
            if "smeta" in ch:
                for k, (T, lst) in enumerate(json.loads(zstd.decompress(ch["smeta"]))):
                    for (off, nb), arr in zip(lst, qr.self_decode(T, ch[f"s{k}"], stream=self.stream)):
                        a = arr.to_host(stream=self.stream) if isinstance(arr, dev.DeviceArray) else np.asarray(arr)
                        out[off:off + nb] = a.reshape(-1).view(np.uint8)[:nb]
            if "o" in ch:
                o, pos = zstd.decompress(ch["o"]), 0
                for off, nb in json.loads(zstd.decompress(ch["ometa"])):
                    out[off:off + nb] = np.frombuffer(o, np.uint8, nb, pos)
                    pos += nb
            header.fill_rest(out, rest.result(), lay)
        return out
