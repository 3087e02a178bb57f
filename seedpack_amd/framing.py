"""Chunk framing of the coded parts (the reference's codecs_gguf.py:26-56 pack format): u32 count,
then per chunk u16 name length, name, u64 data length, data. pack_parts keeps the pieces in a list
(a big stream stays in its pieces, never joined); unpack returns slices of the buffer (no copies for
a memoryview)."""
import struct


def nbytes(data):
    """size of a bytes-like object or of a list of them"""
    if isinstance(data, list):
        return sum(nbytes(d) for d in data)
    return memoryview(data).nbytes


def pack_parts(chunks):
    """chunks {name: bytes-like or list of them} -> list of buffers whose concatenation is pack()"""
    out = [struct.pack("<I", len(chunks))]
    for name, data in chunks.items():
        nb = name.encode()
        out += [struct.pack("<H", len(nb)), nb, struct.pack("<Q", nbytes(data))]
        out += data if isinstance(data, list) else [data]
    return out


def pack(chunks):
    """the chunks in one bytes object (bytes-like parts joined without an intermediate copy)"""
    return b"".join(p if isinstance(p, (bytes, bytearray, memoryview)) else memoryview(p).cast("B")
                    for p in pack_parts(chunks))


def unpack(buf):
    """-> {name: slice of buf}"""
    (n,), pos, chunks = struct.unpack_from("<I", buf), 4, {}
    for _ in range(n):
        (ln,) = struct.unpack_from("<H", buf, pos)
        pos += 2
        name = bytes(buf[pos:pos + ln]).decode()
        pos += ln
        (dl,) = struct.unpack_from("<Q", buf, pos)
        pos += 8
        chunks[name] = buf[pos:pos + dl]
        pos += dl
    return chunks


def index(read, size, base=0):
    """{name: (offset, length)} of the chunks of a packed buffer of `size` bytes that starts at `base`,
    reading only its framing through read(offset, n) -> bytes"""
    (n,), pos, out = struct.unpack("<I", read(base, 4)), base + 4, {}
    for _ in range(n):
        (ln,) = struct.unpack("<H", read(pos, 2))
        name = read(pos + 2, ln).decode()
        (dl,) = struct.unpack("<Q", read(pos + 2 + ln, 8))
        pos += 10 + ln
        if pos + dl > base + size:
            raise ValueError(f"part {name!r} runs past the end of its buffer")
        out[name] = (pos, dl)
        pos += dl
    return out
