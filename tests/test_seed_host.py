"""Host parts of the seed codec (seedpack_amd/seed.py): the minimal GGUF writer reads back with the GGUF
reader, BF16 <-> F16 conversions are exact where the value allows, bits per weight picks the senior
quant."""
import numpy as np

from seedpack_amd import gguf, seed


def test_gguf_bytes_reads_back():
    a = np.arange(96, dtype=np.uint16).tobytes()
    b = np.arange(33, dtype=np.uint8).tobytes()
    data = seed.gguf_bytes([("x.weight", (32, 3), 30, a), ("y", (33,), 24, b)])
    g = gguf.GGUF(np.frombuffer(data, np.uint8))
    assert [(t.name, t.shape, t.type) for t in g.tensors] == [("x.weight", (32, 3), 30), ("y", (33,), 24)]
    t0, t1 = g.tensors
    assert data[t0.offset:t0.offset + t0.nbytes] == a and data[t1.offset:t1.offset + t1.nbytes] == b
    assert t0.offset % 32 == 0 and t1.offset % 32 == 0


def test_f16_bf16_conversions():
    g = np.random.Generator(np.random.PCG64(1))
    bf = (g.normal(0, 0.05, 4096).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    f16 = seed.f16_from_bf16(bf)
    # values F16 holds come back exactly; BF16 values convert to F16 and back without change
    held = np.abs(bf.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    ok = (np.abs(held) >= 2.0 ** -14) & (np.abs(held) < 65504)
    assert np.array_equal(seed.bf16_of_f16(f16)[ok], bf[ok])
    # an F16 value that is not a BF16 value is truncated, and flagged by the round trip
    u = np.array([0x3C01], np.uint16)                 # 1 + 2^-10
    assert seed.bf16_of_f16(u)[0] == 0x3F80 and seed.f16_from_bf16(seed.bf16_of_f16(u))[0] != u[0]


def test_bits_per_weight_orders_quants():
    T = gguf.Tensor
    q8 = [T("a", (256, 4), 8, 0, 4 * 8 * 34)]
    q4k = [T("a", (256, 4), 12, 0, 4 * 144)]
    assert seed.bits_per_weight(q8) == 8.5 and seed.bits_per_weight(q4k) == 4.5
