"""HIP dequantizers vs the reference's own dequantize_row_<type> (oracle/_ref, the C sources compiled
by oracle/Makefile): bit-identical float32 for every type, on blocks the quantizers produce and on
random blocks (every code, grid point and sign pattern; fp16 fields kept finite)."""
import sys

import numpy as np
import pytest

from oracle import ref
from seedpack_amd import device as dev
from seedpack_amd import synth
from seedpack_amd.gpuquant import GPUQuant
from seedpack_amd.requant import NAMES, NEED_IMATRIX, QFUN

pytestmark = pytest.mark.gpu
TYPES = sorted(QFUN)

# byte offsets of fp16 fields per block (d, dmin / m); IQ1_M spreads its scale over 4 nibbles
F16_FIELDS = {2: [0], 3: [0, 2], 6: [0], 7: [0, 2], 8: [0], 42: [0], 10: [80, 82], 11: [108], 12: [0, 2], 13: [0, 2],
              14: [208], 16: [0], 17: [0], 18: [0], 19: [0], 20: [0], 21: [0], 22: [0], 23: [0], 29: []}


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gq():
    if not ref.available():
        pytest.skip("oracle/_ref is not built")
    return GPUQuant()


def _check(gq, t, blocks, npr):
    n = len(blocks) // QFUN[t][2] * QFUN[t][1]
    got = gq.dequantize(t, dev.DeviceArray.from_host(blocks), npr).to_host()
    want = ref.dequantize(t, blocks, n)
    assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), NAMES[t]


@pytest.mark.parametrize("t", TYPES)
def test_dequant_of_quantized(gq, t):
    say("case dequant of quantized", NAMES[t])
    g = np.random.Generator(np.random.PCG64(61 + t))
    rows, npr = 24, 1024
    x = synth.bf16_bits(g.standard_t(5, (rows, npr)).astype(np.float32) * 0.02)
    imx = g.lognormal(0, 1, npr).astype(np.float32) if t in NEED_IMATRIX or t % 2 else None
    q = gq.quantize_batch(t, [synth.bf16_to_f32(x).reshape(rows, npr)], [imx])[0]
    _check(gq, t, q.to_host() if isinstance(q, dev.DeviceArray) else np.asarray(q), npr)


def _random_blocks(g, t, nb):
    """nb blocks of random bytes with finite fp16 fields"""
    bs = QFUN[t][2]
    b = g.integers(0, 256, (nb, bs), dtype=np.uint8)
    for o in F16_FIELDS[t]:
        h = (g.normal(0, 0.05, nb)).astype(np.float16)
        b[:, o:o + 2] = h.view(np.uint8).reshape(nb, 2)
    if t == 29:
        b[:, 55] &= 0xBF                      # the scale's exponent stays below 31 (finite)
    return b.reshape(-1)


@pytest.mark.parametrize("t", TYPES)
def test_dequant_of_random_blocks(gq, t):
    say("case dequant of random blocks", NAMES[t])
    g = np.random.Generator(np.random.PCG64(71 + t))
    qk = QFUN[t][1]
    _check(gq, t, _random_blocks(g, t, 4096 * 32 // qk), qk * 32)


@pytest.mark.parametrize("t", TYPES)
def test_dequant_part_tile_and_unaligned_source(gq, t):
    """a block count that leaves a part tile of 4096 weights (and one single block), with the source
    at byte offsets 0, 1, 2, 4 and 8 of an allocation (the kernel's 16-, 4- and 1-byte copy paths)"""
    say("case dequant part tile, unaligned", NAMES[t])
    g = np.random.Generator(np.random.PCG64(81 + t))
    qk, bs = QFUN[t][1], QFUN[t][2]
    for nb in (1, 4096 // qk * 3 + 5):
        blocks = _random_blocks(g, t, nb)
        want = ref.dequantize(t, blocks, nb * qk)
        for off in (0, 1, 2, 4, 8):
            raw = np.zeros(nb * bs + 16, np.uint8)
            raw[off:off + nb * bs] = blocks
            d = dev.DeviceArray.from_host(raw)
            view = dev.DeviceArray(nb * bs, np.uint8, ptr=d.ptr + off, owner=d)
            got = gq.dequantize(t, view, qk).to_host()
            assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), (NAMES[t], nb, off)
