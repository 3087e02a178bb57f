"""BLAKE3 on the device (spa_blake3): regions of one buffer, every tree shape across the stage
boundaries (256 chunks per first-stage workgroup, 512 nodes per later one), unaligned and empty
regions, against the oracle restatement and the library's host hasher (pinned to the published
digests by tests/test_blake3.py)."""
import sys

import numpy as np
import pytest

from oracle import blake3 as ob
from seedpack_amd import blake3
from seedpack_amd import device as dev

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def test_device_small_regions_equal_oracle():
    say("case blake3 small regions")
    g = np.random.Generator(np.random.PCG64(11))
    buf = g.integers(0, 256, 64 << 10, dtype=np.uint8)
    regions = [(0, 0), (0, 1), (3, 63), (16, 64), (5, 65), (0, 1024), (1, 1024), (32, 1025), (100, 3073),
               (0, 4096), (4096, 9 * 1024 + 17), (777, 20000)]
    d = dev.DeviceArray.from_host(buf)
    got = blake3.device_digests(d, regions)
    for (o, n), h in zip(regions, got):
        assert h == ob.digest(buf[o:o + n].tobytes()), (o, n)
    pub = np.frombuffer(bytes(i % 251 for i in range(4096)), np.uint8)
    dp = dev.DeviceArray.from_host(pub)
    assert blake3.device_digests(dp, [(0, 3073)])[0].hex() == "7124b49501012f81cc7f11ca069ec9226cecb8a2c850cfe644e327d22d3e1cd3"
    assert blake3.device_digests(dp, [(0, 0)])[0].hex() == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"


@pytest.mark.parametrize("nchunks", [255, 256, 257, 511, 512, 513, 256 * 512 - 1, 256 * 512, 256 * 512 + 1,
                                     256 * 512 * 3 + 5])
def test_device_stage_boundaries_equal_host(nchunks):
    say("case blake3 chunks", nchunks)
    g = np.random.Generator(np.random.PCG64(nchunks))
    for extra in (0, 333):
        n = nchunks * 1024 + extra
        buf = g.integers(0, 256, n + 16, dtype=np.uint8)
        d = dev.DeviceArray.from_host(buf)
        got = blake3.device_digests(d, [(0, n), (16, n)])
        assert got[0].hex() == blake3.hexdigest(buf[:n]), (nchunks, extra)
        assert got[1].hex() == blake3.hexdigest(buf[16:16 + n]), (nchunks, extra)


def test_device_many_regions_one_call():
    say("case blake3 many regions")
    g = np.random.Generator(np.random.PCG64(12))
    buf = g.integers(0, 256, 24 << 20, dtype=np.uint8)
    sizes = g.integers(0, 600 << 10, 120)
    offs = g.integers(0, (24 << 20) - (600 << 10), 120) // 32 * 32
    regions = [(int(o), int(s)) for o, s in zip(offs, sizes)] + [(0, 24 << 20)]
    buf[offs[7]:offs[7] + 5000] = buf[offs[9]:offs[9] + 5000]
    regions += [(int(offs[7]), 5000), (int(offs[9]), 5000)]
    d = dev.DeviceArray.from_host(buf)
    got = blake3.device_digests(d, regions)
    for (o, n), h in zip(regions, got):
        assert h.hex() == blake3.hexdigest(buf[o:o + n]), (o, n)
    assert got[-1] == got[-2]                      # equal bytes at different places: equal keys
