"""The seed codec (seedpack_amd/seed.py) on the MI355X: a base-less quantized GGUF coded by parts equals
the reference's SeedCodec output part by part (tests/golden/seed_vectors.npz, written by
make_seed_golden.py through the reference's --cpu backend), and the reference's chunks decode back
to the exact file."""
import os
import sys

import numpy as np
import pytest

from seedpack_amd import framing, seed, zstd

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CASES = ["tok", "plain"]
ZSTD_PARTS = ("layout", "fmeta", "fexc", "smeta", "o", "ometa")


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(ROOT, "tests", "golden", "seed_vectors.npz"))


@pytest.mark.parametrize("name", CASES)
def test_seed_codec_equals_reference(gold, name):
    say("case seed", name)
    data = gold[f"{name}/input"].tobytes()
    want = gold[f"{name}/chunk"].tobytes()
    mine = seed.SeedCodec().compress(data)
    a, b = framing.unpack(mine), framing.unpack(want)
    assert list(a) == list(b), f"parts {list(a)} vs {list(b)}"
    for k in b:
        x, y = bytes(a[k]), bytes(b[k])
        if k in ZSTD_PARTS:
            x, y = zstd.decompress(x), zstd.decompress(y)
        if k in ("q8", "f"):
            pa, pb = framing.unpack(x), framing.unpack(y)
            assert list(pa) == list(pb), f"part {k}: {list(pa)} vs {list(pb)}"
            for kk in pb:
                assert bytes(pa[kk]) == bytes(pb[kk]), f"part {k}/{kk}"
        assert x == y, f"part {k}"
    assert mine == want


@pytest.mark.parametrize("name", CASES)
def test_seed_codec_decodes_reference(gold, name):
    say("case seed decode", name)
    data = gold[f"{name}/input"].tobytes()
    out = seed.SeedCodec().decompress(gold[f"{name}/chunk"].tobytes())
    assert out.tobytes() == data
