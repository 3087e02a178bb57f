"""zstd framing of the small coded parts: round trip, and the same frames when another libzstd is
already in the process's global symbol scope (a profiler's preloaded library links the system one;
without binding the preferred copy to itself, its internal calls land in the other version and
either crash or change the level-19 output)."""
import glob
import os
import subprocess
import sys

import numpy as np
import pytest

from seedpack_amd import zstd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_PROBE = """
import sys, numpy as np
sys.path.insert(0, %r)
from seedpack_amd import zstd
g = np.random.default_rng(1)
for n in (100, 5000, 300000):
    d = (g.integers(0, 20, n) ** 2).astype(np.uint16).tobytes()
    c = zstd.compress(d)
    assert zstd.decompress(c) == d
    print(n, len(c), bytes(c[-8:]).hex())
""" % ROOT


def test_round_trip():
    g = np.random.default_rng(7)
    for n in (0, 1, 4096, 100000):
        d = g.integers(0, 7, n).astype(np.uint8).tobytes()
        assert zstd.decompress(zstd.compress(d)) == d


def test_other_libzstd_in_global_scope():
    system = sorted(glob.glob("/lib/x86_64-linux-gnu/libzstd.so.1*")) + sorted(glob.glob("/usr/lib/x86_64-linux-gnu/libzstd.so.1*"))
    if not system:
        pytest.skip("no system libzstd to preload")
    plain = subprocess.run([sys.executable, "-c", _PROBE], capture_output=True, text=True, timeout=120)
    assert plain.returncode == 0, plain.stderr
    env = dict(os.environ, LD_PRELOAD=system[0])
    pre = subprocess.run([sys.executable, "-c", _PROBE], capture_output=True, text=True, timeout=120, env=env)
    assert pre.returncode == 0, pre.stderr
    assert pre.stdout == plain.stdout
