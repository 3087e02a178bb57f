"""M24 (method m28's BF16 codec, seedpack_amd/m24.py) on the MI355X: side information, tables,
segment lengths and stream bytes equal the reference's own kernels and statistics
(tests/golden/m24_vectors.npz, written by make_m24_golden.py through the reference's --cpu backend);
chunks decode back to the file's exact bytes."""
import os
import sys

import numpy as np
import pytest

from seedpack_amd import device as dev
from seedpack_amd import gguf, header, m24, zstd
from seedpack_amd.r2 import load_tables
from tests.golden.r2_cases import CASES, case_file

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(ROOT, "tests", "golden", "m24_vectors.npz"))


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_m24_equals_reference(gold, name):
    say("case m24", name)
    data, lay, _ = case_file(name)
    layout = {"size": lay["size"], "t": lay["t"]}
    host = np.frombuffer(data, np.uint8)
    codec = m24.M24BF16()
    d = dev.DeviceArray.from_host(host)
    rfi, cfi, scl = codec.side_info(d, layout)
    assert np.array_equal(rfi, gold[f"{name}/rfi"]) and np.array_equal(cfi, gold[f"{name}/cfi"]), "rfi / cfi"
    assert np.array_equal(scl, gold[f"{name}/scl"]), "scl"
    stream, lens, tabs = codec.encode(d, layout, rfi, cfi, scl)
    freq, used = load_tables(tabs)
    assert np.array_equal(used, gold[f"{name}/used"]) and np.array_equal(freq, gold[f"{name}/freq"]), "tables"
    assert np.array_equal(lens, gold[f"{name}/lens"]), "segment lengths"
    assert np.frombuffer(stream, np.uint8).tobytes() == gold[f"{name}/stream"].tobytes(), "stream"
    ch = {"layout": zstd.zstd_c(__import__("json").dumps(layout).encode()),
          "side": zstd.zstd_c(rfi.tobytes() + cfi.tobytes() + scl.tobytes(), 19), "tables": tabs,
          "lens": zstd.zstd_c(lens.astype(np.uint32).tobytes()), "stream": stream,
          "rest": header.header_x(header.rest_of(data, layout))}
    assert codec.decompress_dev(ch).to_host().tobytes() == data


def test_m24_gguf_round_trip():
    """a GGUF with a tokenizer (the header coder's P form), BF16 matrices, F32 norms"""
    from tests.golden.header_cases import case_file as hcase
    data, _ = hcase("bpe")
    codec = m24.M24BF16()
    buf = codec.compress(data)
    from seedpack_amd.framing import unpack
    parts = unpack(memoryview(buf))
    assert list(parts) == ["layout", "side", "tables", "lens", "stream", "rest"]
    assert bytes(parts["rest"][:1]) == b"P"
    assert codec.decompress(buf).tobytes() == data
    g = gguf.GGUF(data)
    assert len(m24.layout_of(g, len(data))["t"]) == 3
