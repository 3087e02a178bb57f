"""Residual-stage decisions on the host (seedpack/repo3.py:691-700, :1100-1109, :1861-1867)."""
from seedpack_amd import residual as r


def test_kind():
    assert r.kind(r.BF16, 1024, r.F16, 1024, 2048) == "xor"
    assert r.kind(r.BF16, 1024, 12, 1024, 4 * 144) == "rq"
    assert r.kind(r.BF16, 1024, 12, 1024, 4 * 144 + 1) is None          # odd byte size
    assert r.kind(r.BF16, 512, 12, 1024, 4 * 144) is None               # shape mismatch
    assert r.kind(None, 1024, 12, 1024, 4 * 144) is None                # no base tensor
    assert r.kind(77, 1024, 12, 1024, 4 * 144) is None                  # base of another kind
    assert r.kind(12, 1024, 14, 1024, 4 * 210) == "rq"                  # quantized base (seed)


def test_first_variant():
    assert r.v0("rq", True) == 0
    assert r.v0("rq", False) == r.UNIT_W
    assert r.v0("xor", False) == 0
    assert r.v0("rq", True, fitted_set=2, in_fitted_set=True) == 2 * r.RECOV
    assert r.v0("rq", False, fitted_set=2, in_fitted_set=False) == r.UNIT_W


def test_candidates():
    assert r.candidates(29, 0) == [1]                                    # IQ1_M: its older search
    assert r.candidates(12, 0) == []
    assert r.candidates(12, r.UNIT_W) == [0]                             # unit weights -> unweighted
    assert r.candidates(29, r.UNIT_W) == [r.UNIT_W + 1]                  # IQ types have no unweighted path
    assert r.candidates(16, r.UNIT_W) == []
    assert r.candidates(29, 3 * r.RECOV) == [3 * r.RECOV + 1, 0, 1]
    assert r.candidates(12, 3 * r.RECOV) == [0]


def test_split_variant():
    assert r.split_variant(0) == (0, False, 0)
    assert r.split_variant(1) == (0, False, 1)
    assert r.split_variant(r.UNIT_W + 1) == (0, True, 1)
    assert r.split_variant(2 * r.RECOV + 1) == (2, False, 1)
