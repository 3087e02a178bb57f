"""The library's IQ lattice tables equal the reference's table fixture (digests of iqtables.npz)."""
import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

from seedpack_amd._lib import check, lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAMES = ["iq2_data_0", "iq2_data_1", "iq2_data_2", "iq2_data_3", "iq3_data_0", "iq3_data_1"]


def host_table(i):
    g, gn, m, mn, nb, nbn = (ctypes.c_void_p(), ctypes.c_int(), ctypes.c_void_p(), ctypes.c_int(), ctypes.c_void_p(),
                             ctypes.c_int())
    check(lib().spa_iq_table_host(i, ctypes.byref(g), ctypes.byref(gn), ctypes.byref(m), ctypes.byref(mn),
                                  ctypes.byref(nb), ctypes.byref(nbn)))
    grid = np.ctypeslib.as_array(ctypes.cast(g, ctypes.POINTER(ctypes.c_uint8)), (gn.value,)).copy()
    kmap = np.ctypeslib.as_array(ctypes.cast(m, ctypes.POINTER(ctypes.c_int32)), (mn.value,)).copy()
    nbs = np.ctypeslib.as_array(ctypes.cast(nb, ctypes.POINTER(ctypes.c_uint16)), (nbn.value,)).copy()
    return grid, kmap, nbs


@pytest.mark.parametrize("i", range(6))
def test_iq_tables_equal_reference_fixture(i):
    man = json.load(open(os.path.join(ROOT, "tests", "golden", "iqtables_sha256.json")))
    grid, kmap, nbs = host_table(i)
    name = NAMES[i]
    g = grid.view(np.uint64 if i < 4 else np.uint32)
    assert hashlib.sha256(g.tobytes()).hexdigest() == man[name + "_grid"]["sha256"]
    assert hashlib.sha256(kmap.tobytes()).hexdigest() == man[name + "_map"]["sha256"]
    assert nbs.size == man[name + "_nb"]["n"]
    assert hashlib.sha256(nbs.tobytes()).hexdigest() == man[name + "_nb"]["sha256"]


def test_neighbour_lists_are_nearest_by_brute_force():
    """IQ3_XXS: every listed neighbour of an off-grid index is within the nwant nearest distances and
    the list is ordered by (distance, index)"""
    grid, kmap, nbs = host_table(4)
    pts = grid.reshape(-1, 4).astype(np.int64)
    for i in [1, 7, 100, 1000, 4095]:
        if kmap[i] >= 0:
            continue
        pos = 2 * ((i >> (3 * np.arange(4))) & 7) + 1
        d2 = ((pts - pos) ** 2).sum(1)
        o = -kmap[i] - 1
        lst = nbs[o + 1:o + 1 + nbs[o]]
        levels = np.unique(d2)[:2]
        want = [j for d in levels for j in np.flatnonzero(d2 == d)]
        assert list(lst) == want
