"""spa_qr_encode_noalloc (the allocation-free QR encoder, static per-device scratch) against
spa_qr_encode (caller workspace) through the C ABI: the same segment lengths and the same stream
bytes, on two calls in a row, the second with a smaller batch (the scratch keeps the first call's
contents)."""
import ctypes
import sys

import numpy as np
import pytest

from seedpack_amd import device as dev
from seedpack_amd import qr, synth
from seedpack_amd._lib import check, lib
from seedpack_amd.gpuquant import GPUQuant

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _batch(T, rows, cols, seed):
    """(F, P, seed tensor, imatrix or None): P the type's quantization of a seeded tensor, F = P with
    1% of its blocks changed in one byte"""
    g = np.random.Generator(np.random.PCG64(seed))
    w = synth.normal_bf16(g, (rows, cols), 0.02, outlier_frac=0.001)
    imx = g.lognormal(0, 1, cols).astype(np.float32) if T in qr.GRID_TYPES else None
    P = GPUQuant().quantize_tensors(T, [(w.reshape(-1), cols)], [imx])[0]
    Fb = P.copy().reshape(-1, qr.BS[T])
    idx = g.choice(len(Fb), size=max(1, len(Fb) // 100), replace=False)
    Fb[idx, g.integers(0, qr.BS[T], len(idx))] ^= np.uint8(0x24)
    return Fb.reshape(-1), P, w.reshape(-1), imx


def _encode_both(T, F, P, w, imx, cols):
    """the batch encoded by spa_qr_encode and by spa_qr_encode_noalloc with the same tables ->
    ((lens, slots) of each)"""
    L = lib()
    sd = dev.DeviceArray.from_host(w.view(np.uint8))
    imx_d = None if imx is None else dev.DeviceArray.from_host(imx)
    item = (F, P, 0, 30, cols, 0 if imx is not None else -1)
    parts = qr.encode_parts(T, [item], sd, imx_d)           # histogram and tables
    tm, sg, nb = qr._descriptors(T, [len(F) // qr.BS[T]], [item[2:]])
    nseg = len(sg)
    remap = np.full(qr.NTAB2, -1, np.int32)
    remap[parts["used"]] = np.arange(len(parts["used"]), dtype=np.int32)
    cum = qr.cum_of(parts["freq"])
    Fd, Pd = dev.DeviceArray.from_host(F), dev.DeviceArray.from_host(P)
    tm_d, sg_d = dev.DeviceArray.from_host(tm.view(np.uint8)), dev.DeviceArray.from_host(sg.view(np.uint8))
    remap_d, freq_d, cum_d = (dev.DeviceArray.from_host(a) for a in (remap, parts["freq"], cum))
    gk = qr._gk_ptr(T)
    cap = qr.seg_blocks(T) * (3 * qr.BS[T] if T in qr.GRID_TYPES else (qr.QK[T] + qr.NSB_MAX) * 2) + 1024
    out = []
    for noalloc in (False, True):
        slots = dev.DeviceArray(nseg * cap, np.uint8)
        check(L.spa_memset(slots.ptr, 0, slots.nbytes, None))
        lens = dev.DeviceArray(nseg, np.uint32).zero()
        args = (T, Fd.ptr, Pd.ptr, sd.ptr, tm_d.ptr, sg_d.ptr, nseg, remap_d.ptr, freq_d.ptr, cum_d.ptr, slots.ptr,
                cap, lens.ptr, gk, None if imx_d is None else imx_d.ptr, qr.MODEL)
        if noalloc:
            check(L.spa_qr_encode_noalloc(*args, None))
        else:
            work = dev.DeviceArray(max(1, L.spa_qr_work_bytes(T, nseg)), np.uint8)
            check(L.spa_qr_encode(*args, work.ptr, None))
        dev.synchronize()
        out.append((lens.to_host(), slots.to_host()))
    assert np.array_equal(out[0][0], parts["lens"]), "spa_qr_encode differs from encode_parts"
    return out


@pytest.mark.parametrize("T,shapes", [(2, ((512, 4096), (96, 1024))), (12, ((256, 4096), (64, 2048))),
                                      (17, ((64, 4096), (16, 2048)))])
def test_noalloc_encoder_equals_workspace_encoder(T, shapes):
    for k, (rows, cols) in enumerate(shapes):
        say(f"case qr noalloc T={T} rows={rows} cols={cols}")
        F, P, w, imx = _batch(T, rows, cols, 0x7007 + 16 * T + k)
        (l0, s0), (l1, s1) = _encode_both(T, F, P, w, imx, cols)
        assert (l0 != 0xFFFFFFFF).all()
        assert np.array_equal(l0, l1), "segment lengths"
        assert s0.tobytes() == s1.tobytes(), "segment slots"


def test_noalloc_rejects_a_batch_beyond_its_scratch():
    L = lib()
    big = 1
    while L.spa_qr_work_bytes(8, big) <= L.spa_qr_noalloc_scratch_bytes():
        big *= 2
    rc = L.spa_qr_encode_noalloc(8, None, None, None, None, None, big, None, None, None, None, 1 << 16, None, None, None,
                                 2, None)
    assert rc == -4 and b"static scratch" in L.spa_last_error()


def _prepare(T, F, P, w, imx, cols):
    """device inputs and tables of one batch -> (argument tuple without out/lens, nseg, cap, keep)"""
    sd = dev.DeviceArray.from_host(w.view(np.uint8))
    imx_d = None if imx is None else dev.DeviceArray.from_host(imx)
    item = (F, P, 0, 30, cols, 0 if imx is not None else -1)
    parts = qr.encode_parts(T, [item], sd, imx_d)
    tm, sg, nb = qr._descriptors(T, [len(F) // qr.BS[T]], [item[2:]])
    remap = np.full(qr.NTAB2, -1, np.int32)
    remap[parts["used"]] = np.arange(len(parts["used"]), dtype=np.int32)
    keep = [sd, imx_d, dev.DeviceArray.from_host(F), dev.DeviceArray.from_host(P),
            dev.DeviceArray.from_host(tm.view(np.uint8)), dev.DeviceArray.from_host(sg.view(np.uint8)),
            dev.DeviceArray.from_host(remap), dev.DeviceArray.from_host(parts["freq"]),
            dev.DeviceArray.from_host(qr.cum_of(parts["freq"]))]
    cap = qr.seg_blocks(T) * (3 * qr.BS[T] if T in qr.GRID_TYPES else (qr.QK[T] + qr.NSB_MAX) * 2) + 1024
    return keep, len(sg), cap, parts


def test_noalloc_calls_on_two_streams_do_not_race():
    """two batches encoded by spa_qr_encode_noalloc on two streams, queued back to back with no wait
    between them: each gives the bytes of its batch encoded alone, one call at a time (the library
    orders the shared scratch's uses by its per-device event)"""
    L = lib()
    T = 12
    say(f"case qr noalloc two streams T={T}")
    batches = []
    for k, (rows, cols) in enumerate(((384, 4096), (256, 2048))):
        F, P, w, imx = _batch(T, rows, cols, 0x7707 + k)
        batches.append(_prepare(T, F, P, w, imx, cols))
    streams = [dev.Stream(), dev.Stream()]
    res = []
    for rep in range(3):
        outs = []
        for (keep, nseg, cap, parts), st in zip(batches, streams):
            sd, imx_d, Fd, Pd, tm_d, sg_d, remap_d, freq_d, cum_d = keep
            slots = dev.DeviceArray(nseg * cap, np.uint8)
            lens = dev.DeviceArray(nseg, np.uint32)
            check(L.spa_memset(slots.ptr, 0, slots.nbytes, st.handle))
            check(L.spa_memset(lens.ptr, 0, lens.nbytes, st.handle))
            check(L.spa_qr_encode_noalloc(T, Fd.ptr, Pd.ptr, sd.ptr, tm_d.ptr, sg_d.ptr, nseg, remap_d.ptr, freq_d.ptr,
                                          cum_d.ptr, slots.ptr, cap, lens.ptr, qr._gk_ptr(T), None, qr.MODEL, st.handle))
            if rep == 0:                  # the reference run: one call at a time
                st.synchronize()
            outs.append((slots, lens))
        for st in streams:
            st.synchronize()
        res.append([(l.to_host(), s.to_host()) for s, l in outs])
    for k, (keep, nseg, cap, parts) in enumerate(batches):
        assert np.array_equal(res[0][k][0], parts["lens"]), f"batch {k}: lengths differ from encode_parts"
        for rep in range(1, 3):
            assert np.array_equal(res[rep][k][0], res[0][k][0])
            assert res[rep][k][1].tobytes() == res[0][k][1].tobytes()
