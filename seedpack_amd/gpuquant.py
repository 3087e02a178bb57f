"""Host side of the regrow quantizers: the reference's GPUQuant interface over the HIP C ABI.

Mirrors seedpack/gpuquant.py:284-456 (GPUQuant.quantize_tensors / quantize_batch): same argument
meaning and result layout. Differences that follow from the MI355X design:
  * weights are widened BF16/F16 -> f32 inside the quantizer's load (no f32 staging buffer, so
    `max_weights` only bounds how many weights one call hands to the GPU at a time);
  * every tensor is one launch of one kernel over its contiguous run of blocks (the reference runs
    one thread per row, gpuquant.py:432-456).
"""
import numpy as np

from . import device as dev
from ._lib import check, lib
from .requant import NEED_IMATRIX, QFUN, VARIANTS

SRC_BF16, SRC_F16, SRC_F32 = 0, 1, 2


def _src_kind(a):
    dt = np.dtype(a.dtype)
    if dt == np.uint16:
        return SRC_BF16
    if dt == np.float16:
        return SRC_F16
    if dt == np.float32:
        return SRC_F32
    raise TypeError(f"weights must be bf16 bits (uint16), float16 or float32, not {dt}")


def quantize_into(ttype, src, n_per_row, dst, imatrix=None, variant=0, stream=None):
    """one tensor: src DeviceArray (nrows*n_per_row weights) -> dst DeviceArray (bytes); enqueue only"""
    if ttype not in QFUN:
        raise ValueError(f"unknown ggml type {ttype}")
    nrows = src.size // n_per_row
    assert nrows * n_per_row == src.size, "tensor size is not a whole number of rows"
    need = nrows * (n_per_row // QFUN[ttype][1]) * QFUN[ttype][2]
    assert dst.nbytes >= need, (dst.nbytes, need)
    wb = lib().spa_quantize_work_bytes(ttype, nrows, n_per_row, imatrix is not None)
    # the scratch goes back to this thread's cache when the call returns: the next block taken from
    # it is used on the same stream, after this launch
    work = dev.DeviceArray(wb, np.uint8) if wb else None
    check(lib().spa_quantize(ttype, variant, src.ptr, _src_kind(src), nrows, n_per_row,
                             None if imatrix is None else imatrix.ptr, dst.ptr, None if work is None else work.ptr,
                             stream))
    return dst


class GPUQuant:
    """llama.cpp quantizers on the MI355X, byte-identical to the CPU library (gpuquant.py:284)."""

    def __init__(self, fmad=False, stream=None):
        if fmad:
            raise ValueError("fmad=True (FMA-contracted quantizers) is not built: every kernel is compiled "
                             "with -ffp-contract=off")
        lib()
        self.stream = stream

    def _dev(self, a):
        # uploads go on this quantizer's stream: the library's streams do not wait for the null
        # stream, and a block freed here is reused by the next upload while earlier launches on the
        # stream may still read it
        return a if isinstance(a, dev.DeviceArray) else dev.DeviceArray.from_host(np.ascontiguousarray(a), self.stream)

    def _imx(self, imx, npr):
        if imx is None:
            return None
        if isinstance(imx, dev.DeviceArray):
            return imx
        imx = np.ascontiguousarray(imx, np.float32).reshape(-1)
        assert imx.size == npr, (imx.size, npr)
        return dev.DeviceArray.from_host(imx, self.stream)

    def quantize_tensors(self, ttype, srcs, imatrices, variant=0, max_weights=1 << 28, on_result=None, device=False):
        """srcs: list of (weights, n_per_row); weights are bf16 bits (uint16) / f16 / f32 (device or host
        array) or an object with `size` and `into(out)` that writes its float32 weights into the
        DeviceArray `out` (a seed's tensor dequantized straight into the launch's input, as the
        reference's _Dequant does, repo3.py:545-557). Consecutive tensors are handed to the device in
        groups of at most `max_weights` weights (the `into` sources of a group share one float32
        buffer; a larger array is quantized in row pieces); the quantizer runs once per tensor over its
        run of blocks. Returns the quantized bytes of every tensor (host numpy arrays, DeviceArrays with
        `device`), or with on_result calls on_result(index, bytes) per tensor as its group completes and
        returns None (gpuquant.py:360-411)."""
        if ttype in NEED_IMATRIX and any(m is None for m in imatrices):
            raise ValueError(f"type {ttype} requires an imatrix")
        if variant >= VARIANTS.get(ttype, 1):
            raise ValueError(f"type {ttype} has no variant {variant}")
        _, qk, bs = QFUN[ttype]
        out, i = [], 0
        while i < len(srcs):
            j, n = i, 0
            while j < len(srcs) and (j == i or n + srcs[j][0].size <= max_weights):
                n += srcs[j][0].size
                j += 1
            lazy = sum(srcs[k][0].size for k in range(i, j) if hasattr(srcs[k][0], "into"))
            X = dev.DeviceArray(lazy, np.float32) if lazy else None
            at, done = 0, []
            for k in range(i, j):
                a, npr = srcs[k]
                if hasattr(a, "into"):
                    x = X.view(4 * at, (a.size,), np.float32)
                    a.into(x)
                    at += a.size
                else:
                    x = self._dev(a)
                w = self._imx(imatrices[k], npr)
                nrow = x.size // npr
                if nrow * npr != x.size or npr % qk:
                    raise ValueError(f"tensor {k}: {x.size} weights are not whole rows of {npr} (type {ttype})")
                rb = npr // qk * bs
                y = dev.DeviceArray(nrow * rb, np.uint8)
                step = max(1, max_weights // npr)
                for r0 in range(0, nrow, step):
                    r1 = min(nrow, r0 + step)
                    xs = x.view(r0 * npr * x.dtype.itemsize, (r1 - r0) * npr, x.dtype)
                    quantize_into(ttype, xs, npr, y.view(r0 * rb, (r1 - r0) * rb, np.uint8), w, variant, self.stream)
                done.append(y)
            for k, y in enumerate(done, i):
                res = y if device else y.to_host(stream=self.stream)
                if on_result:
                    on_result(k, res)
                else:
                    out.append(res)
            del X
            i = j
        return None if on_result else out

    def dequantize(self, ttype, y, npr, out=None):
        """quantized bytes of a tensor (DeviceArray or host uint8, rows of npr weights) -> float32
        DeviceArray (or into `out`), llama.cpp's dequantize_row_<type> (gpuquant.py:413-421)"""
        if ttype not in QFUN:
            raise ValueError(f"unknown ggml type {ttype}")
        _, qk, bs = QFUN[ttype]
        y = self._dev(y)
        rb = npr // qk * bs
        nrows = y.nbytes // rb
        if npr % qk or nrows * rb != y.nbytes:
            raise ValueError(f"{y.nbytes} bytes are not whole rows of {npr} weights of type {ttype}")
        x = dev.DeviceArray(nrows * npr, np.float32) if out is None else out
        if x.nbytes < nrows * npr * 4:
            raise ValueError("output too small")
        check(lib().spa_dequantize(ttype, y.ptr, nrows, npr, x.ptr, self.stream))
        return x

    def quantize_batch(self, ttype, xs, imatrices, variant=0):
        """xs: list of float32 arrays (nrows, n_per_row); returns device uint8 arrays (gpuquant.py:424-430)"""
        return self.quantize_tensors(ttype, [(x, x.shape[-1]) for x in xs], imatrices, variant, device=True)
