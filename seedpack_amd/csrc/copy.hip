// A plain streaming copy kernel: device-to-device copy of whole 16-byte words. It is the
// bandwidth yardstick that HBM traffic counters of the other kernels are scaled against.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace {
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}
}  // namespace

extern "C" int spa_copy(void* dst, const void* src, size_t nbytes, void* stream) {
    if ((nbytes & 15u) || (reinterpret_cast<uintptr_t>(dst) & 15u) || (reinterpret_cast<uintptr_t>(src) & 15u))
        return spa::fail(SPA_ERR_ARG, "spa_copy: pointers and size must be 16-byte multiples");
    const int64_t n = (int64_t)(nbytes / 16);
    if (n == 0) return SPA_OK;
    const int64_t blocks = (n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192;
    hipLaunchKernelGGL(k_copy16, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)src, (uint4*)dst, n);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}
