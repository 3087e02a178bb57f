// A plain streaming copy kernel: device-to-device copy of whole 16-byte words. It is the
// bandwidth yardstick that HBM traffic counters of the other kernels are scaled against.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace {
// Synthetic BF16 weights N(0, std) for benchmark inputs generated in place: a counter-based
// splitmix64 hash of (seed, index) gives two 24-bit uniforms, Box-Muller's cosine branch a normal
// deviate, rounded to BF16 to nearest even.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ __launch_bounds__(256) void k_synth_normal_bf16(uint16_t* __restrict__ dst, int64_t n, uint64_t seed, float std) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t h = splitmix64(seed * 0xD1342543DE82EF95ull + (uint64_t)i);
        const float u1 = ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
        const float u2 = ((float)(uint32_t)(h & 0xFFFFFFu) + 0.5f) * (1.0f / 16777216.0f);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2) * std;
        const uint32_t u = __float_as_uint(z);
        dst[i] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
}

// Synthetic "published" quant files for benchmarks: in about per_million / 10^6 of the blocks (chosen
// by the same counter hash of (seed, block)), one byte XORed with a non-zero value.
__global__ __launch_bounds__(256) void k_perturb_blocks(uint8_t* __restrict__ dst, int64_t nblocks, int bs,
                                                        uint32_t per_million, uint64_t seed) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks; b += stride) {
        const uint64_t h = splitmix64(seed * 0xD1342543DE82EF95ull + (uint64_t)b);
        if ((uint32_t)(h % 1000000u) < per_million) {
            const int64_t at = b * bs + (int64_t)((h >> 20) % (uint64_t)bs);
            dst[at] ^= (uint8_t)(1 + (h >> 40) % 255u);
        }
    }
}

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

extern "C" int spa_synth_normal_bf16(void* dst, int64_t n, uint64_t seed, float std, void* stream) {
    if (n < 0 || (n > 0 && !dst)) return spa::fail(SPA_ERR_ARG, "spa_synth_normal_bf16: bad arguments");
    if (n == 0) return SPA_OK;
    const int64_t blocks = (n + 255) / 256 < 16384 ? (n + 255) / 256 : 16384;
    hipLaunchKernelGGL(k_synth_normal_bf16, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (uint16_t*)dst, n, seed, std);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

extern "C" int spa_perturb_blocks(void* dst, int64_t nblocks, int block_bytes, uint32_t per_million, uint64_t seed,
                                  void* stream) {
    if (nblocks < 0 || block_bytes <= 0 || per_million > 1000000u || (nblocks > 0 && !dst))
        return spa::fail(SPA_ERR_ARG, "spa_perturb_blocks: bad arguments");
    if (nblocks == 0) return SPA_OK;
    const int64_t blocks = (nblocks + 255) / 256 < 16384 ? (nblocks + 255) / 256 : 16384;
    hipLaunchKernelGGL(k_perturb_blocks, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (uint8_t*)dst,
                       nblocks, block_bytes, per_million, seed);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}
