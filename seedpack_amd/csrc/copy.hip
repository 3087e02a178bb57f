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

// VALU issue-rate probe: every lane advances CHAINS independent chains UNROLL times per loop trip
// (OP 0: v_fma_f32 steps, 1: v_add_f32, 2: integer steps of v_xor_b32 + v_add_u32, 3: FP32 chains
// and integer chains side by side, 4: v_mul_f32 and v_add_f32 chains, 5: v_mul_f32), so a launch retires nblocks x 4 waves x iters x the loop's VALU
// instructions (spa_valu_probe_insts; the loop control is scalar), plus a few per lane around it. The chains' sum is stored
// so that nothing is dropped. The time of a large launch over that count is the chip's VALU issue
// rate for plain (non-packed) 32-bit instructions, the roof of the VALU-bound searches.
constexpr int PROBE_CHAINS = 8, PROBE_UNROLL = 16;
template <int OP>
__global__ __launch_bounds__(256) void k_valu_probe(float* __restrict__ out, int iters, float m, float c) {
    float a[PROBE_CHAINS];
    uint32_t u[PROBE_CHAINS];
    const uint32_t x = __float_as_uint(m), y = __float_as_uint(c);
#pragma unroll
    for (int k = 0; k < PROBE_CHAINS; ++k) {
        a[k] = (float)(threadIdx.x + k) * 1e-3f;
        u[k] = threadIdx.x * 2654435761u + (uint32_t)k;
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < PROBE_UNROLL; ++r) {
#pragma unroll
            for (int k = 0; k < PROBE_CHAINS; ++k) {
                if (OP == 0) a[k] = __builtin_fmaf(a[k], m, c);
                else if (OP == 1) a[k] = a[k] + c;
                else if (OP == 2) u[k] = (u[k] ^ x) + y;                        // integer only
                else if (OP == 4) a[k] = k % 2 ? a[k] * m : a[k] + c;           // v_mul_f32 and v_add_f32 chains
                else if (OP == 5) a[k] = a[k] * m;                              // v_mul_f32 only
                else if (k % 2) a[k] = __builtin_fmaf(a[k], m, c);             // FP32 and integer chains
                else u[k] = (u[k] ^ x) + y;
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < PROBE_CHAINS; ++k) s += a[k] + (float)u[k];
    if (s == 12345.678f) out[blockIdx.x * blockDim.x + threadIdx.x] = s;   // never true for the probe's inputs
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

extern "C" int spa_valu_probe(int op, int64_t nblocks, int iters, float* out, void* stream) {
    if (op < 0 || op > 5 || nblocks <= 0 || nblocks > 0x7fffffff || iters <= 0 || !out)
        return spa::fail(SPA_ERR_ARG, "spa_valu_probe: bad arguments");
    void (*const ks[6])(float*, int, float, float) = {k_valu_probe<0>, k_valu_probe<1>, k_valu_probe<2>,
                                                      k_valu_probe<3>, k_valu_probe<4>, k_valu_probe<5>};
    void (*k)(float*, int, float, float) = ks[op];
    hipLaunchKernelGGL(k, dim3((unsigned)nblocks), dim3(256), 0, (hipStream_t)stream, out, iters, 1.0000001f, 1e-7f);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

extern "C" int64_t spa_valu_probe_insts(int op, int64_t nblocks, int iters) {
    // loop VALU instructions of one launch: waves x trips x steps per trip (the compiled loops: op 0
    // 128 v_fma_f32, op 1 128 v_add_f32, op 2 128 v_xor_b32 + 128 v_add_u32, op 3 64 v_fma_f32 +
    // 64 v_xor_b32 + 64 v_add_u32, op 4 64 v_mul_f32 + 64 v_add_f32, op 5 128 v_mul_f32)
    const int64_t per = op == 2 ? 2 * PROBE_CHAINS * PROBE_UNROLL : op == 3 ? 3 * PROBE_CHAINS * PROBE_UNROLL / 2
                                                                          : PROBE_CHAINS * PROBE_UNROLL;   // 0, 1, 4, 5
    return nblocks * 4 * (int64_t)iters * per;
}
