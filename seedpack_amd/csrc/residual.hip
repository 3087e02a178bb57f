// Difference residual on the device (the reference does this on the host after downloading every
// prediction, seedpack/repo3.py:456-510): XOR of a file region with its prediction, a second
// prediction XOR-ed in (r ^ p0 ^ pv), byte-difference counts, and the float-tensor predictions
// (BF16 base -> F32 / F16 / BF16 bytes, repo3.py:673-689).
//
// All byte streams: 16 bytes per lane per step (uint4) when every pointer is 16-byte aligned, bytes
// otherwise; grid-stride loops over a grid sized to the chip (HBM-bound). Counts are 64-bit:
// per-lane counts, summed across the wave by shuffles, one atomic per wave.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace spa {
namespace {

constexpr int WG = 256;

__device__ __forceinline__ uint32_t nz_bytes(uint32_t v) {
    // number of non-zero bytes of v
    const uint32_t t = ((v & 0x7f7f7f7fu) + 0x7f7f7f7fu) | v;
    return __popc(t & 0x80808080u);
}
__device__ __forceinline__ uint32_t nz_bytes(uint4 v) { return nz_bytes(v.x) + nz_bytes(v.y) + nz_bytes(v.z) + nz_bytes(v.w); }
__device__ __forceinline__ uint4 operator^(uint4 a, uint4 b) { return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w); }

__device__ __forceinline__ void add_count(unsigned long long* count, unsigned long long c) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) c += __shfl_xor(c, m, 64);
    if ((threadIdx.x & 63) == 0 && c) atomicAdd(count, c);
}

__global__ void k_zero_u64(unsigned long long* p) { *p = 0; }

// dst = a ^ b (^ c); count += non-zero bytes of dst (count may be null)
template <bool THREE>
__global__ __launch_bounds__(WG) void k_xor_v(uint4* dst, const uint4* a, const uint4* b, const uint4* c, int64_t n16,
                                              unsigned long long* count) {
    unsigned long long cnt = 0;
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n16; i += (int64_t)gridDim.x * WG) {
        uint4 v = a[i] ^ b[i];
        if constexpr (THREE) v = v ^ c[i];
        dst[i] = v;
        cnt += nz_bytes(v);
    }
    if (count) add_count(count, cnt);
}
template <bool THREE>
__global__ __launch_bounds__(WG) void k_xor_b(uint8_t* dst, const uint8_t* a, const uint8_t* b, const uint8_t* c, int64_t n,
                                              unsigned long long* count) {
    unsigned long long cnt = 0;
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n; i += (int64_t)gridDim.x * WG) {
        uint8_t v = a[i] ^ b[i];
        if constexpr (THREE) v ^= c[i];
        dst[i] = v;
        cnt += v != 0;
    }
    if (count) add_count(count, cnt);
}

// count of bytes where a and b differ (b null: non-zero bytes of a)
__global__ __launch_bounds__(WG) void k_diff_v(const uint4* a, const uint4* b, int64_t n16, unsigned long long* count) {
    unsigned long long cnt = 0;
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n16; i += (int64_t)gridDim.x * WG)
        cnt += nz_bytes(b ? (a[i] ^ b[i]) : a[i]);
    add_count(count, cnt);
}
__global__ __launch_bounds__(WG) void k_diff_b(const uint8_t* a, const uint8_t* b, int64_t n, unsigned long long* count) {
    unsigned long long cnt = 0;
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n; i += (int64_t)gridDim.x * WG)
        cnt += (b ? (a[i] ^ b[i]) : a[i]) != 0;
    add_count(count, cnt);
}

// count of non-zero bytes a[0], a[stride], a[2 stride], ... below n
__global__ __launch_bounds__(WG) void k_count_every(const uint8_t* a, int64_t n, int64_t stride, unsigned long long* count) {
    unsigned long long cnt = 0;
    const int64_t m = (n + stride - 1) / stride;
    for (int64_t k = (int64_t)blockIdx.x * WG + threadIdx.x; k < m; k += (int64_t)gridDim.x * WG)
        cnt += a[k * stride] != 0;
    add_count(count, cnt);
}

// float prediction: source weights (BF16 bits, F16, F32) -> bytes of the file's float type:
// F32 as is, F16 by round-to-nearest-even (the astype of repo3.py:685), BF16 by
// (u + 0x7FFF + ((u >> 16) & 1)) >> 16. A NaN goes to F16 as numpy's conversion (the reference's
// --cpu path) takes it: sign, all-ones exponent and the top 10 payload bits, 0x7C01 when those are 0.
__device__ __forceinline__ uint16_t pred_f16(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        const uint32_t m = (u >> 13) & 0x3ffu;
        return (uint16_t)(((u >> 16) & 0x8000u) | 0x7c00u | (m ? m : 1u));
    }
    return f32_to_f16(x);
}
__device__ __forceinline__ float src_value(const void* src, int kind, int64_t i) {
    if (kind == SRC_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(src)[i]);
    if (kind == SRC_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(src)[i]);
    return reinterpret_cast<const float*>(src)[i];
}
__global__ __launch_bounds__(WG) void k_float_pred(const void* src, int kind, int dst_type, int64_t n, uint8_t* dst) {
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n; i += (int64_t)gridDim.x * WG) {
        const float x = src_value(src, kind, i);
        if (dst_type == 0) {
            reinterpret_cast<float*>(dst)[i] = x;
        } else if (dst_type == 1) {
            reinterpret_cast<uint16_t*>(dst)[i] = pred_f16(x);
        } else {
            const uint32_t u = __float_as_uint(x);
            reinterpret_cast<uint16_t*>(dst)[i] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
        }
    }
}

unsigned grid_for(int64_t work) {
    const int64_t g = (work + WG - 1) / WG;
    return (unsigned)(g < 1 ? 1 : (g > 8192 ? 8192 : g));
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int xor_impl(void* dst, const void* a, const void* b, const void* c, size_t n, unsigned long long* count, hipStream_t st) {
    if (!dst || !a || !b) return fail(SPA_ERR_ARG, "spa_xor: null pointer");
    if (count) hipLaunchKernelGGL(k_zero_u64, dim3(1), dim3(1), 0, st, count);
    if (n) {
        if (aligned16(dst) && aligned16(a) && aligned16(b) && aligned16(c) && n % 16 == 0) {
            const int64_t n16 = (int64_t)(n / 16);
            if (c)
                hipLaunchKernelGGL(k_xor_v<true>, dim3(grid_for(n16)), dim3(WG), 0, st, (uint4*)dst, (const uint4*)a,
                                   (const uint4*)b, (const uint4*)c, n16, count);
            else
                hipLaunchKernelGGL(k_xor_v<false>, dim3(grid_for(n16)), dim3(WG), 0, st, (uint4*)dst, (const uint4*)a,
                                   (const uint4*)b, (const uint4*)nullptr, n16, count);
        } else {
            if (c)
                hipLaunchKernelGGL(k_xor_b<true>, dim3(grid_for((int64_t)n / 16)), dim3(WG), 0, st, (uint8_t*)dst,
                                   (const uint8_t*)a, (const uint8_t*)b, (const uint8_t*)c, (int64_t)n, count);
            else
                hipLaunchKernelGGL(k_xor_b<false>, dim3(grid_for((int64_t)n / 16)), dim3(WG), 0, st, (uint8_t*)dst,
                                   (const uint8_t*)a, (const uint8_t*)b, (const uint8_t*)nullptr, (int64_t)n, count);
        }
    }
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // namespace
}  // namespace spa

using spa::fail;

extern "C" {

int spa_xor(void* dst, const void* a, const void* b, size_t n, unsigned long long* nonzero, void* stream) {
    return spa::xor_impl(dst, a, b, nullptr, n, nonzero, (hipStream_t)stream);
}

int spa_xor3(void* dst, const void* a, const void* b, const void* c, size_t n, unsigned long long* nonzero, void* stream) {
    if (!c) return fail(SPA_ERR_ARG, "spa_xor3: null pointer");
    return spa::xor_impl(dst, a, b, c, n, nonzero, (hipStream_t)stream);
}

int spa_diff_count(const void* a, const void* b, size_t n, unsigned long long* count, void* stream) {
    if (!a || !count) return fail(SPA_ERR_ARG, "spa_diff_count: null pointer");
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(spa::k_zero_u64, dim3(1), dim3(1), 0, st, count);
    if (n) {
        if (spa::aligned16(a) && spa::aligned16(b) && n % 16 == 0)
            hipLaunchKernelGGL(spa::k_diff_v, dim3(spa::grid_for((int64_t)n / 16)), dim3(spa::WG), 0, st, (const uint4*)a,
                               (const uint4*)b, (int64_t)(n / 16), count);
        else
            hipLaunchKernelGGL(spa::k_diff_b, dim3(spa::grid_for((int64_t)n / 16)), dim3(spa::WG), 0, st, (const uint8_t*)a,
                               (const uint8_t*)b, (int64_t)n, count);
    }
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_count_every(const void* a, size_t n, size_t stride, unsigned long long* count, void* stream) {
    if (!count || (n && !a)) return fail(SPA_ERR_ARG, "spa_count_every: null pointer");
    if (!stride) return fail(SPA_ERR_ARG, "spa_count_every: stride 0");
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(spa::k_zero_u64, dim3(1), dim3(1), 0, st, count);
    if (n) {
        const int64_t m = (int64_t)((n + stride - 1) / stride);
        hipLaunchKernelGGL(spa::k_count_every, dim3(spa::grid_for(m)), dim3(spa::WG), 0, st, (const uint8_t*)a, (int64_t)n,
                           (int64_t)stride, count);
    }
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_float_pred(const void* src, int src_kind, int64_t n, int dst_type, void* dst, void* stream) {
    if (src_kind < SPA_SRC_BF16 || src_kind > SPA_SRC_F32) return fail(SPA_ERR_ARG, "spa_float_pred: bad src_kind %d", src_kind);
    if (dst_type != 0 && dst_type != 1 && dst_type != 30)
        return fail(SPA_ERR_TYPE, "spa_float_pred: file type %d is not F32 (0), F16 (1) or BF16 (30)", dst_type);
    if (n < 0) return fail(SPA_ERR_ARG, "spa_float_pred: negative count");
    if (n == 0) return SPA_OK;
    if (!src || !dst) return fail(SPA_ERR_ARG, "spa_float_pred: null pointer");
    hipLaunchKernelGGL(spa::k_float_pred, dim3(spa::grid_for(n / 4)), dim3(spa::WG), 0, (hipStream_t)stream, src, src_kind,
                       dst_type == 30 ? 2 : dst_type, n, (uint8_t*)dst);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
