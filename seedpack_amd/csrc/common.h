// Device primitives shared by every quantizer kernel (gfx950, wave64).
//
// Bit-exactness contract (matches the reference's scalar C build, seedpack/ggml/build.sh:7 and
// seedpack/gpuquant.py:300):
//   * every file is compiled with -ffp-contract=off and without fast-math, so a*b+c is two roundings;
//   * '/' and sqrtf are IEEE correctly rounded (hipcc's default
//     -fhip-fp32-correctly-rounded-divide-sqrt), f32 denormals are kept;
//   * float sums run left to right in index order inside one lane; lanes never share a sum.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spa {

constexpr int WAVE = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// IEEE binary32 -> binary16 with round-to-nearest-even, subnormals kept, overflow to infinity and
// every NaN to the quiet NaN 0x7E00 (sign kept). This is the value set of ggml's software
// conversion (ggml-impl.h:417-443); written here with integer arithmetic only.
__host__ __device__ __forceinline__ uint16_t f32_to_f16(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          // NaN
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         // >= 65520 rounds to inf
    if (a >= 0x38800000u) {                                          // normal half (>= 2^-14)
        uint32_t v = a - 0x38000000u;                                // exponent rebias 127 -> 15
        v += 0x0fffu + ((v >> 13) & 1u);                             // RNE on the 13 dropped bits
        return (uint16_t)(sign | (v >> 13));
    }
    const uint32_t e = a >> 23;
    if (e < 102u) return (uint16_t)sign;                             // below half the smallest subnormal
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const uint32_t s = 126u - e;                                     // 14..24
    const uint32_t q = (m + (1u << (s - 1)) - 1u + ((m >> s) & 1u)) >> s;
    return (uint16_t)(sign | q);
}

// binary16 -> binary32, exact for every input (ggml-impl.h:394-415 value set).
__host__ __device__ __forceinline__ float f16_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t u;
    if (ex == 0x1fu) {
        u = sign | 0x7f800000u | (mant << 13);
    } else if (ex != 0) {
        u = sign | ((ex + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
        u = sign;
    } else {                                                         // subnormal: normalise
        uint32_t e = 113u;
        while (!(mant & 0x400u)) { mant <<= 1; --e; }
        u = sign | (e << 23) | ((mant & 0x3ffu) << 13);
    }
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

// Round to nearest by adding 1.5*2^23 (ggml-quants.c:621-626): ties go to even, valid for
// |f| <= 4194303.
__device__ __forceinline__ int nearest_int(float f) {
    const float v = f + 12582912.f;
    return (int)(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

// C's roundf: half away from zero.
__device__ __forceinline__ float round_half_away(float v) { return roundf(v); }

// Workgroups go to the 8 XCDs in turn (workgroup i to XCD i % 8). xcd_block(i, n) renumbers them so
// that each XCD takes one contiguous range of the n logical blocks: what neighbouring blocks share
// (a tensor's coding tables) then stays in that XCD's L2. A bijection on [0, n).
__device__ __forceinline__ unsigned xcd_block(unsigned i, unsigned n) {
    const unsigned x = i & 7u, k = i >> 3, q = n >> 3, r = n & 7u;
    return x * q + (x < r ? x : r) + k;
}

template <typename T> __device__ __forceinline__ T tmin(T a, T b) { return a < b ? a : b; }
template <typename T> __device__ __forceinline__ T tmax(T a, T b) { return a > b ? a : b; }

// Source element kinds accepted by every quantize entry point.
enum SrcKind { SRC_BF16 = 0, SRC_F16 = 1, SRC_F32 = 2 };

// Loads n consecutive weights starting at element index `e` of a tensor stored as `kind`, widening to
// f32 in registers (the reference widens in a separate pass, gpuquant.py:248-260).
template <int N>
__device__ __forceinline__ void load_weights(const void* __restrict__ src, int kind, int64_t e, float (&x)[N]) {
    if (kind == SRC_BF16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + e);
#pragma unroll
        for (int k = 0; k < N / 8; ++k) {
            const uint4 v = p[k];
            x[8 * k + 0] = bf16_to_f32(v.x & 0xffffu); x[8 * k + 1] = bf16_to_f32(v.x >> 16);
            x[8 * k + 2] = bf16_to_f32(v.y & 0xffffu); x[8 * k + 3] = bf16_to_f32(v.y >> 16);
            x[8 * k + 4] = bf16_to_f32(v.z & 0xffffu); x[8 * k + 5] = bf16_to_f32(v.z >> 16);
            x[8 * k + 6] = bf16_to_f32(v.w & 0xffffu); x[8 * k + 7] = bf16_to_f32(v.w >> 16);
        }
    } else if (kind == SRC_F16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + e);
#pragma unroll
        for (int k = 0; k < N / 8; ++k) {
            const uint4 v = p[k];
            x[8 * k + 0] = f16_to_f32(v.x & 0xffffu); x[8 * k + 1] = f16_to_f32(v.x >> 16);
            x[8 * k + 2] = f16_to_f32(v.y & 0xffffu); x[8 * k + 3] = f16_to_f32(v.y >> 16);
            x[8 * k + 4] = f16_to_f32(v.z & 0xffffu); x[8 * k + 5] = f16_to_f32(v.z >> 16);
            x[8 * k + 6] = f16_to_f32(v.w & 0xffffu); x[8 * k + 7] = f16_to_f32(v.w >> 16);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(src) + e);
#pragma unroll
        for (int k = 0; k < N / 4; ++k) {
            const float4 v = p[k];
            x[4 * k + 0] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
        }
    }
}

// Byte writer into an LDS output tile. Every ggml block size is even, so a block starts on a
// 2-byte boundary; bytes are paired and written as u16.
struct TileOut {
    uint16_t* base;   // LDS, 2-byte aligned start of this block
    __device__ __forceinline__ void put2(int off, uint32_t lo, uint32_t hi) const {
        base[off >> 1] = (uint16_t)((lo & 0xffu) | ((hi & 0xffu) << 8));
    }
    __device__ __forceinline__ void put16(int off, uint32_t v) const { base[off >> 1] = (uint16_t)v; }
};

// Copies `nbytes` (even) from an LDS tile to global memory at dst (2-byte aligned), using every
// thread of the workgroup; dword stores when dst is 4-byte aligned.
__device__ __forceinline__ void store_tile(const uint16_t* __restrict__ lds, uint8_t* __restrict__ dst, int nbytes,
                                           int tid = threadIdx.x) {
    const int nt = blockDim.x;
    if ((reinterpret_cast<uintptr_t>(dst) & 3u) == 0) {
        const int nw = nbytes >> 2;
        const uint32_t* l32 = reinterpret_cast<const uint32_t*>(lds);
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
        for (int i = tid; i < nw; i += nt) d32[i] = l32[i];
        if ((nbytes & 3) && tid == 0) reinterpret_cast<uint16_t*>(dst)[(nbytes >> 1) - 1] = lds[(nbytes >> 1) - 1];
    } else {
        const int nh = nbytes >> 1;
        uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
        for (int i = tid; i < nh; i += nt) d16[i] = lds[i];
    }
}

}  // namespace spa
