// IQ4_NL (32-weight blocks) and IQ4_XS (256-weight super-blocks of 8 x 32): non-linear 4-bit codes
// on the kvalues_iq4nl codebook -- quantize_row_iq4_nl_impl (ggml-quants.c:4938-5047) with ntry = 7,
// as quantize_iq4_nl (:5049-5069) and quantize_iq4_xs (:5087-5105) call it.
//
// Mapping: one lane per 32-weight block. IQ4_NL blocks are independent; IQ4_XS uses groups of 8
// lanes per super-block: the 256-term sum of squares is handed lane to lane in index order (shuffle),
// every lane searches its own block scale, the 8 scales reach every lane of the group by shuffles,
// and each lane requantizes its own block with the shared super-scale. Lane 0 packs the block.
#include "common.h"
#include "launch.h"

namespace spa {
namespace {

constexpr int WG = 256;
constexpr float GROUP_MAX_EPS = 1e-15f;

// kvalues_iq4nl (ggml-common.h:1120)
__constant__ const int8_t KVALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// best_index_int8(16, kvalues_iq4nl, x) -- ggml-quants.c:28-37: binary search, ties to the upper value.
// The four halvings run unconditionally (the reference skips a step only on its [0, 1] range, where
// the step cannot move: x > kvalues[0] there) and carry the values at both ends, so the final
// nearest-of-two test needs no lookup. Levels 1-2 compare against constants; levels 3-4 read the
// codebook from LDS (16 words on distinct banks): no per-lane global loads.
struct Near {
    int idx;     // best_index_int8's result
    float val;   // kvalues_iq4nl[idx]
};
__device__ __forceinline__ Near nearest_iq4(const float* __restrict__ kv, float x) {
    int lo = 0, hi = 15;
    float vlo = (float)KVALUES[0], vhi = (float)KVALUES[15];
    // level 1: mid 7
    const bool c1 = x < (float)KVALUES[7];
    if (c1) { hi = 7; vhi = (float)KVALUES[7]; } else { lo = 7; vlo = (float)KVALUES[7]; }
    // level 2: mid 3 or 11
    const float v2 = c1 ? (float)KVALUES[3] : (float)KVALUES[11];
    const int m2 = c1 ? 3 : 11;
    if (x < v2) { hi = m2; vhi = v2; } else { lo = m2; vlo = v2; }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int mid = (lo + hi) >> 1;
        const float v = kv[mid];
        if (x < v) { hi = mid; vhi = v; } else { lo = mid; vlo = v; }
    }
    Near r = x - vlo < vhi - x ? Near{lo, vlo} : Near{hi, vhi};
    if (x >= (float)KVALUES[15]) r = Near{15, (float)KVALUES[15]};
    if (x <= (float)KVALUES[0]) r = Near{0, (float)KVALUES[0]};
    return r;
}
__device__ __forceinline__ int best_index(const float* __restrict__ kv, float x) { return nearest_iq4(kv, x).idx; }

// scale search of one 32-weight block (ggml-quants.c:4962-5010, ntry = 7); returns the block scale
__device__ __forceinline__ float block_scale(const float* __restrict__ kv, const float (&x)[32], const float (&w)[32]) {
    float amax = 0, max = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float ax = fabsf(x[j]);
        if (ax > amax) { amax = ax; max = x[j]; }
    }
    if (amax < GROUP_MAX_EPS) return 0.f;
    float d = -max / (float)KVALUES[0];
    float id = 1 / d;
    float sumqx = 0, sumq2 = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float q = nearest_iq4(kv, id * x[j]).val;
        sumqx += w[j] * q * x[j];
        sumq2 += w[j] * q * q;
    }
    d = sumq2 > 0 ? sumqx / sumq2 : 0.f;
    float best = d * sumqx;
    for (int itry = -7; itry <= 7; ++itry) {
        id = (float)(itry + KVALUES[0]) / max;
        sumqx = sumq2 = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const float q = nearest_iq4(kv, id * x[j]).val;
            sumqx += w[j] * q * x[j];
            sumq2 += w[j] * q * q;
        }
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            d = sumqx / sumq2;
            best = d * sumqx;
        }
    }
    return d;
}

// IQ4_NL: one lane per 32-weight block (sigma2 over the block itself)
__global__ __launch_bounds__(WG) void k_iq4_nl(const void* __restrict__ src, int kind, uint8_t* __restrict__ dst,
                                               int64_t nblocks, int64_t bpr, const float* __restrict__ imx) {
    __shared__ __align__(16) uint16_t tile[WG * 18 / 2];
    __shared__ float kv[16];
    if (threadIdx.x < 16) kv[threadIdx.x] = (float)KVALUES[threadIdx.x];
    __syncthreads();
    const int64_t b0 = (int64_t)blockIdx.x * WG;
    const int64_t b = b0 + threadIdx.x;
    if (b < nblocks) {
        float x[32];
        load_weights<32>(src, kind, b * 32, x);
        float sigma2 = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) sigma2 += x[j] * x[j];
        sigma2 *= 2.f / 32;
        float w[32];
        if (imx) {
            const float* qw = imx + (b % bpr) * 32;
#pragma unroll
            for (int j = 0; j < 32; ++j) w[j] = qw[j] * sqrtf(sigma2 + x[j] * x[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) w[j] = x[j] * x[j];
        }
        const float d = block_scale(kv, x, w);
        const float id = d != 0.f ? 1 / d : 0.f;
        TileOut o{tile + threadIdx.x * 9};
        o.put16(0, f32_to_f16(d));
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            const uint32_t b0_ = best_index(kv, id * x[j]) | (best_index(kv, id * x[16 + j]) << 4);
            const uint32_t b1_ = best_index(kv, id * x[j + 1]) | (best_index(kv, id * x[17 + j]) << 4);
            o.put2(2 + j, b0_, b1_);
        }
    }
    __syncthreads();
    const int nb = (int)(nblocks - b0 < WG ? nblocks - b0 : WG);
    store_tile(tile, dst + b0 * 18, nb * 18);
}

// IQ4_XS: 8 lanes per super-block
__global__ __launch_bounds__(WG) void k_iq4_xs(const void* __restrict__ src, int kind, uint8_t* __restrict__ dst,
                                               int64_t nsb, int64_t sbpr, const float* __restrict__ imx) {
    constexpr int G = 8, SBW = WG / G;
    __shared__ __align__(16) uint8_t ltile[SBW * 256];
    __shared__ __align__(16) uint16_t otile[SBW * 136 / 2];
    __shared__ int lsc[SBW][G];
    __shared__ float kv[16];
    if (threadIdx.x < 16) kv[threadIdx.x] = (float)KVALUES[threadIdx.x];
    __syncthreads();
    const int lsb = threadIdx.x / G, sub = threadIdx.x % G;
    const int64_t sb0 = (int64_t)blockIdx.x * SBW;
    const int64_t sb = sb0 + lsb;
    const bool active = sb < nsb;
    const int64_t sbc = active ? sb : nsb - 1;
    float x[32];
    load_weights<32>(src, kind, sbc * 256 + sub * 32, x);
    // sum of squares of the super-block, in index order across the group
    float sq[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) sq[j] = x[j] * x[j];
    float sigma2 = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (sub == g) {
#pragma unroll
            for (int j = 0; j < 32; ++j) sigma2 += sq[j];
        }
        sigma2 = __shfl(sigma2, g, G);
    }
    sigma2 *= 2.f / 256;
    float w[32];
    if (imx) {
        const float* qw = imx + (sbc % sbpr) * 256 + sub * 32;
#pragma unroll
        for (int j = 0; j < 32; ++j) w[j] = qw[j] * sqrtf(sigma2 + x[j] * x[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) w[j] = sq[j];
    }
    const float scale = block_scale(kv, x, w);
    // the scale with the largest magnitude (first one on ties), then the super-scale
    float max_scale = 0, amax_scale = 0;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const float s = __shfl(scale, k, G);
        if (fabsf(s) > amax_scale) { amax_scale = fabsf(s); max_scale = s; }
    }
    const float d = -max_scale / 32;
    const float id = d != 0.f ? 1 / d : 0.f;
    int l = nearest_int(id * scale);
    l = tmax(-32, tmin(31, l));
    const float dl = d * (float)l;
    const float idl = dl != 0.f ? 1 / dl : 0.f;
    uint32_t* lt = reinterpret_cast<uint32_t*>(ltile + lsb * 256 + sub * 32);
#pragma unroll
    for (int j = 0; j < 32; j += 4)
        lt[j / 4] = (uint32_t)best_index(kv, idl * x[j]) | ((uint32_t)best_index(kv, idl * x[j + 1]) << 8) |
                    ((uint32_t)best_index(kv, idl * x[j + 2]) << 16) | ((uint32_t)best_index(kv, idl * x[j + 3]) << 24);
    lsc[lsb][sub] = l + 32;
    __syncthreads();
    if (active && sub == 0) {
        // d, scales_h, scales_l[4], qs[128] (ggml-common.h block_iq4_xs; ggml-quants.c:5021-5030, :5040-5046)
        TileOut o{otile + lsb * 68};
        const uint8_t* L = ltile + lsb * 256;
        o.put16(0, f32_to_f16(d));
        uint32_t sh = 0;
        for (int ib = 0; ib < 8; ++ib) sh |= (uint32_t)(lsc[lsb][ib] >> 4) << (2 * ib);
        o.put16(2, sh);
        for (int ib = 0; ib < 8; ib += 4)
            o.put2(4 + ib / 2, (lsc[lsb][ib] & 0xf) | ((lsc[lsb][ib + 1] & 0xf) << 4),
                   (lsc[lsb][ib + 2] & 0xf) | ((lsc[lsb][ib + 3] & 0xf) << 4));
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 16; j += 2)
                o.put2(8 + 16 * i + j, L[32 * i + j] | (L[32 * i + 16 + j] << 4), L[32 * i + j + 1] | (L[32 * i + 17 + j] << 4));
    }
    __syncthreads();
    const int nb = (int)(nsb - sb0 < SBW ? nsb - sb0 : SBW);
    store_tile(otile, dst + sb0 * 136, nb * 136);
}

}  // namespace

int launch_iq4(const QuantArgs& a) {
    if (a.type == 20) {
        const int64_t nb = a.nrows * a.n_per_row / 32;
        hipLaunchKernelGGL(k_iq4_nl, dim3((unsigned)((nb + WG - 1) / WG)), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nb, a.n_per_row / 32, a.imatrix);
    } else if (a.type == 23) {
        const int64_t nsb = a.nrows * a.n_per_row / 256;
        hipLaunchKernelGGL(k_iq4_xs, dim3((unsigned)((nsb + 31) / 32)), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nsb, a.n_per_row / 256, a.imatrix);
    } else {
        return fail(-2, "launch_iq4: type %d", a.type);
    }
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace spa
