// Legacy 32/64-weight block quantizers: Q8_0, Q4_0, Q4_1, Q5_0, Q5_1 (reference and imatrix
// paths) and Q2_0.
//
// Mapping: one lane per block. A workgroup of 256 lanes quantizes 256 consecutive blocks (the
// tensor is one contiguous run of blocks, rows back to back), assembles their bytes in LDS and
// writes them with coalesced dword stores. The imatrix paths need the row's mean square
// (sum_x2 / n_per_row, summed left to right over the whole row, ggml-quants.c:2082-2084); it comes
// from a one-lane-per-row pre-pass.
#include "common.h"
#include "launch.h"
#include "search.h"

namespace spa {
namespace {

constexpr int WG = 256;

// quantize_row_q8_0_ref -- ggml-quants.c:276-299.
struct Q8_0 {
    static constexpr int QK = 32, BS = 34;
    __device__ static void ref(const float (&x)[QK], TileOut o) {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; ++j) amax = tmax(amax, fabsf(x[j]));
        const float d = amax / 127;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        o.put16(0, f32_to_f16(d));
#pragma unroll
        for (int j = 0; j < QK; j += 2) {
            const int q0 = (int)roundf(x[j] * id);
            const int q1 = (int)roundf(x[j + 1] * id);
            o.put2(2 + j, (uint32_t)q0, (uint32_t)q1);
        }
    }
};

// Q4_0: quantize_row_q4_0_ref (ggml-quants.c:113-148), quantize_row_q4_0_impl (:2071-2097).
struct Q4_0 {
    static constexpr int QK = 32, BS = 18;
    __device__ static void ref(const float (&x)[QK], TileOut o) {
        float amax = 0.0f, max = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float v = x[j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        o.put16(0, f32_to_f16(d));
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            uint32_t b[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float x0 = x[j + k] * id;
                const float x1 = x[16 + j + k] * id;
                const int xi0 = tmin(15, (int)(int8_t)(int)(x0 + 8.5f));
                const int xi1 = tmin(15, (int)(int8_t)(int)(x1 + 8.5f));
                b[k] = (uint32_t)(xi0 & 0xff) | (uint32_t)((xi1 << 4) & 0xff);
            }
            o.put2(2 + j, b[0], b[1]);
        }
    }
    __device__ static void impl(const float (&x)[QK], const float (&w)[QK], TileOut o) {
        int L[QK];
        const float d = make_qx_quants<QK, true>(8, x, w, L);
        o.put16(0, f32_to_f16(d));
#pragma unroll
        for (int j = 0; j < 16; j += 2)
            o.put2(2 + j, (uint32_t)(L[j] | (L[j + 16] << 4)), (uint32_t)(L[j + 1] | (L[j + 17] << 4)));
    }
};

// Q4_1: quantize_row_q4_1_ref (ggml-quants.c:150-182), quantize_row_q4_1_impl (:2144-2172).
struct Q4_1 {
    static constexpr int QK = 32, BS = 20;
    __device__ static void ref(const float (&x)[QK], TileOut o) {
        float min = 3.402823466e+38F, max = -3.402823466e+38F;
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float v = x[j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / 15;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        o.put16(0, f32_to_f16(d));
        o.put16(2, f32_to_f16(min));
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            uint32_t b[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float x0 = (x[j + k] - min) * id;
                const float x1 = (x[16 + j + k] - min) * id;
                const int xi0 = tmin(15, (int)(int8_t)(int)(x0 + 0.5f));
                const int xi1 = tmin(15, (int)(int8_t)(int)(x1 + 0.5f));
                b[k] = (uint32_t)(xi0 & 0xff) | (uint32_t)((xi1 << 4) & 0xff);
            }
            o.put2(4 + j, b[0], b[1]);
        }
    }
    __device__ static void impl(const float (&x)[QK], const float (&w)[QK], TileOut o) {
        int L[QK];
        float min;
        const float d = make_qkx3_quants<QK, 15>(x, w, L, min, -0.9f, 0.05f, 36);
        o.put16(0, f32_to_f16(d));
        o.put16(2, f32_to_f16(-min));
#pragma unroll
        for (int j = 0; j < 16; j += 2)
            o.put2(4 + j, (uint32_t)(L[j] | (L[j + 16] << 4)), (uint32_t)(L[j + 1] | (L[j + 17] << 4)));
    }
};

// Writes the Q5 nibbles and high bits of L (values 0..31) at byte offset `qh_off` (qh) and
// `qh_off + 4` (qs) -- ggml-quants.c:211-223.
__device__ __forceinline__ void put_q5(TileOut o, int qh_off, const int (&xi)[32]) {
    uint32_t qh = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        qh |= (((uint32_t)xi[j] & 0x10u) >> 4) << (j + 0);
        qh |= (((uint32_t)xi[j + 16] & 0x10u) >> 4) << (j + 16);
    }
    o.put16(qh_off, qh & 0xffffu);
    o.put16(qh_off + 2, qh >> 16);
#pragma unroll
    for (int j = 0; j < 16; j += 2)
        o.put2(qh_off + 4 + j, (uint32_t)((xi[j] & 0x0f) | ((xi[j + 16] & 0x0f) << 4)),
               (uint32_t)((xi[j + 1] & 0x0f) | ((xi[j + 17] & 0x0f) << 4)));
}

// Q5_0: quantize_row_q5_0_ref (ggml-quants.c:185-226), quantize_row_q5_0_impl (:2189-2225).
struct Q5_0 {
    static constexpr int QK = 32, BS = 22;
    __device__ static void ref(const float (&x)[QK], TileOut o) {
        float amax = 0.0f, max = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float v = x[j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -16;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        o.put16(0, f32_to_f16(d));
        int xi[QK];
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float v = x[j] * id;
            xi[j] = tmin(31, (int)(int8_t)(int)(v + 16.5f)) & 0xff;
        }
        put_q5(o, 2, xi);
    }
    __device__ static void impl(const float (&x)[QK], const float (&w)[QK], TileOut o) {
        int L[QK];
        const float d = make_qx_quants<QK, true>(16, x, w, L);
        o.put16(0, f32_to_f16(d));
        put_q5(o, 2, L);
    }
};

// Q5_1: quantize_row_q5_1_ref (ggml-quants.c:228-271), quantize_row_q5_1_impl (:2243-2278).
struct Q5_1 {
    static constexpr int QK = 32, BS = 24;
    __device__ static void ref(const float (&x)[QK], TileOut o) {
        float min = 3.402823466e+38F, max = -3.402823466e+38F;
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float v = x[j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / 31;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        o.put16(0, f32_to_f16(d));
        o.put16(2, f32_to_f16(min));
        int xi[QK];
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float v = (x[j] - min) * id;
            xi[j] = (int)(uint8_t)(int)(v + 0.5f);
        }
        put_q5(o, 4, xi);
    }
    __device__ static void impl(const float (&x)[QK], const float (&w)[QK], TileOut o) {
        int L[QK];
        float min;
        const float d = make_qkx3_quants<QK, 31>(x, w, L, min, -0.9f, 0.05f, 36);
        o.put16(0, f32_to_f16(d));
        o.put16(2, f32_to_f16(-min));
        put_q5(o, 4, L);
    }
};

// quantize_row_q2_0_ref -- ggml-quants.c:74-110 (the imatrix is ignored, :2114-2127).
struct Q2_0 {
    static constexpr int QK = 64, BS = 18;
    __device__ static void ref(const float (&x)[QK], TileOut o) {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; ++j) {
            const float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        const float d = amax;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        o.put16(0, f32_to_f16(d));
#pragma unroll
        for (int j = 0; j < QK / 4; j += 2) {
            uint32_t b[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                uint32_t byte = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    int q = (int)roundf(x[4 * (j + k) + t] * id) + 1;
                    q = q < 0 ? 0 : (q > 3 ? 3 : q);
                    byte |= (uint32_t)q << (2 * t);
                }
                b[k] = byte;
            }
            o.put2(2 + j, b[0], b[1]);
        }
    }
};

template <class Op, bool IMPL>
__global__ __launch_bounds__(WG) void k_legacy(const void* __restrict__ src, int kind, uint8_t* __restrict__ dst,
                                               int64_t nblocks, int64_t blocks_per_row,
                                               const float* __restrict__ imx, const float* __restrict__ sigma2) {
    __shared__ __align__(16) uint16_t tile[WG * Op::BS / 2];
    const int64_t b0 = (int64_t)blockIdx.x * WG;
    const int64_t b = b0 + threadIdx.x;
    if (b < nblocks) {
        float x[Op::QK];
        load_weights<Op::QK>(src, kind, b * Op::QK, x);
        TileOut o{tile + threadIdx.x * (Op::BS / 2)};
        if constexpr (IMPL) {
            const int64_t row = b / blocks_per_row;
            const int64_t col = (b - row * blocks_per_row) * Op::QK;
            const float s2 = sigma2[row];
            float w[Op::QK];
#pragma unroll
            for (int j = 0; j < Op::QK; ++j) w[j] = imx[col + j] * sqrtf(s2 + x[j] * x[j]);
            Op::impl(x, w, o);
        } else {
            Op::ref(x, o);
        }
    }
    __syncthreads();
    const int nb = (int)(nblocks - b0 < WG ? nblocks - b0 : WG);
    store_tile(tile, dst + b0 * Op::BS, nb * Op::BS);
}

// sigma2[row] = (sum over the row of x*x, left to right) / n_per_row -- ggml-quants.c:2082-2084.
__global__ __launch_bounds__(64) void k_row_mean_sq(const void* __restrict__ src, int kind, int64_t nrows,
                                                    int64_t npr, float* __restrict__ sigma2) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= nrows) return;
    float s = 0;
    for (int64_t j = 0; j < npr; j += 8) {
        float x[8];
        load_weights<8>(src, kind, row * npr + j, x);
#pragma unroll
        for (int k = 0; k < 8; ++k) s += x[k] * x[k];
    }
    sigma2[row] = s / (float)npr;
}

// The same for BF16 rows: 64 rows per workgroup, 64x64 tiles through LDS (read as 16-byte vectors,
// 8 lanes per row: coalesced), the next tile's loads issued before the current tile's sums; each lane
// adds its row's squares in index order. Rows of npr % 64 == 32 end with a half tile read per lane.
constexpr int RS = 64;
__global__ __launch_bounds__(RS) void k_row_mean_sq_bf16(const uint16_t* __restrict__ w, int64_t nrows, int64_t npr,
                                                         float* __restrict__ sigma2) {
    __shared__ uint32_t tile[RS][RS / 2 + 1];
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * RS, row = r0 + lane;
    const int64_t nt = npr / RS;
    float s = 0;
    uint4 v[8];
    auto load = [&](int64_t c0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t r = r0 + (lane >> 3) + 8 * k;
            v[k] = r < nrows ? *reinterpret_cast<const uint4*>(w + r * npr + c0 + (lane & 7) * 8) : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    if (nt) load(0);
    for (int64_t t = 0; t < nt; ++t) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t* d = &tile[(lane >> 3) + 8 * k][(lane & 7) * 4];
            d[0] = v[k].x; d[1] = v[k].y; d[2] = v[k].z; d[3] = v[k].w;
        }
        __syncthreads();
        if (t + 1 < nt) load((t + 1) * RS);
#pragma unroll 8
        for (int j = 0; j < RS / 2; ++j) {
            const uint32_t pr = tile[lane][j];
            const float x0 = bf16_to_f32(pr & 0xffffu), x1 = bf16_to_f32(pr >> 16);
            s += x0 * x0;
            s += x1 * x1;
        }
    }
    if (row >= nrows) return;
    for (int64_t j = nt * RS; j < npr; j += 8) {
        const uint4 u = *reinterpret_cast<const uint4*>(w + row * npr + j);
        const uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float x0 = bf16_to_f32(q[k] & 0xffffu), x1 = bf16_to_f32(q[k] >> 16);
            s += x0 * x0;
            s += x1 * x1;
        }
    }
    sigma2[row] = s / (float)npr;
}

template <class Op>
int run_ref(const QuantArgs& a) {
    const int64_t nblocks = a.nrows * a.n_per_row / Op::QK;
    if (nblocks == 0) return 0;
    const int64_t grid = (nblocks + WG - 1) / WG;
    hipLaunchKernelGGL((k_legacy<Op, false>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                       (uint8_t*)a.dst, nblocks, a.n_per_row / Op::QK, nullptr, nullptr);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

template <class Op>
int run_impl(const QuantArgs& a) {
    const int64_t nblocks = a.nrows * a.n_per_row / Op::QK;
    if (nblocks == 0) return 0;
    float* sigma2 = nullptr;
    SPA_HIP_TRY(hipMallocAsync((void**)&sigma2, (size_t)a.nrows * sizeof(float), a.stream));
    if (a.src_kind == SRC_BF16)
        hipLaunchKernelGGL(k_row_mean_sq_bf16, dim3((unsigned)((a.nrows + RS - 1) / RS)), dim3(RS), 0, a.stream,
                           (const uint16_t*)a.src, a.nrows, a.n_per_row, sigma2);
    else
        hipLaunchKernelGGL(k_row_mean_sq, dim3((unsigned)((a.nrows + 63) / 64)), dim3(64), 0, a.stream, a.src, a.src_kind,
                           a.nrows, a.n_per_row, sigma2);
    const int64_t grid = (nblocks + WG - 1) / WG;
    hipLaunchKernelGGL((k_legacy<Op, true>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                       (uint8_t*)a.dst, nblocks, a.n_per_row / Op::QK, a.imatrix, sigma2);
    const hipError_t le = hipGetLastError();
    SPA_HIP_TRY(hipFreeAsync(sigma2, a.stream));
    if (le != hipSuccess) return fail(-5, "k_legacy launch: %s", hipGetErrorString(le));
    return 0;
}

}  // namespace

int launch_legacy(const QuantArgs& a) {
    const bool w = a.imatrix != nullptr;
    switch (a.type) {
        case 8: return run_ref<Q8_0>(a);                                  // imatrix ignored (:2296-2301)
        case 2: return w ? run_impl<Q4_0>(a) : run_ref<Q4_0>(a);
        case 3: return w ? run_impl<Q4_1>(a) : run_ref<Q4_1>(a);
        case 6: return w ? run_impl<Q5_0>(a) : run_ref<Q5_0>(a);
        case 7: return w ? run_impl<Q5_1>(a) : run_ref<Q5_1>(a);
        case 42: return run_ref<Q2_0>(a);                                 // imatrix ignored (:2114-2127)
        default: return fail(-2, "launch_legacy: type %d is not a legacy type", a.type);
    }
}

}  // namespace spa
