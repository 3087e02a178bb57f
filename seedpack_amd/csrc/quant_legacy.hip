// Legacy 32/64-weight block quantizers: Q8_0, Q4_0, Q4_1, Q5_0, Q5_1 (reference and imatrix
// paths) and Q2_0.
//
// Mapping: one lane per block. A workgroup of 256 lanes quantizes 256 consecutive blocks (the
// tensor is one contiguous run of blocks, rows back to back), assembles their bytes in LDS and
// writes them with coalesced dword stores. The imatrix paths need the row's mean square
// (sum_x2 / n_per_row, summed left to right over the whole row, ggml-quants.c:2082-2084). Given
// scratch, a first launch computes it for every row (k_row_ms: 32 serial chains per workgroup fed
// from LDS) and the quantizer reads it; without scratch each quantizer workgroup walks the rows
// its blocks belong to in one lane per row first (2.4-4.3x slower: those chains are serial and
// their loads are not coalesced).
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

// (sum over row `row` of x*x, added left to right) / n_per_row -- ggml-quants.c:2082-2084. One lane
// walks the whole row; the next 32 weights are requested before the current 32 are added, so the
// dependent adds, not the loads, set the pace.
__device__ float row_mean_sq(const void* __restrict__ src, int kind, int64_t row, int64_t npr) {
    float s = 0;
    float x[32], nx[32];
    load_weights<32>(src, kind, row * npr, nx);
    for (int64_t j = 0; j < npr; j += 32) {
#pragma unroll
        for (int k = 0; k < 32; ++k) x[k] = nx[k];
        if (j + 32 < npr) load_weights<32>(src, kind, row * npr + j + 32, nx);
#pragma unroll
        for (int k = 0; k < 32; ++k) s += x[k] * x[k];
    }
    return s / (float)npr;
}

// The same mean squares for rows r0 .. r0 + 31, one lane of the first wave per row: the adds of a
// row are one serial chain in the reference's order. The workgroup's 256 lanes stage the 32 rows in
// LDS, 128 columns (a tile) at a time, with coalesced 16-byte loads issued MS_DEPTH tiles ahead
// into registers, so HBM latency hides behind the first wave's adds. Every lane issues the same
// loads in every step (addresses past the rows or the row end are clamped and their values never
// stored), so the waits before the LDS stores count exactly the loads still in flight. The staging
// lanes store the squares x*x (rounded to float, as the reference's sum_x2 += x*x rounds them), so
// the first wave's stream is one 16-byte LDS read per four adds. Rows are 132 floats apart: 16-byte
// aligned, and eight lanes reading 16 bytes each cover the 32 banks once.
constexpr int MS_ROWS = 32, MS_COLS = 128, MS_LD = MS_COLS + 4, MS_DEPTH = 4;
template <int KIND>
__global__ __launch_bounds__(WG) void k_row_ms(const void* __restrict__ src, int64_t nrows, int64_t npr,
                                               float* __restrict__ out) {
    __shared__ __align__(16) float tile[2][MS_ROWS * MS_LD];
    constexpr int PPR = MS_COLS / 8, NP = MS_ROWS * PPR / WG;            // pieces of 8 weights
    const int64_t r0 = (int64_t)blockIdx.x * MS_ROWS;
    const int nr = (int)(nrows - r0 < MS_ROWS ? nrows - r0 : MS_ROWS);
    const int nch = (int)((npr + MS_COLS - 1) / MS_COLS);
    float v[MS_DEPTH][NP][8];
    auto load = [&](float (&w)[NP][8], int k) {
        const int64_t c0 = (int64_t)k * MS_COLS;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int q = (int)threadIdx.x + p * WG, r = q / PPR, c = (q % PPR) * 8;
            const int64_t rr = r < nr ? r : nr - 1, cc = c0 + c < npr ? c0 + c : npr - 8;
            load_weights<8>(src, KIND, (r0 + rr) * npr + cc, w[p]);
        }
    };
    auto put = [&](float* t, const float (&w)[NP][8], int k) {
        const int64_t c0 = (int64_t)k * MS_COLS;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int q = (int)threadIdx.x + p * WG, r = q / PPR, c = (q % PPR) * 8;
            if (r < nr && c0 + c < npr) {
#pragma unroll
                for (int e = 0; e < 8; ++e) t[r * MS_LD + c + e] = w[p][e] * w[p][e];
            }
        }
    };
    const int lane = (int)threadIdx.x;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < MS_DEPTH; ++i) load(v[i], i);
    put(tile[0], v[0], 0);
    __syncthreads();
    // steps past the last tile (up to a multiple of MS_DEPTH) add nothing and store nothing
    for (int k0 = 0; k0 < nch; k0 += MS_DEPTH) {
#pragma unroll
        for (int i = 0; i < MS_DEPTH; ++i) {          // tile k = k0 + i is in LDS, its slot v[i] is free
            const int k = k0 + i;
            load(v[i], k + MS_DEPTH);
            const int64_t c0 = (int64_t)k * MS_COLS;
            const int n = c0 >= npr ? 0 : (int)(npr - c0 < MS_COLS ? npr - c0 : MS_COLS);
            if (lane < nr) {
                const float* t = tile[k & 1] + lane * MS_LD;
                if (n == MS_COLS) {                   // whole tile: 32 squares read ahead of their adds
                    const float4* t4 = reinterpret_cast<const float4*>(t);
#pragma unroll
                    for (int j0 = 0; j0 < MS_COLS / 4; j0 += 8) {
                        float4 a[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) a[j] = t4[j0 + j];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            s += a[j].x;
                            s += a[j].y;
                            s += a[j].z;
                            s += a[j].w;
                        }
                    }
                } else {
                    for (int j = 0; j < n; ++j) s += t[j];
                }
            }
            // the other buffer was last read before the previous barrier
            put(tile[(k + 1) & 1], v[(i + 1) % MS_DEPTH], k + 1);
            __syncthreads();
        }
    }
    if (lane < nr) out[r0 + lane] = s / (float)npr;
}

// One lane per block, 256 blocks per workgroup. MODE 0: no imatrix. MODE 1: imatrix, the
// workgroup first computes the mean square of every row its blocks touch (one lane per row, at
// most 256 rows) when no scratch holds them. MODE 2: imatrix, the mean squares read from `s2r`
// (k_row_ms).
template <class Op, int MODE>
__global__ __launch_bounds__(WG) void k_legacy(const void* __restrict__ src, int kind, uint8_t* __restrict__ dst,
                                               int64_t nblocks, int64_t blocks_per_row,
                                               const float* __restrict__ imx, const float* __restrict__ s2r) {
    __shared__ __align__(16) uint16_t tile[WG * Op::BS / 2];
    __shared__ float s2_rows[MODE == 1 ? WG : 1];
    const int64_t b0 = (int64_t)blockIdx.x * WG;
    const int64_t b = b0 + threadIdx.x;
    const int nb = (int)(nblocks - b0 < WG ? nblocks - b0 : WG);
    const int64_t row_lo = b0 / blocks_per_row;
    if constexpr (MODE == 1) {
        // rows row_lo .. (b0 + nb - 1) / blocks_per_row: at most WG of them (blocks_per_row >= 1)
        const int nrow = (int)((b0 + nb - 1) / blocks_per_row - row_lo + 1);
        if ((int)threadIdx.x < nrow)
            s2_rows[threadIdx.x] = row_mean_sq(src, kind, row_lo + threadIdx.x, blocks_per_row * Op::QK);
        __syncthreads();
    }
    if (b < nblocks) {
        float x[Op::QK];
        load_weights<Op::QK>(src, kind, b * Op::QK, x);
        TileOut o{tile + threadIdx.x * (Op::BS / 2)};
        if constexpr (MODE != 0) {
            const int64_t row = b / blocks_per_row;
            const int64_t col = (b - row * blocks_per_row) * Op::QK;
            const float s2 = MODE == 1 ? s2_rows[row - row_lo] : s2r[row];
            float w[Op::QK];
#pragma unroll
            for (int j = 0; j < Op::QK; ++j) w[j] = imx[col + j] * sqrtf(s2 + x[j] * x[j]);
            Op::impl(x, w, o);
        } else {
            Op::ref(x, o);
        }
    }
    __syncthreads();
    store_tile(tile, dst + b0 * Op::BS, nb * Op::BS);
}

template <class Op, bool IMPL>
int run(const QuantArgs& a) {
    const int64_t nblocks = a.nrows * a.n_per_row / Op::QK;
    if (nblocks == 0) return 0;
    const int64_t grid = (nblocks + WG - 1) / WG;
    const int64_t bpr = a.n_per_row / Op::QK;
    if constexpr (!IMPL) {
        hipLaunchKernelGGL((k_legacy<Op, 0>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nblocks, bpr, nullptr, nullptr);
    } else if (a.work) {
        const dim3 g((unsigned)((a.nrows + MS_ROWS - 1) / MS_ROWS));
        if (a.src_kind == SRC_BF16)
            hipLaunchKernelGGL(k_row_ms<SRC_BF16>, g, dim3(WG), 0, a.stream, a.src, a.nrows, a.n_per_row, a.work);
        else if (a.src_kind == SRC_F16)
            hipLaunchKernelGGL(k_row_ms<SRC_F16>, g, dim3(WG), 0, a.stream, a.src, a.nrows, a.n_per_row, a.work);
        else
            hipLaunchKernelGGL(k_row_ms<SRC_F32>, g, dim3(WG), 0, a.stream, a.src, a.nrows, a.n_per_row, a.work);
        SPA_HIP_TRY(hipGetLastError());
        hipLaunchKernelGGL((k_legacy<Op, 2>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nblocks, bpr, a.imatrix, a.work);
    } else {
        hipLaunchKernelGGL((k_legacy<Op, 1>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nblocks, bpr, a.imatrix, nullptr);
    }
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

int64_t quantize_work_bytes(int type, int64_t nrows, bool imatrix) {
    const bool rows = imatrix && (type == 2 || type == 3 || type == 6 || type == 7);
    return rows && nrows > 0 ? (nrows * (int64_t)sizeof(float) + 255) / 256 * 256 : 0;
}

int launch_legacy(const QuantArgs& a) {
    const bool w = a.imatrix != nullptr;
    switch (a.type) {
        case 8: return run<Q8_0, false>(a);                               // imatrix ignored (:2296-2301)
        case 2: return w ? run<Q4_0, true>(a) : run<Q4_0, false>(a);
        case 3: return w ? run<Q4_1, true>(a) : run<Q4_1, false>(a);
        case 6: return w ? run<Q5_0, true>(a) : run<Q5_0, false>(a);
        case 7: return w ? run<Q5_1, true>(a) : run<Q5_1, false>(a);
        case 42: return run<Q2_0, false>(a);                              // imatrix ignored (:2114-2127)
        default: return fail(-2, "launch_legacy: type %d is not a legacy type", a.type);
    }
}

}  // namespace spa
