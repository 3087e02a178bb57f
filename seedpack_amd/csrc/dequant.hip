// Dequantizers: quantized blocks -> float32, llama.cpp's dequantize_row_<type> for the 20 types of
// the path (ggml-quants.c:439-568, :961-990, :1306-1345, :1530-1550, :1732-1757, :1940-1968,
// :2489-2764). They replace the reference's k_dq_<type> launches (gpuquant.py:214-219) behind
// GPUQuant.dequantize (gpuquant.py:413-421).
//
// Mapping: one lane per 4 consecutive outputs of a row-major run of blocks (every type's block
// holds a multiple of 4 weights), written as one 16-byte store; the lane reads its block's header
// and codes from L1/L2 (neighbouring lanes share the block). HBM-bound: 4 bytes written per weight.
// Each output is the C code's expression for that element, with the same operand order (float
// products left to right, integer parts converted as the C promotions do), so the results are
// bit-identical.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "iq_tables.h"
#include "launch.h"

namespace spa {
namespace {

__constant__ const int8_t KV_IQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
// coordinate values of the lattice grids by level (the bytes of ggml-common.h's iq2*_grid,
// iq3xxs_grid; iq3s_grid stores 2l+1 itself, iq1s_grid l-1)
__constant__ const float IQ2_VAL[3] = {8.f, 25.f, 43.f};
__constant__ const float IQ3XXS_VAL[8] = {4.f, 12.f, 20.f, 28.f, 36.f, 44.f, 52.f, 62.f};
constexpr float IQ1S_DELTA = 0.125f;

__device__ __forceinline__ uint32_t u8(const uint8_t* b, int o) { return b[o]; }
__device__ __forceinline__ uint32_t u16(const uint8_t* b, int o) { return (uint32_t)b[o] | ((uint32_t)b[o + 1] << 8); }
__device__ __forceinline__ uint32_t u32(const uint8_t* b, int o) { return u16(b, o) | (u16(b, o + 2) << 16); }
__device__ __forceinline__ float h(const uint8_t* b, int o) { return f16_to_f32(u16(b, o)); }
// ksigns_iq2xs[i] (ggml-common.h:513): the 7 sign bits and an 8th that makes the count even
__device__ __forceinline__ uint32_t ksigns(uint32_t i) { return i | ((uint32_t)(__popc(i) & 1) << 7); }
// the grid coordinate k of point g as its level (the device tables hold 2l+1 per coordinate)
__device__ __forceinline__ int glevel(const uint8_t* grid, int D, int g, int k) { return ((int)grid[g * D + k] - 1) >> 1; }

struct DQ {
    const uint8_t* grid;    // the type's lattice (IQ types), D coordinates per point
};

template <int T>
__device__ __forceinline__ float dq(const uint8_t* b, int e, const DQ& t);

template <> __device__ __forceinline__ float dq<8>(const uint8_t* b, int e, const DQ&) {     // Q8_0 (:553-567)
    return (float)(int8_t)b[2 + e] * h(b, 0);
}
template <> __device__ __forceinline__ float dq<2>(const uint8_t* b, int e, const DQ&) {     // Q4_0 (:459-477)
    const uint32_t q = e < 16 ? (u8(b, 2 + e) & 0x0F) : (u8(b, 2 + e - 16) >> 4);
    return (float)((int)q - 8) * h(b, 0);
}
template <> __device__ __forceinline__ float dq<3>(const uint8_t* b, int e, const DQ&) {     // Q4_1 (:479-498)
    const uint32_t q = e < 16 ? (u8(b, 4 + e) & 0x0F) : (u8(b, 4 + e - 16) >> 4);
    return (float)(int)q * h(b, 0) + h(b, 2);
}
template <> __device__ __forceinline__ float dq<6>(const uint8_t* b, int e, const DQ&) {     // Q5_0 (:500-524)
    const uint32_t qh = u32(b, 2);
    const int j = e & 15;
    const uint32_t xh = e < 16 ? (((qh >> j) << 4) & 0x10) : ((qh >> (j + 12)) & 0x10);
    const uint32_t lo = e < 16 ? (u8(b, 6 + j) & 0x0F) : (u8(b, 6 + j) >> 4);
    return (float)((int)(lo | xh) - 16) * h(b, 0);
}
template <> __device__ __forceinline__ float dq<7>(const uint8_t* b, int e, const DQ&) {     // Q5_1 (:526-551)
    const uint32_t qh = u32(b, 4);
    const int j = e & 15;
    const uint32_t xh = e < 16 ? (((qh >> j) << 4) & 0x10) : ((qh >> (j + 12)) & 0x10);
    const uint32_t lo = e < 16 ? (u8(b, 8 + j) & 0x0F) : (u8(b, 8 + j) >> 4);
    return (float)(int)(lo | xh) * h(b, 0) + h(b, 2);
}
template <> __device__ __forceinline__ float dq<42>(const uint8_t* b, int e, const DQ&) {    // Q2_0 (:439-457)
    const uint32_t q = (u8(b, 2 + e / 4) >> ((e % 4) * 2)) & 3;
    return (float)((int)q - 1) * h(b, 0);
}
template <> __device__ __forceinline__ float dq<10>(const uint8_t* b, int e, const DQ&) {    // Q2_K (:961-990)
    const int n = e >> 7, r = e & 127, j = r >> 5, part = (r >> 4) & 1, l = r & 15;
    const uint32_t sc = u8(b, n * 8 + 2 * j + part);
    const float dl = h(b, 80) * (float)(int)(sc & 0xF), ml = h(b, 82) * (float)(int)(sc >> 4);
    const uint32_t q = (u8(b, 16 + n * 32 + part * 16 + l) >> (2 * j)) & 3;
    return dl * (float)(int)q - ml;
}
template <> __device__ __forceinline__ float dq<11>(const uint8_t* b, int e, const DQ&) {    // Q3_K (:1306-1345)
    const int n = e >> 7, r = e & 127, j = r >> 5, part = (r >> 4) & 1, l = r & 15;
    const int is = n * 8 + 2 * j + part;
    const uint32_t lo = is < 8 ? (u8(b, 96 + is) & 0xF) : (u8(b, 96 + is - 8) >> 4);
    const int sc = (int)(lo | (((u8(b, 96 + 8 + is % 4) >> (2 * (is / 4))) & 3) << 4)) - 32;
    const float dl = h(b, 108) * (float)sc;
    const int q = (int)((u8(b, 32 + n * 32 + part * 16 + l) >> (2 * j)) & 3);
    const bool hb = (u8(b, part * 16 + l) >> (n * 4 + j)) & 1;
    return dl * (float)(q - (hb ? 0 : 4));
}
__device__ __forceinline__ void k4_scale_min(const uint8_t* sc, int j, uint32_t& d, uint32_t& m) {   // get_scale_min_k4 (:880-887)
    if (j < 4) {
        d = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        d = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}
template <> __device__ __forceinline__ float dq<12>(const uint8_t* b, int e, const DQ&) {    // Q4_K (:1530-1550)
    const int c = e >> 6, r = e & 63, l = r & 31;
    uint32_t sc, m;
    k4_scale_min(b + 4, 2 * c + (r >> 5), sc, m);
    const float d1 = h(b, 0) * (float)sc, m1 = h(b, 2) * (float)m;
    const uint32_t q = u8(b, 16 + c * 32 + l);
    return d1 * (float)(int)(r < 32 ? (q & 0xF) : (q >> 4)) - m1;
}
template <> __device__ __forceinline__ float dq<13>(const uint8_t* b, int e, const DQ&) {    // Q5_K (:1732-1757)
    const int c = e >> 6, r = e & 63, l = r & 31;
    uint32_t sc, m;
    k4_scale_min(b + 4, 2 * c + (r >> 5), sc, m);
    const float d1 = h(b, 0) * (float)sc, m1 = h(b, 2) * (float)m;
    const uint32_t ql = u8(b, 48 + c * 32 + l), qh = u8(b, 16 + l);
    const uint32_t hbit = r < 32 ? (1u << (2 * c)) : (2u << (2 * c));
    const int v = (int)(r < 32 ? (ql & 0xF) : (ql >> 4)) + ((qh & hbit) ? 16 : 0);
    return d1 * (float)v - m1;
}
template <> __device__ __forceinline__ float dq<14>(const uint8_t* b, int e, const DQ&) {    // Q6_K (:1940-1968)
    const int n = e >> 7, r = e & 127, qd = r >> 5, l = r & 31, is = l / 16;
    const uint32_t ql = u8(b, n * 64 + l + (qd & 1) * 32), qh = u8(b, 128 + n * 32 + l);
    const uint32_t lo = qd < 2 ? (ql & 0xF) : (ql >> 4);
    const int q = (int)(int8_t)(uint8_t)(lo | (((qh >> (2 * qd)) & 3) << 4)) - 32;
    const int sc = (int8_t)b[192 + n * 8 + is + 2 * qd];
    return h(b, 208) * (float)sc * (float)q;
}
template <> __device__ __forceinline__ float dq<16>(const uint8_t* b, int e, const DQ& t) {  // IQ2_XXS (:2489-2513)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t a1 = u32(b, 2 + 8 * ib + 4);
    const float db = h(b, 0) * (0.5f + (float)(a1 >> 28)) * 0.25f;
    const int g = (int)u8(b, 2 + 8 * ib + l);
    const uint32_t s = ksigns((a1 >> (7 * l)) & 127);
    return db * IQ2_VAL[glevel(t.grid, 8, g, j)] * ((s >> j) & 1 ? -1.f : 1.f);
}
template <> __device__ __forceinline__ float dq<17>(const uint8_t* b, int e, const DQ& t) {  // IQ2_XS (:2517-2540)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t sc = u8(b, 66 + ib);
    const float db = h(b, 0) * (0.5f + (float)((l < 2 ? sc : sc >> 4) & 0xf)) * 0.25f;
    const uint32_t q = u16(b, 2 + 2 * (4 * ib + l));
    const uint32_t s = ksigns(q >> 9);
    return db * IQ2_VAL[glevel(t.grid, 8, (int)(q & 511), j)] * ((s >> j) & 1 ? -1.f : 1.f);
}
template <> __device__ __forceinline__ float dq<22>(const uint8_t* b, int e, const DQ& t) {  // IQ2_S (:2544-2572)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t sc = u8(b, 74 + ib);
    const float dl = h(b, 0) * (0.5f + (float)((l < 2 ? sc : sc >> 4) & 0xf)) * 0.25f;
    const int g = (int)(u8(b, 2 + 4 * ib + l) | ((u8(b, 66 + ib) << (8 - 2 * l)) & 0x300));
    const uint32_t s = u8(b, 2 + 32 + 4 * ib + l);
    return dl * IQ2_VAL[glevel(t.grid, 8, g, j)] * ((s >> j) & 1 ? -1.f : 1.f);
}
template <> __device__ __forceinline__ float dq<18>(const uint8_t* b, int e, const DQ& t) {  // IQ3_XXS (:2576-2604)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t a = u32(b, 2 + 64 + 4 * ib);
    const float db = h(b, 0) * (0.5f + (float)(a >> 28)) * 0.5f;
    const uint32_t s = ksigns((a >> (7 * l)) & 127);
    const int g = (int)u8(b, 2 + 8 * ib + 2 * l + (j >> 2));
    return db * IQ3XXS_VAL[glevel(t.grid, 4, g, j & 3)] * ((s >> j) & 1 ? -1.f : 1.f);
}
template <> __device__ __forceinline__ float dq<21>(const uint8_t* b, int e, const DQ& t) {  // IQ3_S (:2608-2647)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t sc = u8(b, 106 + ib / 2);
    const float db = h(b, 0) * (float)(1 + 2 * (int)((ib & 1) ? (sc >> 4) : (sc & 0xf)));
    const uint32_t qh = u8(b, 66 + ib);
    const int g = j < 4 ? (int)(u8(b, 2 + 8 * ib + 2 * l) | ((qh << (8 - 2 * l)) & 256))
                        : (int)(u8(b, 2 + 8 * ib + 2 * l + 1) | ((qh << (7 - 2 * l)) & 256));
    const uint32_t s = u8(b, 74 + 4 * ib + l);
    return db * (float)(2 * glevel(t.grid, 4, g, j & 3) + 1) * ((s >> j) & 1 ? -1.f : 1.f);
}
template <> __device__ __forceinline__ float dq<19>(const uint8_t* b, int e, const DQ& t) {  // IQ1_S (:2651-2674)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t qh = u16(b, 34 + 2 * ib);
    const float dl = h(b, 0) * (float)(2 * (int)((qh >> 12) & 7) + 1);
    const float delta = (qh & 0x8000) ? -IQ1S_DELTA : IQ1S_DELTA;
    const int g = (int)(u8(b, 2 + 4 * ib + l) | (((qh >> (3 * l)) & 7) << 8));
    return dl * ((float)(glevel(t.grid, 8, g, j) - 1) + delta);
}
template <> __device__ __forceinline__ float dq<29>(const uint8_t* b, int e, const DQ& t) {  // IQ1_M (:2676-2724)
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint32_t s0 = u16(b, 48), s1 = u16(b, 50), s2 = u16(b, 52), s3 = u16(b, 54);
    const uint32_t sf = (s0 >> 12) | ((s1 >> 8) & 0x00f0) | ((s2 >> 4) & 0x0f00) | (s3 & 0xf000);
    const float d = f16_to_f32(sf);
    const uint32_t sc = u16(b, 48 + 2 * (ib / 2));
    const int sh = 6 * (ib % 2) + (l < 2 ? 0 : 3);
    const float dl = d * (float)(2 * (int)((sc >> sh) & 0x7) + 1);
    const uint32_t qh = u8(b, 32 + 2 * ib + (l >> 1));
    const int g = (int)(u8(b, 4 * ib + l) | ((qh << ((l & 1) ? 4 : 8)) & 0x700));
    const float delta = (qh & ((l & 1) ? 0x80 : 0x08)) ? -IQ1S_DELTA : IQ1S_DELTA;
    return dl * ((float)(glevel(t.grid, 8, g, j) - 1) + delta);
}
template <> __device__ __forceinline__ float dq<20>(const uint8_t* b, int e, const DQ&) {    // IQ4_NL (:2726-2742)
    const uint32_t q = e < 16 ? (u8(b, 2 + e) & 0xf) : (u8(b, 2 + e - 16) >> 4);
    return h(b, 0) * (float)KV_IQ4NL[q];
}
template <> __device__ __forceinline__ float dq<23>(const uint8_t* b, int e, const DQ&) {    // IQ4_XS (:2744-2764)
    const int ib = e >> 5, r = e & 31;
    const int ls = (int)(((u8(b, 4 + ib / 2) >> (4 * (ib % 2))) & 0xf) | (((u16(b, 2) >> (2 * ib)) & 3) << 4));
    const float dl = h(b, 0) * (float)(ls - 32);
    const uint32_t q = u8(b, 8 + 16 * ib + (r & 15));
    return dl * (float)KV_IQ4NL[r < 16 ? (q & 0xf) : (q >> 4)];
}

template <int T, int QK, int BS>
__global__ __launch_bounds__(256) void k_dq(const uint8_t* __restrict__ src, float* __restrict__ dst, int64_t nquads, DQ t) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < nquads; q += stride) {
        const int64_t g = q * 4;
        const int64_t blk = g / QK;
        const int e0 = (int)(g - blk * QK);
        const uint8_t* b = src + blk * BS;
        float4 v;
        v.x = dq<T>(b, e0 + 0, t);
        v.y = dq<T>(b, e0 + 1, t);
        v.z = dq<T>(b, e0 + 2, t);
        v.w = dq<T>(b, e0 + 3, t);
        reinterpret_cast<float4*>(dst)[q] = v;
    }
}

template <int T, int QK, int BS>
int run(const void* src, int64_t n, float* dst, hipStream_t st) {
    DQ t{nullptr};
    const int ti = iq_table_index(T);
    if (ti >= 0) {
        IqDeviceTable tab;
        const int rc = iq_device_table(ti, &tab, st);
        if (rc) return rc;
        t.grid = tab.grid;
    }
    const int64_t nq = n / 4;
    const int64_t blocks = (nq + 255) / 256 < 16384 ? (nq + 255) / 256 : 16384;
    hipLaunchKernelGGL((k_dq<T, QK, BS>), dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)src, dst, nq, t);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // namespace
}  // namespace spa

using namespace spa;

extern "C" int spa_dequantize(int type, const void* src, int64_t nrows, int64_t n_per_row, float* dst, void* stream) {
    if (nrows < 0 || n_per_row <= 0) return fail(SPA_ERR_ARG, "spa_dequantize: bad shape %lld x %lld", (long long)nrows, (long long)n_per_row);
    const int64_t n = nrows * n_per_row;
    if (n == 0) return SPA_OK;
    if (!src || !dst) return fail(SPA_ERR_ARG, "spa_dequantize: null pointer");
    if (reinterpret_cast<uintptr_t>(dst) & 15) return fail(SPA_ERR_ARG, "spa_dequantize: output not 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
#define SPA_DQ(T, QK, BS)                                                                                              \
    case T:                                                                                                            \
        if (n_per_row % QK) return fail(SPA_ERR_ARG, "spa_dequantize: row of %lld not a multiple of %d", (long long)n_per_row, QK); \
        return run<T, QK, BS>(src, n, dst, st);
    switch (type) {
        SPA_DQ(2, 32, 18) SPA_DQ(3, 32, 20) SPA_DQ(6, 32, 22) SPA_DQ(7, 32, 24) SPA_DQ(8, 32, 34)
        SPA_DQ(10, 256, 84) SPA_DQ(11, 256, 110) SPA_DQ(12, 256, 144) SPA_DQ(13, 256, 176) SPA_DQ(14, 256, 210)
        SPA_DQ(16, 256, 66) SPA_DQ(17, 256, 74) SPA_DQ(18, 256, 98) SPA_DQ(19, 256, 50) SPA_DQ(20, 32, 18)
        SPA_DQ(21, 256, 110) SPA_DQ(22, 256, 82) SPA_DQ(23, 256, 136) SPA_DQ(29, 256, 56) SPA_DQ(42, 64, 18)
        default: return fail(SPA_ERR_TYPE, "spa_dequantize: type %d not supported", type);
    }
#undef SPA_DQ
}
