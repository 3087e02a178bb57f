// Dequantizers: quantized blocks -> float32, llama.cpp's dequantize_row_<type> for the 20 types of
// the path (ggml-quants.c:439-568, :961-990, :1306-1345, :1530-1550, :1732-1757, :1940-1968,
// :2489-2764). They replace the reference's k_dq_<type> launches (gpuquant.py:214-219) behind
// GPUQuant.dequantize (gpuquant.py:413-421).
//
// Mapping: a workgroup takes tiles of 4096 weights; the tile's blocks are copied to LDS with
// coalesced loads, then each lane decodes 4 consecutive outputs (every type's runs of equal header
// fields hold a multiple of 4 weights: the header is decoded once per 4 outputs, the codes read as
// one 32-bit word) and writes them as one 16-byte store. HBM-bound: 4 bytes written per weight plus
// the block bytes read once.
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
constexpr float IQ1S_DELTA = 0.125f;

// A block's bytes in the workgroup's LDS tile: byte reads, and 32-bit reads from any offset formed
// from the two aligned words around it (v_alignbyte), so no access depends on unaligned LDS support.
struct Blk {
    const uint8_t* tile;    // the LDS tile, 16-byte aligned, 16 bytes of padding after the last block
    int o;                  // the block's first byte in the tile
    __device__ __forceinline__ uint32_t u8(int k) const { return tile[o + k]; }
    __device__ __forceinline__ uint32_t u16(int k) const { return u8(k) | (u8(k + 1) << 8); }
    __device__ __forceinline__ uint32_t u32(int k) const {
        const int a = o + k;
        const uint32_t* w = reinterpret_cast<const uint32_t*>(tile) + (a >> 2);
        return __builtin_amdgcn_alignbyte(w[1], w[0], (uint32_t)(a & 3));   // bytes a&3.. of w[1]:w[0]
    }
    __device__ __forceinline__ float h(int k) const { return f16_to_f32(u16(k)); }
};
// ksigns_iq2xs[i] (ggml-common.h:513): the 7 sign bits and an 8th that makes the count even
__device__ __forceinline__ uint32_t ksigns(uint32_t i) { return i | ((uint32_t)(__popc(i) & 1) << 7); }
// coordinates j0..j0+3 of point g of a lattice (the device tables hold 2l+1 per coordinate) as one word
template <int D>
__device__ __forceinline__ uint32_t gword(const uint8_t* grid, int g, int j0) {
    return reinterpret_cast<const uint32_t*>(grid)[(g * D + j0) >> 2];
}
__device__ __forceinline__ int glev(uint32_t w, int i) { return ((int)((w >> (8 * i)) & 0xff) - 1) >> 1; }
// coordinate values by level: iq2*_grid bytes 8, 25, 43; iq3xxs_grid bytes 4, 12, ..., 52, 62
__device__ __forceinline__ float iq2_val(int l) { return l == 0 ? 8.f : (l == 1 ? 25.f : 43.f); }
__device__ __forceinline__ float iq3xxs_val(int l) { return (float)(l == 7 ? 62 : 8 * l + 4); }
__device__ __forceinline__ float sgn(uint32_t s, int j) { return (s >> j) & 1 ? -1.f : 1.f; }

struct DQ {
    const uint8_t* grid;    // the type's lattice (IQ types), D coordinates per point
};

// outputs e..e+3 of a block (e a multiple of 4; every type's runs of equal header fields hold a
// multiple of 4 weights), each by the C code's expression for that element
template <int T>
__device__ __forceinline__ void dq4(const Blk& b, int e, const DQ& t, const int8_t* kv, float (&v)[4]);

template <> __device__ __forceinline__ void dq4<8>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {     // Q8_0 (:553-567)
    const float d = b.h(0);
    const uint32_t w = b.u32(2 + e);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)(int8_t)(w >> (8 * i)) * d;
}
template <> __device__ __forceinline__ void dq4<2>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {     // Q4_0 (:459-477)
    const float d = b.h(0);
    const uint32_t w = b.u32(2 + (e & 15)) >> (e < 16 ? 0 : 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((int)((w >> (8 * i)) & 0xF) - 8) * d;
}
template <> __device__ __forceinline__ void dq4<3>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {     // Q4_1 (:479-498)
    const float d = b.h(0), m = b.h(2);
    const uint32_t w = b.u32(4 + (e & 15)) >> (e < 16 ? 0 : 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)(int)((w >> (8 * i)) & 0xF) * d + m;
}
// Q5_0 / Q5_1: the fifth bit of element e (j = e mod 16) is qh bit j (e < 16) or bit j + 16
__device__ __forceinline__ uint32_t q5_code(uint32_t w, uint32_t qh, int e, int i) {
    const int j = (e & 15) + i;
    const uint32_t xh = e < 16 ? (((qh >> j) << 4) & 0x10) : ((qh >> (j + 12)) & 0x10);
    const uint32_t lo = e < 16 ? ((w >> (8 * i)) & 0x0F) : ((w >> (8 * i + 4)) & 0x0F);
    return lo | xh;
}
template <> __device__ __forceinline__ void dq4<6>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {     // Q5_0 (:500-524)
    const float d = b.h(0);
    const uint32_t qh = b.u32(2), w = b.u32(6 + (e & 15));
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((int)q5_code(w, qh, e, i) - 16) * d;
}
template <> __device__ __forceinline__ void dq4<7>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {     // Q5_1 (:526-551)
    const float d = b.h(0), m = b.h(2);
    const uint32_t qh = b.u32(4), w = b.u32(8 + (e & 15));
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)(int)q5_code(w, qh, e, i) * d + m;
}
template <> __device__ __forceinline__ void dq4<42>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {    // Q2_0 (:439-457)
    const float d = b.h(0);
    const uint32_t w = b.u8(2 + e / 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((int)((w >> (2 * i)) & 3) - 1) * d;
}
template <> __device__ __forceinline__ void dq4<10>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {    // Q2_K (:961-990)
    const int n = e >> 7, r = e & 127, j = r >> 5, part = (r >> 4) & 1, l = r & 15;
    const uint32_t sc = b.u8(n * 8 + 2 * j + part);
    const float dl = b.h(80) * (float)(int)(sc & 0xF), ml = b.h(82) * (float)(int)(sc >> 4);
    const uint32_t w = b.u32(16 + n * 32 + part * 16 + l) >> (2 * j);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = dl * (float)(int)((w >> (8 * i)) & 3) - ml;
}
template <> __device__ __forceinline__ void dq4<11>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {    // Q3_K (:1306-1345)
    const int n = e >> 7, r = e & 127, j = r >> 5, part = (r >> 4) & 1, l = r & 15;
    const int is = n * 8 + 2 * j + part;
    const uint32_t lo = is < 8 ? (b.u8(96 + is) & 0xF) : (b.u8(96 + is - 8) >> 4);
    const int sc = (int)(lo | (((b.u8(96 + 8 + is % 4) >> (2 * (is / 4))) & 3) << 4)) - 32;
    const float dl = b.h(108) * (float)sc;
    const uint32_t wq = b.u32(32 + n * 32 + part * 16 + l) >> (2 * j), wh = b.u32(part * 16 + l) >> (n * 4 + j);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = (int)((wq >> (8 * i)) & 3);
        const bool hb = (wh >> (8 * i)) & 1;
        v[i] = dl * (float)(q - (hb ? 0 : 4));
    }
}
__device__ __forceinline__ void k4_scale_min(const Blk& b, int j, uint32_t& d, uint32_t& m) {   // get_scale_min_k4 (:880-887), scales at byte 4
    if (j < 4) {
        d = b.u8(4 + j) & 63;
        m = b.u8(4 + j + 4) & 63;
    } else {
        d = (b.u8(4 + j + 4) & 0xF) | ((b.u8(4 + j - 4) >> 6) << 4);
        m = (b.u8(4 + j + 4) >> 4) | ((b.u8(4 + j) >> 6) << 4);
    }
}
template <> __device__ __forceinline__ void dq4<12>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {    // Q4_K (:1530-1550)
    const int c = e >> 6, r = e & 63, l = r & 31;
    uint32_t sc, m;
    k4_scale_min(b, 2 * c + (r >> 5), sc, m);
    const float d1 = b.h(0) * (float)sc, m1 = b.h(2) * (float)m;
    const uint32_t w = b.u32(16 + c * 32 + l) >> (r < 32 ? 0 : 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = d1 * (float)(int)((w >> (8 * i)) & 0xF) - m1;
}
template <> __device__ __forceinline__ void dq4<13>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {    // Q5_K (:1732-1757)
    const int c = e >> 6, r = e & 63, l = r & 31;
    uint32_t sc, m;
    k4_scale_min(b, 2 * c + (r >> 5), sc, m);
    const float d1 = b.h(0) * (float)sc, m1 = b.h(2) * (float)m;
    const uint32_t wl = b.u32(48 + c * 32 + l) >> (r < 32 ? 0 : 4), wh = b.u32(16 + l);
    const uint32_t hbit = r < 32 ? (1u << (2 * c)) : (2u << (2 * c));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = (int)((wl >> (8 * i)) & 0xF) + (((wh >> (8 * i)) & hbit) ? 16 : 0);
        v[i] = d1 * (float)q - m1;
    }
}
template <> __device__ __forceinline__ void dq4<14>(const Blk& b, int e, const DQ&, const int8_t*, float (&v)[4]) {    // Q6_K (:1940-1968)
    const int n = e >> 7, r = e & 127, qd = r >> 5, l = r & 31, is = l / 16;
    const uint32_t wl = b.u32(n * 64 + l + (qd & 1) * 32) >> (qd < 2 ? 0 : 4), wh = b.u32(128 + n * 32 + l) >> (2 * qd);
    const int sc = (int8_t)b.u8(192 + n * 8 + is + 2 * qd);
    const float ds = b.h(208) * (float)sc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t code = ((wl >> (8 * i)) & 0xF) | (((wh >> (8 * i)) & 3) << 4);
        v[i] = ds * (float)((int)(int8_t)(uint8_t)code - 32);
    }
}
template <> __device__ __forceinline__ void dq4<16>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ2_XXS (:2489-2513)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t a1 = b.u32(2 + 8 * ib + 4);
    const float db = b.h(0) * (0.5f + (float)(a1 >> 28)) * 0.25f;
    const uint32_t s = ksigns((a1 >> (7 * l)) & 127);
    const uint32_t gw = gword<8>(t.grid, (int)b.u8(2 + 8 * ib + l), j0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = db * iq2_val(glev(gw, i)) * sgn(s, j0 + i);
}
template <> __device__ __forceinline__ void dq4<17>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ2_XS (:2517-2540)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t sc = b.u8(66 + ib);
    const float db = b.h(0) * (0.5f + (float)((l < 2 ? sc : sc >> 4) & 0xf)) * 0.25f;
    const uint32_t q = b.u16(2 + 2 * (4 * ib + l));
    const uint32_t s = ksigns(q >> 9);
    const uint32_t gw = gword<8>(t.grid, (int)(q & 511), j0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = db * iq2_val(glev(gw, i)) * sgn(s, j0 + i);
}
template <> __device__ __forceinline__ void dq4<22>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ2_S (:2544-2572)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t sc = b.u8(74 + ib);
    const float dl = b.h(0) * (0.5f + (float)((l < 2 ? sc : sc >> 4) & 0xf)) * 0.25f;
    const int g = (int)(b.u8(2 + 4 * ib + l) | ((b.u8(66 + ib) << (8 - 2 * l)) & 0x300));
    const uint32_t s = b.u8(2 + 32 + 4 * ib + l);
    const uint32_t gw = gword<8>(t.grid, g, j0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = dl * iq2_val(glev(gw, i)) * sgn(s, j0 + i);
}
template <> __device__ __forceinline__ void dq4<18>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ3_XXS (:2576-2604)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t a = b.u32(2 + 64 + 4 * ib);
    const float db = b.h(0) * (0.5f + (float)(a >> 28)) * 0.5f;
    const uint32_t s = ksigns((a >> (7 * l)) & 127);
    const uint32_t gw = gword<4>(t.grid, (int)b.u8(2 + 8 * ib + 2 * l + (j0 >> 2)), 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = db * iq3xxs_val(glev(gw, i)) * sgn(s, j0 + i);
}
template <> __device__ __forceinline__ void dq4<21>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ3_S (:2608-2647)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t sc = b.u8(106 + ib / 2);
    const float db = b.h(0) * (float)(1 + 2 * (int)((ib & 1) ? (sc >> 4) : (sc & 0xf)));
    const uint32_t qh = b.u8(66 + ib);
    const int g = j0 < 4 ? (int)(b.u8(2 + 8 * ib + 2 * l) | ((qh << (8 - 2 * l)) & 256))
                         : (int)(b.u8(2 + 8 * ib + 2 * l + 1) | ((qh << (7 - 2 * l)) & 256));
    const uint32_t s = b.u8(74 + 4 * ib + l);
    const uint32_t gw = gword<4>(t.grid, g, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = db * (float)(2 * glev(gw, i) + 1) * sgn(s, j0 + i);
}
template <> __device__ __forceinline__ void dq4<19>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ1_S (:2651-2674)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t qh = b.u16(34 + 2 * ib);
    const float dl = b.h(0) * (float)(2 * (int)((qh >> 12) & 7) + 1);
    const float delta = (qh & 0x8000) ? -IQ1S_DELTA : IQ1S_DELTA;
    const uint32_t gw = gword<8>(t.grid, (int)(b.u8(2 + 4 * ib + l) | (((qh >> (3 * l)) & 7) << 8)), j0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = dl * ((float)(glev(gw, i) - 1) + delta);
}
template <> __device__ __forceinline__ void dq4<29>(const Blk& b, int e, const DQ& t, const int8_t*, float (&v)[4]) {  // IQ1_M (:2676-2724)
    const int ib = e >> 5, l = (e >> 3) & 3, j0 = e & 7;
    const uint32_t s0 = b.u16(48), s1 = b.u16(50), s2 = b.u16(52), s3 = b.u16(54);
    const uint32_t sf = (s0 >> 12) | ((s1 >> 8) & 0x00f0) | ((s2 >> 4) & 0x0f00) | (s3 & 0xf000);
    const float d = f16_to_f32(sf);
    const uint32_t sc = b.u16(48 + 2 * (ib / 2));
    const int sh = 6 * (ib % 2) + (l < 2 ? 0 : 3);
    const float dl = d * (float)(2 * (int)((sc >> sh) & 0x7) + 1);
    const uint32_t qh = b.u8(32 + 2 * ib + (l >> 1));
    const int g = (int)(b.u8(4 * ib + l) | ((qh << ((l & 1) ? 4 : 8)) & 0x700));
    const float delta = (qh & ((l & 1) ? 0x80 : 0x08)) ? -IQ1S_DELTA : IQ1S_DELTA;
    const uint32_t gw = gword<8>(t.grid, g, j0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = dl * ((float)(glev(gw, i) - 1) + delta);
}
template <> __device__ __forceinline__ void dq4<20>(const Blk& b, int e, const DQ&, const int8_t* kv, float (&v)[4]) {  // IQ4_NL (:2726-2742)
    const float d = b.h(0);
    const uint32_t w = b.u32(2 + (e & 15)) >> (e < 16 ? 0 : 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = d * (float)kv[(w >> (8 * i)) & 0xf];
}
template <> __device__ __forceinline__ void dq4<23>(const Blk& b, int e, const DQ&, const int8_t* kv, float (&v)[4]) {  // IQ4_XS (:2744-2764)
    const int ib = e >> 5, r = e & 31;
    const int ls = (int)(((b.u8(4 + ib / 2) >> (4 * (ib % 2))) & 0xf) | (((b.u16(2) >> (2 * ib)) & 3) << 4));
    const float dl = b.h(0) * (float)(ls - 32);
    const uint32_t w = b.u32(8 + 16 * ib + (r & 15)) >> (r < 16 ? 0 : 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = dl * (float)kv[(w >> (8 * i)) & 0xf];
}

// Each workgroup takes tiles of TILE weights (TILE / QK whole blocks, a multiple of 16 bytes): the
// tile's block bytes are copied to LDS with coalesced loads (16-byte loads when the source is
// 16-byte aligned, else 4- or 1-byte loads), then lane q of the tile decodes weights 4q..4q+3 from
// LDS and writes them as one 16-byte store, so consecutive lanes write consecutive bytes.
constexpr int TILE = 4096;
template <int T, int QK, int BS>
__global__ __launch_bounds__(256) void k_dq(const uint8_t* __restrict__ src, float* __restrict__ dst, int64_t nblocks,
                                            DQ t, int align) {
    constexpr int TB = TILE / QK, TBYTES = TB * BS;
    static_assert(TBYTES % 16 == 0, "tile bytes keep the source's 16-byte alignment");
    __shared__ __align__(16) uint8_t tile[TBYTES + 16];
    __shared__ int8_t kv[16];
    if (T == 20 || T == 23) {
        if (threadIdx.x < 16) kv[threadIdx.x] = KV_IQ4NL[threadIdx.x];
    }
    const int64_t ntiles = (nblocks + TB - 1) / TB;
    for (int64_t ti = blockIdx.x; ti < ntiles; ti += gridDim.x) {
        const int64_t b0 = ti * TB;
        const int nb = (int)(nblocks - b0 < TB ? nblocks - b0 : TB);
        const int bytes = nb * BS;
        const uint8_t* s = src + b0 * BS;
        __syncthreads();                     // the last tile's readers are done with it
        int done = 0;
        if (align >= 16) {
            for (int u = threadIdx.x; u < (bytes >> 4); u += 256)
                reinterpret_cast<uint4*>(tile)[u] = reinterpret_cast<const uint4*>(s)[u];
            done = bytes & ~15;
        } else if (align >= 4) {
            for (int u = threadIdx.x; u < (bytes >> 2); u += 256)
                reinterpret_cast<uint32_t*>(tile)[u] = reinterpret_cast<const uint32_t*>(s)[u];
            done = bytes & ~3;
        }
        for (int k = done + threadIdx.x; k < bytes; k += 256) tile[k] = s[k];
        __syncthreads();
        float4* out = reinterpret_cast<float4*>(dst + b0 * QK);
        for (int q = threadIdx.x; q < nb * (QK / 4); q += 256) {
            const int e = q * 4, blk = e / QK;
            float v[4];
            dq4<T>(Blk{tile, blk * BS}, e - blk * QK, t, kv, v);
            out[q] = make_float4(v[0], v[1], v[2], v[3]);
        }
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
    const int64_t nblocks = n / QK, ntiles = (nblocks + TILE / QK - 1) / (TILE / QK);
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    const int align = (a & 15) == 0 ? 16 : ((a & 3) == 0 ? 4 : 1);
    const int64_t grid = ntiles < 4096 ? ntiles : 4096;
    hipLaunchKernelGGL((k_dq<T, QK, BS>), dim3((unsigned)grid), dim3(256), 0, st, (const uint8_t*)src, dst, nblocks, t, align);
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
