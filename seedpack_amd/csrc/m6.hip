// M6: the reference's GPU segmented context rANS for Q8_0 files (gpu_codec.py:1-169, M6GPU at
// :218-334), and the static context-mixed rANS of rans.py (:55-138) that its CPU methods M3-M5 use.
//
// M6 cuts the file's Q8_0 blocks (34 bytes: fp16 scale lo, hi, 32 int8 weights) into segments of 512
// blocks, one rANS state each (PB 12, RANS_L 2^23, byte renormalisation). A block's symbols, in order:
//   hi   | table grp*TPG + 0   + previous block's hi (0 at a row start or the segment's first block)
//   lo   | table grp*TPG + 256 + hi
//   pos  | table grp*TPG + 512           (the position of the largest |weight|, first of equals)
//   mx   | table grp*TPG + 513           (the weight byte there)
//   qs   | table grp*TPG + 514 + bucket(scale) * 16 + column class, for the other 31 weights
// with bucket = clamp((scale bits - the tensor's median scale bits) >> 8 + 8, 0, 15) (floor division)
// and the column class of the weight's input column (16 quantile classes of the column RMS).
//
// MI355X mapping: the per-tensor statistics are device passes (a 65536-bin histogram of the scale
// bits whose median the host reads; the column mean squares summed in row order, lane per column, as
// the reference's --cpu path sums them); histogram, encoder and decoder run a lane per segment (the
// state is serial); the encoder walks each block's symbols in reverse directly (no per-block list).
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace spa {
namespace m6 {
namespace {

constexpr uint32_t PB = 12, PSCALE = 1u << PB, RANS_L = 1u << 23;
constexpr int SEG = 512, N_COL = 16, N_SB = 16;
constexpr int TPG = 256 + 256 + 1 + 1 + N_SB * N_COL;
constexpr int T_HI = 0, T_LO = 256, T_POS = 512, T_MX = 513, T_QS = 514;

struct Meta { int32_t first, nblocks, nb_row, grp, colbase, med; };     // per tensor (gpu_codec.py:190 META_DT)
static_assert(sizeof(Meta) == 24, "descriptor layout");

__device__ __forceinline__ int tensor_of(const int32_t* tfirst, int ntens, int b) {
    int lo = 0, hi = ntens - 1;                      // the last tensor whose first block is <= b
    while (lo < hi) {
        const int m = (lo + hi + 1) >> 1;
        if (tfirst[m] <= b) lo = m; else hi = m - 1;
    }
    return lo;
}

__device__ __forceinline__ int sbucket(int lo, int hi, int med) {
    const int v = (((lo | (hi << 8)) - med) >> 8) + N_SB / 2;          // arithmetic shift: floor division
    return v < 0 ? 0 : (v > N_SB - 1 ? N_SB - 1 : v);
}

// counts[lo | hi << 8] += 1 over blocks [first, first + nb): the scale bits' histogram
__global__ __launch_bounds__(256) void k_scale_hist(const uint8_t* __restrict__ blocks, int64_t first, int64_t nb,
                                                    uint32_t* __restrict__ counts) {
    for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < nb; b += (int64_t)gridDim.x * 256) {
        const uint8_t* blk = blocks + (first + b) * 34;
        atomicAdd(&counts[blk[0] | (blk[1] << 8)], 1u);
    }
}

// rms[c] = sqrt(mean over rows of q^2) for column c of a tensor of nrows x (nb_row * 32) weights: float32
// squares added in row order, divided by the row count in float32 (numpy's mean over axis 0)
__global__ __launch_bounds__(256) void k_col_rms(const uint8_t* __restrict__ blocks, int64_t first, int64_t nrows, int nb_row,
                                                 float* __restrict__ rms) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= nb_row * 32) return;
    const uint8_t* p = blocks + (first + c / 32) * 34 + 2 + (c & 31);
    const int64_t stride = (int64_t)nb_row * 34;
    float s = 0.f;
    constexpr int AHEAD = 8;
    for (int64_t r0 = 0; r0 < nrows; r0 += AHEAD) {
        float q[AHEAD];
#pragma unroll
        for (int k = 0; k < AHEAD; ++k) q[k] = r0 + k < nrows ? (float)(int8_t)p[(r0 + k) * stride] : 0.f;
#pragma unroll
        for (int k = 0; k < AHEAD; ++k)
            if (r0 + k < nrows) s = s + q[k] * q[k];
    }
    rms[c] = sqrtf(s / (float)nrows);
}

// pos[b]: the first position of the largest |weight| of block b
__global__ __launch_bounds__(256) void k_pos(const uint8_t* __restrict__ blocks, int64_t n, uint8_t* __restrict__ pos) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= n) return;
    const uint8_t* q = blocks + b * 34 + 2;
    int best = -1, bp = 0;
    for (int j = 0; j < 32; ++j) {
        const int a = abs((int)(int8_t)q[j]);
        if (a > best) { best = a; bp = j; }
    }
    pos[b] = (uint8_t)bp;
}

struct Args {
    const uint8_t* blocks;
    const uint8_t* pos;
    const Meta* M;
    const int32_t* tfirst;
    int ntens;
    const uint8_t* colmap;
    int nblocks;
};

// the symbols of block b in coding order: emit(table, symbol)
template <class F>
__device__ __forceinline__ void block_symbols(const Args& a, int t, int b, int b0, F&& emit) {
    const Meta m = a.M[t];
    const uint8_t* blk = a.blocks + (int64_t)b * 34;
    const int inrow = (b - m.first) % m.nb_row;
    const int base = m.grp * TPG;
    const int prev = (inrow == 0 || b == b0) ? 0 : a.blocks[(int64_t)(b - 1) * 34 + 1];
    const int lo = blk[0], hi = blk[1], p = a.pos[b];
    emit(base + T_HI + prev, hi);
    emit(base + T_LO + hi, lo);
    emit(base + T_POS, p);
    emit(base + T_MX, blk[2 + p]);
    const int qb = base + T_QS + sbucket(lo, hi, m.med) * N_COL;
    const uint8_t* cm = a.colmap + m.colbase + inrow * 32;
    for (int j = 0; j < 32; ++j)
        if (j != p) emit(qb + cm[j], blk[2 + j]);
}

__global__ __launch_bounds__(128) void k_hist(Args a, uint32_t* __restrict__ counts) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    const int b0 = s * SEG;
    if (b0 >= a.nblocks) return;
    const int b1 = min(b0 + SEG, a.nblocks);
    int t = tensor_of(a.tfirst, a.ntens, b0);
    for (int b = b0; b < b1; ++b) {
        if (t + 1 < a.ntens && b >= a.tfirst[t + 1]) ++t;
        block_symbols(a, t, b, b0, [&](int tab, int sym) { atomicAdd(&counts[tab * 256 + sym], 1u); });
    }
}

// a segment coded backwards into its slot [s * cap, (s + 1) * cap), written downwards from the end;
// a block's symbols are pushed in reverse order (31 weights last to first, mx, pos, lo, hi)
__global__ __launch_bounds__(128) void k_enc(Args a, const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                             uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    const int b0 = s * SEG;
    if (b0 >= a.nblocks) return;
    const int b1 = min(b0 + SEG, a.nblocks);
    uint8_t* const end = out + (uint64_t)(s + 1) * cap;
    uint8_t* ptr = end;
    uint32_t x = RANS_L;
    auto put = [&](int tab, int sym) {
        const uint32_t f = freq[tab * 256 + sym], c = cum[tab * 257 + sym];
        const uint32_t x_max = ((RANS_L >> PB) << 8) * f;
        while (x >= x_max) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
        x = ((x / f) << PB) + (x % f) + c;
    };
    int t = tensor_of(a.tfirst, a.ntens, b1 - 1);
    for (int b = b1 - 1; b >= b0; --b) {
        while (b < a.M[t].first) --t;
        const Meta m = a.M[t];
        const uint8_t* blk = a.blocks + (int64_t)b * 34;
        const int inrow = (b - m.first) % m.nb_row;
        const int base = m.grp * TPG;
        const int prev = (inrow == 0 || b == b0) ? 0 : a.blocks[(int64_t)(b - 1) * 34 + 1];
        const int lo = blk[0], hi = blk[1], p = a.pos[b];
        const int qb = base + T_QS + sbucket(lo, hi, m.med) * N_COL;
        const uint8_t* cm = a.colmap + m.colbase + inrow * 32;
        for (int j = 31; j >= 0; --j)
            if (j != p) put(qb + cm[j], blk[2 + j]);
        put(base + T_MX, blk[2 + p]);
        put(base + T_POS, p);
        put(base + T_LO + hi, lo);
        put(base + T_HI + prev, hi);
    }
    for (int i = 0; i < 4; ++i) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
    out_len[s] = (uint32_t)(end - ptr);
}

// (bytes past in_bytes read as zeros: a damaged stream decodes to wrong blocks, never outside the buffers;
// a position symbol is taken modulo 32 for the same reason)
__global__ __launch_bounds__(128) void k_dec(const uint8_t* __restrict__ in, uint64_t in_bytes, const uint64_t* __restrict__ in_off,
                                             Args a, const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                             const uint8_t* __restrict__ lut, uint8_t* __restrict__ blocks) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    const int b0 = s * SEG;
    if (b0 >= a.nblocks) return;
    const int b1 = min(b0 + SEG, a.nblocks);
    uint64_t at = in_off[s];
    auto byte = [&]() -> uint32_t { const uint32_t v = at < in_bytes ? in[at] : 0u; ++at; return v; };
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) x = (x << 8) | byte();
    auto get = [&](int tab) {
        const uint32_t slot = x & (PSCALE - 1);
        const int sym = lut[(int64_t)tab * PSCALE + slot];
        x = freq[tab * 256 + sym] * (x >> PB) + slot - cum[tab * 257 + sym];
        while (x < RANS_L) x = (x << 8) | byte();
        return sym;
    };
    int t = tensor_of(a.tfirst, a.ntens, b0), prev = 0;
    for (int b = b0; b < b1; ++b) {
        if (t + 1 < a.ntens && b >= a.tfirst[t + 1]) ++t;
        const Meta m = a.M[t];
        uint8_t* blk = blocks + (int64_t)b * 34;
        const int inrow = (b - m.first) % m.nb_row;
        const int base = m.grp * TPG;
        if (inrow == 0 || b == b0) prev = 0;
        const int hi = get(base + T_HI + prev);
        const int lo = get(base + T_LO + hi);
        const int p = get(base + T_POS) & 31;
        const int mx = get(base + T_MX);
        blk[0] = (uint8_t)lo; blk[1] = (uint8_t)hi; blk[2 + p] = (uint8_t)mx;
        prev = hi;
        const int qb = base + T_QS + sbucket(lo, hi, m.med) * N_COL;
        const uint8_t* cm = a.colmap + m.colbase + inrow * 32;
        for (int j = 0; j < 32; ++j)
            if (j != p) blk[2 + j] = (uint8_t)get(qb + cm[j]);
    }
}

}  // namespace
}  // namespace m6

// ---------------------------------------------------------------- rans.py: static context-mixed rANS
//
// One stream per lane: symbols of 8 bits, each coded with the frequency table of its context
// (rows of n_sym entries summing to 2^14), RANS_L 2^23, byte renormalisation; the encoder runs from
// the last symbol to the first and ends with the 4-byte state, the decoder reads that state first.
// A stream's context is given per symbol, or (o1 streams, rans.py:108-138) is the previous symbol,
// reset to 0 every `period` symbols.
namespace crans {
namespace {

constexpr uint32_t PB = 14, PSCALE = 1u << PB, RANS_L = 1u << 23;

struct Stream { int64_t sym_off, n, ctx_off, tab_row, out_off; int32_t period, pad; };   // 48 bytes
static_assert(sizeof(Stream) == 48, "descriptor layout");

__global__ __launch_bounds__(64) void k_enc(const uint8_t* __restrict__ sym, const int32_t* __restrict__ ctx, int n_sym,
                                            const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                            const Stream* __restrict__ st, int nst, uint8_t* __restrict__ out,
                                            uint32_t* __restrict__ out_len) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= nst) return;
    const Stream S = st[k];
    uint8_t* const end = out + S.out_off + 2 * S.n + 16;      // the slot of rans.encode (rans.py:150)
    uint8_t* ptr = end;
    uint32_t x = RANS_L;
    for (int64_t i = S.n - 1; i >= 0; --i) {
        const int64_t row = S.tab_row + ctx[S.ctx_off + i];
        const int s = sym[S.sym_off + i];
        const uint32_t f = freq[row * n_sym + s], c = cum[row * (n_sym + 1) + s];
        const uint32_t x_max = ((RANS_L >> PB) << 8) * f;
        while (x >= x_max) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
        x = ((x / f) << PB) + (x % f) + c;
    }
    for (int i = 0; i < 4; ++i) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
    out_len[k] = (uint32_t)(end - ptr);
}

__global__ __launch_bounds__(64) void k_dec(const uint8_t* __restrict__ in, uint64_t in_bytes, const int32_t* __restrict__ ctx,
                                            int n_sym, const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                            const uint8_t* __restrict__ lut, const Stream* __restrict__ st, int nst,
                                            uint8_t* __restrict__ sym) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= nst) return;
    const Stream S = st[k];
    uint64_t at = (uint64_t)S.out_off;
    auto byte = [&]() -> uint32_t { const uint32_t v = at < in_bytes ? in[at] : 0u; ++at; return v; };   // past the end: zeros
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) x = (x << 8) | byte();
    int prev = 0;
    for (int64_t i = 0; i < S.n; ++i) {
        int c;
        if (S.period > 0) {
            if (i % S.period == 0) prev = 0;
            c = prev;
        } else {
            c = ctx[S.ctx_off + i];
        }
        const int64_t row = S.tab_row + c;
        const uint32_t slot = x & (PSCALE - 1);
        const int s = lut[row * PSCALE + slot];
        sym[S.sym_off + i] = (uint8_t)s;
        prev = s;
        x = freq[row * n_sym + s] * (x >> PB) + slot - cum[row * (n_sym + 1) + s];
        while (x < RANS_L) x = (x << 8) | byte();
    }
}

}  // namespace
}  // namespace crans
}  // namespace spa

using spa::fail;

extern "C" {

int spa_m6_scale_hist(const void* blocks, int64_t first, int64_t nb, uint32_t* counts, void* stream) {
    if (first < 0 || nb < 0) return fail(SPA_ERR_ARG, "spa_m6_scale_hist: blocks %lld + %lld", (long long)first, (long long)nb);
    if (!nb) return SPA_OK;
    if (!blocks || !counts) return fail(SPA_ERR_ARG, "spa_m6_scale_hist: null pointer");
    const int64_t g = (nb + 255) / 256;
    hipLaunchKernelGGL(spa::m6::k_scale_hist, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blocks, first, nb, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_m6_col_rms(const void* blocks, int64_t first, int64_t nrows, int nb_row, float* rms, void* stream) {
    if (first < 0 || nrows <= 0 || nb_row <= 0)
        return fail(SPA_ERR_ARG, "spa_m6_col_rms: %lld rows of %d blocks", (long long)nrows, nb_row);
    if (!blocks || !rms) return fail(SPA_ERR_ARG, "spa_m6_col_rms: null pointer");
    hipLaunchKernelGGL(spa::m6::k_col_rms, dim3((unsigned)((nb_row * 32 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blocks, first, nrows, nb_row, rms);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_m6_pos(const void* blocks, int64_t n, uint8_t* pos, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_m6_pos: %lld blocks", (long long)n);
    if (!n) return SPA_OK;
    if (!blocks || !pos) return fail(SPA_ERR_ARG, "spa_m6_pos: null pointer");
    hipLaunchKernelGGL(spa::m6::k_pos, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blocks, n, pos);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

static int m6_args(const char* who, const void* blocks, const uint8_t* pos, const void* meta, const int32_t* tfirst, int ntens,
                   const uint8_t* colmap, int nblocks, spa::m6::Args* a) {
    if (nblocks < 0 || ntens <= 0) return fail(SPA_ERR_ARG, "%s: %d blocks in %d tensors", who, nblocks, ntens);
    if (!blocks || !pos || !meta || !tfirst || !colmap) return fail(SPA_ERR_ARG, "%s: null pointer", who);
    *a = {(const uint8_t*)blocks, pos, (const spa::m6::Meta*)meta, tfirst, ntens, colmap, nblocks};
    return SPA_OK;
}

int spa_m6_segments(int nblocks) { return nblocks > 0 ? (nblocks + spa::m6::SEG - 1) / spa::m6::SEG : 0; }

int spa_m6_hist(const void* blocks, const uint8_t* pos, const void* meta, const int32_t* tfirst, int ntens,
                const uint8_t* colmap, int nblocks, uint32_t* counts, void* stream) {
    spa::m6::Args a;
    if (int e = m6_args("spa_m6_hist", blocks, pos, meta, tfirst, ntens, colmap, nblocks, &a)) return e;
    if (!counts) return fail(SPA_ERR_ARG, "spa_m6_hist: null pointer");
    const int nseg = spa_m6_segments(nblocks);
    if (!nseg) return SPA_OK;
    hipLaunchKernelGGL(spa::m6::k_hist, dim3((unsigned)((nseg + 127) / 128)), dim3(128), 0, (hipStream_t)stream, a, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_m6_encode(const void* blocks, const uint8_t* pos, const void* meta, const int32_t* tfirst, int ntens,
                  const uint8_t* colmap, int nblocks, const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap,
                  uint32_t* out_len, void* stream) {
    spa::m6::Args a;
    if (int e = m6_args("spa_m6_encode", blocks, pos, meta, tfirst, ntens, colmap, nblocks, &a)) return e;
    if (!freq || !cum || !out || !out_len) return fail(SPA_ERR_ARG, "spa_m6_encode: null pointer");
    if (cap < (uint64_t)spa::m6::SEG * 34 * 2 + 16) return fail(SPA_ERR_ARG, "spa_m6_encode: slot capacity %llu too small", (unsigned long long)cap);
    const int nseg = spa_m6_segments(nblocks);
    if (!nseg) return SPA_OK;
    hipLaunchKernelGGL(spa::m6::k_enc, dim3((unsigned)((nseg + 127) / 128)), dim3(128), 0, (hipStream_t)stream, a, freq,
                       cum, (uint8_t*)out, cap, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_m6_decode(const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* meta, const int32_t* tfirst, int ntens,
                  const uint8_t* colmap, int nblocks, const uint16_t* freq, const uint32_t* cum, const uint8_t* lut,
                  void* blocks, void* stream) {
    if (nblocks < 0 || ntens <= 0) return fail(SPA_ERR_ARG, "spa_m6_decode: %d blocks in %d tensors", nblocks, ntens);
    if (!in || !in_off || !meta || !tfirst || !colmap || !freq || !cum || !lut || !blocks)
        return fail(SPA_ERR_ARG, "spa_m6_decode: null pointer");
    const int nseg = spa_m6_segments(nblocks);
    if (!nseg) return SPA_OK;
    // the decoder reads each block's scale and position before its weights: the blocks it writes
    const spa::m6::Args a{(const uint8_t*)blocks, nullptr, (const spa::m6::Meta*)meta, tfirst, ntens, colmap, nblocks};
    hipLaunchKernelGGL(spa::m6::k_dec, dim3((unsigned)((nseg + 127) / 128)), dim3(128), 0, (hipStream_t)stream,
                       (const uint8_t*)in, in_bytes, in_off, a, freq, cum, lut, (uint8_t*)blocks);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_crans_encode(const uint8_t* sym, const int32_t* ctx, int n_sym, const uint16_t* freq, const uint32_t* cum,
                     const void* streams, int nst, void* out, uint32_t* out_len, void* stream) {
    if (nst < 0 || n_sym <= 0 || n_sym > 256) return fail(SPA_ERR_ARG, "spa_crans_encode: %d streams of %d symbols", nst, n_sym);
    if (!nst) return SPA_OK;
    if (!sym || !ctx || !freq || !cum || !streams || !out || !out_len) return fail(SPA_ERR_ARG, "spa_crans_encode: null pointer");
    hipLaunchKernelGGL(spa::crans::k_enc, dim3((unsigned)((nst + 63) / 64)), dim3(64), 0, (hipStream_t)stream, sym, ctx,
                       n_sym, freq, cum, (const spa::crans::Stream*)streams, nst, (uint8_t*)out, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_crans_decode(const void* in, uint64_t in_bytes, const int32_t* ctx, int n_sym, const uint16_t* freq, const uint32_t* cum,
                     const uint8_t* lut, const void* streams, int nst, uint8_t* sym, void* stream) {
    if (nst < 0 || n_sym <= 0 || n_sym > 256) return fail(SPA_ERR_ARG, "spa_crans_decode: %d streams of %d symbols", nst, n_sym);
    if (!nst) return SPA_OK;
    if (!in || !freq || !cum || !lut || !streams || !sym) return fail(SPA_ERR_ARG, "spa_crans_decode: null pointer");
    hipLaunchKernelGGL(spa::crans::k_dec, dim3((unsigned)((nst + 63) / 64)), dim3(64), 0, (hipStream_t)stream,
                       (const uint8_t*)in, in_bytes, ctx, n_sym, freq, cum, lut, (const spa::crans::Stream*)streams, nst, sym);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
