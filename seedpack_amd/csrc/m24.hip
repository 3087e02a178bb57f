// M24: the first-generation GPU BF16 codec of the reference (gpu_bf16.py:36-132, method m28's base
// codec). Per weight three symbols coded with one rANS state per segment of 16384 weights:
//   exponent  | context eb  = clamp((rfi[row] + cfi[col] + 108) >> 1, 0, 127)       (tables tab + eb)
//   mantissa  | context rel = clamp(ex - ((rfi + cfi + 508) >> 2) + 8, 0, 15)       (tab + 128 + rel)
//   sign      | context     = the column's bias class scl[col]                       (tab + 144 + scl)
// with rfi / cfi the row and column RMS in quarter octaves and 160 tables per tensor. PB 12,
// RANS_L 2^23, byte renormalisation; a segment is coded backwards (sign, mantissa, exponent per
// weight) and ends with the 4-byte state.
//
// MI355X mapping: the column statistics are one pass over the BF16 tensor (lane per column, the
// row-normalised values formed on the fly, both sums in row order); the histogram takes a
// workgroup per segment with the exponent counts of a 32-context window, the mantissa and sign
// counts in LDS (other exponent contexts go straight to the global counts); encode and decode run a
// lane per segment (the state is serial), the encoder's step division-free with per-(table, symbol)
// reciprocals.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace spa {
namespace m24 {
namespace {

constexpr uint32_t PB = 12, PSCALE = 1u << PB, RANS_L = 1u << 23;
constexpr int SEG = 16384, EWIN = 32;

struct TB { int64_t off; int32_t rowlen, rowbase, colbase, tab; };      // gpu_bf16.py:271 TB_DT
struct SG { int32_t t, n; int64_t i0; };                                // gpu_bf16.py:272 SG_DT
static_assert(sizeof(TB) == 24 && sizeof(SG) == 16, "descriptor layout");

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ float bf(uint32_t u) { return __uint_as_float(u << 16); }

// s1[c] = sum_r w[r][c] / rfa[r], s2[c] = sum_r (w[r][c] / rfa[r])^2: float32 quotients, float64 sums in
// row order (detmath.cols of the row-normalised tensor, gpu_bf16.py:362-366)
__global__ __launch_bounds__(256) void k_cols(const uint16_t* __restrict__ w, const float* __restrict__ rfa, int64_t nr,
                                              int rowlen, double* __restrict__ s1, double* __restrict__ s2) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= rowlen) return;
    double a = 0.0, b = 0.0;
    constexpr int AHEAD = 8;
    for (int64_t r0 = 0; r0 < nr; r0 += AHEAD) {
        float q[AHEAD];
#pragma unroll
        for (int k = 0; k < AHEAD; ++k) q[k] = r0 + k < nr ? bf(w[(r0 + k) * rowlen + c]) / rfa[r0 + k] : 0.f;
#pragma unroll
        for (int k = 0; k < AHEAD; ++k) {
            if (r0 + k < nr) {
                const double d = (double)q[k];
                a = a + d;
                b = b + d * d;
            }
        }
    }
    s1[c] = a;
    s2[c] = b;
}

struct Ctx {
    int eb, sh;                                    // exponent context, the mantissa's reference level
};
__device__ __forceinline__ Ctx ctx_of(const TB& T, const int16_t* rfi, const int16_t* cfi, int r, int j) {
    const int pred4 = rfi[T.rowbase + r] + cfi[T.colbase + j];
    return Ctx{clampi((pred4 + 108) >> 1, 0, 127), (pred4 + 508) >> 2};
}

// a workgroup per segment
__global__ __launch_bounds__(256) void k_hist(const uint8_t* __restrict__ file, const TB* __restrict__ tb,
                                              const SG* __restrict__ sg, const int16_t* __restrict__ rfi,
                                              const int16_t* __restrict__ cfi, const int8_t* __restrict__ scl,
                                              uint32_t* __restrict__ counts) {
    __shared__ uint32_t ce[EWIN * 256];
    __shared__ uint32_t cm[16 * 128];
    __shared__ uint32_t cs[16 * 2];
    __shared__ int s_lo;
    const SG g = sg[blockIdx.x];
    const TB T = tb[g.t];
    const uint16_t* w = reinterpret_cast<const uint16_t*>(file + T.off) + g.i0;
    for (int i = threadIdx.x; i < EWIN * 256; i += 256) ce[i] = 0;
    for (int i = threadIdx.x; i < 16 * 128; i += 256) cm[i] = 0;
    if (threadIdx.x < 32) cs[threadIdx.x] = 0;
    if (threadIdx.x == 0) {
        const int r = (int)(g.i0 / T.rowlen), j = (int)(g.i0 % T.rowlen);
        s_lo = clampi(ctx_of(T, rfi, cfi, r, j).eb - EWIN / 2, 0, 128 - EWIN);
    }
    __syncthreads();
    const int lo = s_lo;
    for (int k = threadIdx.x; k < g.n; k += 256) {
        const int64_t i = g.i0 + k;
        const int r = (int)(i / T.rowlen), j = (int)(i % T.rowlen);
        const uint32_t u = w[k];
        const int ex = (u >> 7) & 255, man = u & 127, sgn = u >> 15;
        const Ctx c = ctx_of(T, rfi, cfi, r, j);
        const int rel = clampi(ex - c.sh + 8, 0, 15);
        if (c.eb >= lo && c.eb < lo + EWIN) atomicAdd(&ce[(c.eb - lo) * 256 + ex], 1u);
        else atomicAdd(&counts[(size_t)(T.tab + c.eb) * 256 + ex], 1u);
        atomicAdd(&cm[rel * 128 + man], 1u);
        atomicAdd(&cs[scl[T.colbase + j] * 2 + sgn], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < EWIN * 256; i += 256)
        if (ce[i]) atomicAdd(&counts[(size_t)(T.tab + lo + i / 256) * 256 + (i % 256)], ce[i]);
    for (int i = threadIdx.x; i < 16 * 128; i += 256)
        if (cm[i]) atomicAdd(&counts[(size_t)(T.tab + 128 + i / 128) * 256 + (i % 128)], cm[i]);
    if (threadIdx.x < 32 && cs[threadIdx.x])
        atomicAdd(&counts[(size_t)(T.tab + 144 + threadIdx.x / 2) * 256 + (threadIdx.x % 2)], cs[threadIdx.x]);
}

// the encoder's reciprocal per (used table, symbol): Giesen's rans_byte form (see qr.hip enc_rcp)
__global__ __launch_bounds__(256) void k_rcp(const int* __restrict__ remap, const uint16_t* __restrict__ freq, int ntab,
                                             uint32_t* __restrict__ rcp) {
    const int tab = blockIdx.x;
    if (tab >= ntab) return;
    const int tt = remap[tab];
    if (tt < 0) return;
    const uint32_t f = freq[tt * 256 + threadIdx.x];
    uint32_t r = 0xffffffffu;
    if (f >= 2) {
        const uint32_t sh = 32 - __clz(f - 1);
        r = (uint32_t)(((1ull << (31 + sh)) + f - 1) / f);
    }
    rcp[tt * 256 + threadIdx.x] = r;
}

struct Enc {
    uint32_t x;
    uint8_t* ptr;
    const int* remap;
    const uint16_t* freq;
    const uint32_t* cum;
    const uint32_t* rcp;
    __device__ __forceinline__ void put(int tab, uint32_t s) {
        const int tt = remap[tab];
        const uint32_t f = freq[tt * 256 + s], c = cum[tt * 257 + s], r = rcp[tt * 256 + s];
        const uint32_t xm = ((RANS_L >> PB) << 8) * f;
        while (x >= xm) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
        const uint32_t sh = f < 2 ? 0u : 31u - __clz(f - 1);
        const uint32_t q = __umulhi(x, r) >> sh;
        x = x + c + (f < 2 ? PSCALE - 1 : 0u) + q * (PSCALE - f);
    }
};

__global__ __launch_bounds__(64) void k_enc(const uint8_t* __restrict__ file, const TB* __restrict__ tb,
                                            const SG* __restrict__ sg, int nseg, const int16_t* __restrict__ rfi,
                                            const int16_t* __restrict__ cfi, const int8_t* __restrict__ scl,
                                            const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                            const uint32_t* __restrict__ cum, const uint32_t* __restrict__ rcp,
                                            uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const SG g = sg[s];
    const TB T = tb[g.t];
    const uint16_t* w = reinterpret_cast<const uint16_t*>(file + T.off) + g.i0;
    const int64_t last = g.i0 + g.n - 1;
    int r = (int)(last / T.rowlen), j = (int)(last % T.rowlen);
    uint8_t* const start = out + (uint64_t)s * cap;
    uint8_t* const end = start + cap;
    Enc e{RANS_L, end, remap, freq, cum, rcp};
    for (int k = g.n - 1; k >= 0; --k) {
        const uint32_t u = w[k];
        const int ex = (u >> 7) & 255, man = u & 127, sgn = u >> 15;
        const Ctx c = ctx_of(T, rfi, cfi, r, j);
        const int rel = clampi(ex - c.sh + 8, 0, 15);
        e.put(T.tab + 144 + scl[T.colbase + j], (uint32_t)sgn);
        e.put(T.tab + 128 + rel, (uint32_t)man);
        e.put(T.tab + c.eb, (uint32_t)ex);
        if (e.ptr - start < 64) { out_len[s] = 0xffffffffu; return; }      // slot overflow
        if (--j < 0) { j = T.rowlen - 1; --r; }
    }
    for (int i = 0; i < 4; ++i) { *--e.ptr = (uint8_t)(e.x & 0xff); e.x >>= 8; }
    out_len[s] = (uint32_t)(end - e.ptr);
}

__global__ __launch_bounds__(64) void k_dec(const uint8_t* __restrict__ in, uint64_t in_bytes, const uint64_t* __restrict__ in_off,
                                            uint8_t* __restrict__ file, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                            int nseg, const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                            const int8_t* __restrict__ scl, const int* __restrict__ remap,
                                            const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                            const uint8_t* __restrict__ lut) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const SG g = sg[s];
    const TB T = tb[g.t];
    uint16_t* w = reinterpret_cast<uint16_t*>(file + T.off) + g.i0;
    int r = (int)(g.i0 / T.rowlen), j = (int)(g.i0 % T.rowlen);
    const uint8_t* ptr = in + (in_off[s] < in_bytes ? in_off[s] : in_bytes);
    const uint8_t* const endp = in + in_bytes;
    auto byte = [&]() -> uint32_t { const uint32_t b = ptr < endp ? *ptr : 0u; ++ptr; return b; };
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) x = (x << 8) | byte();
    auto get = [&](int tab) -> int {
        const int tt = remap[tab];
        const uint32_t slot = x & (PSCALE - 1);
        const int v = lut[(size_t)tt * PSCALE + slot];
        x = freq[tt * 256 + v] * (x >> PB) + slot - cum[tt * 257 + v];
        while (x < RANS_L) x = (x << 8) | byte();
        return v;
    };
    for (int k = 0; k < g.n; ++k) {
        const Ctx c = ctx_of(T, rfi, cfi, r, j);
        const int ex = get(T.tab + c.eb);
        const int rel = clampi(ex - c.sh + 8, 0, 15);
        const int man = get(T.tab + 128 + rel);
        const int sgn = get(T.tab + 144 + scl[T.colbase + j]);
        w[k] = (uint16_t)((sgn << 15) | (ex << 7) | man);
        if (++j == T.rowlen) { j = 0; ++r; }
    }
}

}  // namespace
}  // namespace m24
}  // namespace spa

using spa::fail;

extern "C" {

int spa_m24_cols(const void* w, const float* rfa, int64_t nr, int rowlen, double* s1, double* s2, void* stream) {
    if (nr < 0 || rowlen <= 0) return fail(SPA_ERR_ARG, "spa_m24_cols: shape %lld x %d", (long long)nr, rowlen);
    if (!w || !rfa || !s1 || !s2) return fail(SPA_ERR_ARG, "spa_m24_cols: null pointer");
    hipLaunchKernelGGL(spa::m24::k_cols, dim3((unsigned)((rowlen + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)w, rfa, nr, rowlen, s1, s2);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_m24_hist(const void* file, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                 const int8_t* scl, uint32_t* counts, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_m24_hist: negative segment count");
    if (!nseg) return SPA_OK;
    if (!file || !tb || !sg || !rfi || !cfi || !scl || !counts) return fail(SPA_ERR_ARG, "spa_m24_hist: null pointer");
    hipLaunchKernelGGL(spa::m24::k_hist, dim3((unsigned)nseg), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)file,
                       (const spa::m24::TB*)tb, (const spa::m24::SG*)sg, rfi, cfi, scl, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

size_t spa_m24_rcp_bytes(int ntab) { return ntab > 0 ? (size_t)ntab * 256 * 4 : 0; }

int spa_m24_encode(const void* file, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                   const int8_t* scl, const int* remap, int ntab, const uint16_t* freq, const uint32_t* cum, uint32_t* rcp,
                   void* out, uint64_t cap, uint32_t* out_len, void* stream) {
    if (nseg < 0 || ntab <= 0) return fail(SPA_ERR_ARG, "spa_m24_encode: %d segments, %d tables", nseg, ntab);
    if (cap < (uint64_t)spa::m24::SEG * 2 + 1024) return fail(SPA_ERR_ARG, "spa_m24_encode: slot capacity %llu too small", (unsigned long long)cap);
    if (!nseg) return SPA_OK;
    if (!file || !tb || !sg || !rfi || !cfi || !scl || !remap || !freq || !cum || !rcp || !out || !out_len)
        return fail(SPA_ERR_ARG, "spa_m24_encode: null pointer");
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(spa::m24::k_rcp, dim3((unsigned)ntab), dim3(256), 0, st, remap, freq, ntab, rcp);
    hipLaunchKernelGGL(spa::m24::k_enc, dim3((unsigned)((nseg + 63) / 64)), dim3(64), 0, st, (const uint8_t*)file,
                       (const spa::m24::TB*)tb, (const spa::m24::SG*)sg, nseg, rfi, cfi, scl, remap, freq, cum,
                       (const uint32_t*)rcp, (uint8_t*)out, cap, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_m24_decode(const void* in, uint64_t in_bytes, const uint64_t* in_off, void* file, const void* tb, const void* sg,
                   int nseg, const int16_t* rfi, const int16_t* cfi, const int8_t* scl, const int* remap,
                   const uint16_t* freq, const uint32_t* cum, const uint8_t* lut, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_m24_decode: negative segment count");
    if (!nseg) return SPA_OK;
    if (!in || !in_off || !file || !tb || !sg || !rfi || !cfi || !scl || !remap || !freq || !cum || !lut)
        return fail(SPA_ERR_ARG, "spa_m24_decode: null pointer");
    hipLaunchKernelGGL(spa::m24::k_dec, dim3((unsigned)((nseg + 63) / 64)), dim3(64), 0, (hipStream_t)stream,
                       (const uint8_t*)in, in_bytes, in_off, (uint8_t*)file, (const spa::m24::TB*)tb,
                       (const spa::m24::SG*)sg, nseg, rfi, cfi, scl, remap, freq, cum, lut);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
