// R2 BF16 base codec kernels (seedpack/bf16v2.py semantics, with seedpack/detmath.py's arithmetic).
//
// Per tensor of BF16 bits (rows x rl):
//   side information  rfi[row] = rint(8 log2(rms(row) + 1e-30)), cfi[col] the same of the column
//                     after dividing each row by 2^(rf/8), scl[col] = clip(floor(16 mean / 2^(cfi/8)) + 8),
//                     all from float64 sums in index order and detmath's log2 / exp2
//                     (bf16v2.py:225-244, detmath.py:20-106);
//   row fingerprint   FNV-style 64-bit hash per row for duplicate detection (bf16v2.py:148-155);
//   symbols           per weight: exponent (context: the predicted level rfi + cfi, 512), mantissa
//                     (context: 8 exponent - prediction, 128), sign (context: scl, 16), into tables
//                     shared by a role (bf16v2.py:54-75);
//   rANS              segments of 16384 weights, PB = 15, coded backwards (bf16v2.py:77-137).
//
// Mapping on the MI355X:
//   * row statistics: one lane per row, the rows staged through LDS in 64 x 64 tiles so the loads
//     stay coalesced while each lane sums its own row in index order (float64);
//   * column statistics: one lane per column (loads coalesced across the lanes), chunks of rows
//     summed as the reference's 16M-weight chunks are;
//   * histogram: weight-parallel (a workgroup per segment), atomics aggregated across the wave for
//     the exponent and sign symbols;
//   * encode: the table lookups are independent of the coder state, so a weight-parallel pass
//     writes each symbol's (frequency << 16 | cumulative) word; the serial coder (one lane per
//     segment, as the format requires) then streams those words;
//   * decode: one lane per segment.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace spa {
namespace r2 {
namespace {

constexpr int PB = 15;
constexpr uint32_t PSCALE = 1u << PB;
constexpr uint32_t RANS_L = 1u << 23;
constexpr int SEG = 16384;
constexpr int K = 8;

struct TB { int64_t doff; int32_t rowlen, rowbase, colbase, tab, rmap, pad; };   // bf16v2.py:157 TB_DT
struct SG { int32_t t, n; int64_t i0; };                                         // bf16v2.py:158 SG_DT
static_assert(sizeof(TB) == 32 && sizeof(SG) == 16, "descriptor layout");

// ---- detmath: float64 log2 / exp2 from IEEE basic operations only (detmath.py:20-58)
__device__ __forceinline__ double dm_rint(double x) {
    if (!(fabs(x) < 4503599627370496.0)) return x;
    double y = fabs(x) + 4503599627370496.0;
    y = y - 4503599627370496.0;
    return copysign(y, x);
}

__device__ double dm_log2(double x) {
    if (isnan(x)) return x;
    if (x < 0.0) return __longlong_as_double(0x7ff8000000000000LL);
    if (x == 0.0) return __longlong_as_double((long long)0xfff0000000000000ULL);
    if (isinf(x)) return x;
    long long u = __double_as_longlong(x);
    int e = (int)((u >> 52) & 0x7ff);
    if (e == 0) {                               // subnormal: scaled by 2^54
        x = x * 18014398509481984.0;
        u = __double_as_longlong(x);
        e = (int)((u >> 52) & 0x7ff) - 54;
    }
    e -= 1023;
    double m = __longlong_as_double((u & 0x000fffffffffffffLL) | 0x3ff0000000000000LL);
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0), z = s * s;     // ln m = 2 atanh s
    constexpr double C[12] = {0.043478260869565216, 0.047619047619047616, 0.05263157894736842, 0.058823529411764705,
                              0.06666666666666667,  0.07692307692307693,  0.09090909090909091, 0.1111111111111111,
                              0.14285714285714285,  0.2,                  0.3333333333333333,  1.0};
    double p = 0.04;
#pragma unroll
    for (int i = 0; i < 12; ++i) p = p * z + C[i];
    return (double)e + (2.0 * s * p) * 1.4426950408889634;
}

__device__ double dm_exp2(double y) {
    if (isnan(y)) return y;
    if (y >= 1024.0) return __longlong_as_double(0x7ff0000000000000LL);
    if (y < -1075.0) return 0.0;
    const double n = dm_rint(y), t = (y - n) * 0.6931471805599453;
    constexpr double C[17] = {4.779477332387385e-14,  7.647163731819816e-13, 1.1470745597729725e-11, 1.6059043836821613e-10,
                              2.08767569878681e-09,   2.505210838544172e-08, 2.7557319223985893e-07, 2.755731922398589e-06,
                              2.48015873015873e-05,   0.0001984126984126984, 0.001388888888888889,   0.008333333333333333,
                              0.041666666666666664,   0.16666666666666666,   0.5,                    1.0,
                              1.0};
    double p = 2.8114572543455206e-15;
#pragma unroll
    for (int i = 0; i < 17; ++i) p = p * t + C[i];
    const int k = (int)n, k1 = k / 2, k2 = k - k1;
    return p * __longlong_as_double((long long)(k1 + 1023) << 52) * __longlong_as_double((long long)(k2 + 1023) << 52);
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ int16_t to_i16(double v) {
    // clip(rint(v), -32768, 32767) as int16 (NaN, which the statistics do not produce, maps to 0)
    const double r = rint(v);
    return (int16_t)(r < -32768.0 ? -32768 : (r > 32767.0 ? 32767 : (r == r ? (int)r : 0)));
}

// ---- row statistics and fingerprints: 64 rows per workgroup, 64 x 64 tiles through LDS
constexpr int RT = 64;
__global__ __launch_bounds__(RT) void k_rows(const uint16_t* __restrict__ w, int64_t nr, int rl, int16_t* __restrict__ rfi,
                                             float* __restrict__ rfa, uint64_t* __restrict__ hash, double* __restrict__ rf_out) {
    __shared__ uint16_t tile[RT][RT + 2];
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * RT, row = r0 + lane;
    double s = 0.0;
    uint64_t h = 1469598103934665603ull;
    for (int c0 = 0; c0 < rl; c0 += RT) {
        const int nc = rl - c0 < RT ? rl - c0 : RT;
        for (int i = 0; i < RT; ++i) {
            const int64_t r = r0 + i;
            if (r < nr && lane < nc) tile[i][lane] = w[r * rl + c0 + lane];
        }
        __syncthreads();
        if (row < nr) {
            for (int j = 0; j < nc; ++j) {
                const uint32_t u = tile[lane][j];
                const double v = (double)__uint_as_float(u << 16);
                s = s + v * v;
                h ^= u;
                h *= 1099511628211ull;
                h ^= h >> 29;
            }
        }
        __syncthreads();
    }
    if (row < nr) {
        const double rf = dm_log2(sqrt(s / (double)rl) + 1e-30);
        rfi[row] = to_i16(rf * K);
        rfa[row] = (float)dm_exp2(rf);
        if (hash) hash[row] = h;
        if (rf_out) rf_out[row] = rf;
    }
}

// ---- column statistics: one lane per column, rows in chunks of `step` (bf16v2.py:234-238)
__global__ __launch_bounds__(256) void k_cols(const uint16_t* __restrict__ w, int64_t nr, int rl, int64_t step,
                                              const float* __restrict__ rfa, int16_t* __restrict__ cfi, int8_t* __restrict__ scl) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= rl) return;
    double s2 = 0.0, s1 = 0.0;
    for (int64_t r0 = 0; r0 < nr; r0 += step) {
        const int64_t r1 = r0 + step < nr ? r0 + step : nr;
        double c2 = 0.0, c1 = 0.0;
        for (int64_t r = r0; r < r1; ++r) {
            const float x = __uint_as_float((uint32_t)w[r * rl + c] << 16) / rfa[r];
            const double v = (double)x;
            c2 = c2 + v * v;
            c1 = c1 + v;
        }
        s2 = s2 + c2;
        s1 = s1 + c1;
    }
    const double cf = dm_log2(sqrt(s2 / (double)nr) + 1e-30);
    const int16_t ci = to_i16(cf * K);
    cfi[c] = ci;
    const double bias = (s1 / (double)nr) / dm_exp2((double)ci / K);
    const double fl = floor(bias * 16) + 8;
    scl[c] = (int8_t)(fl < 0.0 ? 0 : (fl > 15.0 ? 15 : (fl == fl ? (int)fl : 0)));
}

// ---- symbols
struct Ctx {
    int pe, rl, sc;
};
__device__ __forceinline__ void weight_at(const uint8_t* dev, const TB& T, const int32_t* rowmap, int64_t idx, int64_t& orow, int& j) {
    const int64_t rc = idx / T.rowlen;
    j = (int)(idx - rc * T.rowlen);
    orow = T.rmap >= 0 ? rowmap[T.rmap + rc] : rc;
}
__device__ __forceinline__ void contexts(const TB& T, int64_t orow, int j, uint32_t u, const int16_t* rfi, const int16_t* cfi,
                                         const int8_t* scl, int& ex, int& man, int& sgn, int& pe, int& rlc, int& sc) {
    ex = (u >> 7) & 255;
    man = u & 127;
    sgn = u >> 15;
    const int pred = rfi[T.rowbase + orow] + cfi[T.colbase + j];
    pe = clampi(pred + 256, 0, 511);
    rlc = clampi(8 * ex - pred - 1016 + 64, 0, 127);
    sc = scl[T.colbase + j];
}

// one workgroup per segment, weight-parallel
__global__ __launch_bounds__(256) void k_hist(const uint8_t* __restrict__ dev, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                              const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                              const int8_t* __restrict__ scl, const int32_t* __restrict__ rowmap,
                                              uint32_t* __restrict__ counts) {
    const SG g = sg[blockIdx.x];
    const TB T = tb[g.t];
    const uint16_t* W = reinterpret_cast<const uint16_t*>(dev + T.doff);
    for (int k0 = 0; k0 < g.n; k0 += 256) {
        const int k = k0 + threadIdx.x;
        const bool on = k < g.n;
        int ex = 0, man = 0, sgn = 0, pe = 0, rlc = 0, sc = 0;
        if (on) {
            int64_t orow;
            int j;
            weight_at(dev, T, rowmap, g.i0 + k, orow, j);
            contexts(T, orow, j, W[orow * T.rowlen + j], rfi, cfi, scl, ex, man, sgn, pe, rlc, sc);
        }
        if (on) atomicAdd(&counts[(uint32_t)(T.tab + 512 + rlc) * 256 + man], 1u);
        const uint32_t ke = on ? (uint32_t)(T.tab + pe) * 256 + ex : 0xffffffffu;
        const uint32_t ks = on ? (uint32_t)(T.tab + 640 + sc) * 256 + sgn : 0xffffffffu;
        // wave-aggregated adds for the concentrated exponent and sign symbols
        {
            uint64_t pending = __ballot(on);
            const int lane = __lane_id();
            while (pending) {
                const int leader = __ffsll((unsigned long long)pending) - 1;
                const uint32_t kk = __shfl(ke, leader);
                const uint64_t same = __ballot(ke == kk) & pending;
                if (lane == leader) atomicAdd(&counts[kk], (uint32_t)__popcll(same));
                pending &= ~same;
            }
            pending = __ballot(on);
            while (pending) {
                const int leader = __ffsll((unsigned long long)pending) - 1;
                const uint32_t kk = __shfl(ks, leader);
                const uint64_t same = __ballot(ks == kk) & pending;
                if (lane == leader) atomicAdd(&counts[kk], (uint32_t)__popcll(same));
                pending &= ~same;
            }
        }
    }
}

// the (freq << 16 | cum) word of each of a segment's symbols, in forward order, at fc + s * SEG * 3
__global__ __launch_bounds__(256) void k_fc(const uint8_t* __restrict__ dev, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                            const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                            const int8_t* __restrict__ scl, const int32_t* __restrict__ rowmap,
                                            const int32_t* __restrict__ remap, const uint16_t* __restrict__ freq,
                                            const uint32_t* __restrict__ cum, uint32_t* __restrict__ fc) {
    const SG g = sg[blockIdx.x];
    const TB T = tb[g.t];
    const uint16_t* W = reinterpret_cast<const uint16_t*>(dev + T.doff);
    uint32_t* o = fc + (int64_t)blockIdx.x * SEG * 3;
    for (int k = threadIdx.x; k < g.n; k += 256) {
        int64_t orow;
        int j, ex, man, sgn, pe, rlc, sc;
        weight_at(dev, T, rowmap, g.i0 + k, orow, j);
        contexts(T, orow, j, W[orow * T.rowlen + j], rfi, cfi, scl, ex, man, sgn, pe, rlc, sc);
        const int t0 = remap[T.tab + pe], t1 = remap[T.tab + 512 + rlc], t2 = remap[T.tab + 640 + sc];
        o[3 * k + 0] = ((uint32_t)freq[t0 * 256 + ex] << 16) | cum[t0 * 257 + ex];
        o[3 * k + 1] = ((uint32_t)freq[t1 * 256 + man] << 16) | cum[t1 * 257 + man];
        o[3 * k + 2] = ((uint32_t)freq[t2 * 256 + sgn] << 16) | cum[t2 * 257 + sgn];
    }
}

// one lane per segment: the words coded backwards (sign, mantissa, exponent of the last weight
// first), 4-byte flush
__global__ __launch_bounds__(64) void k_enc(const SG* __restrict__ sg, int nseg, const uint32_t* __restrict__ fc,
                                            uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int n3 = 3 * sg[s].n;
    const uint32_t* in = fc + (int64_t)s * SEG * 3;
    uint8_t* const start = out + (uint64_t)s * cap;
    uint8_t* const end = start + cap;
    uint8_t* ptr = end;
    uint32_t x = RANS_L;
    for (int i = n3 - 1; i >= 0; --i) {
        const uint32_t wd = in[i];
        const uint32_t f = wd >> 16, c = wd & 0xffffu;
        const uint32_t xm = ((RANS_L >> PB) << 8) * f;
        while (x >= xm) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
        x = ((x / f) << PB) + (x % f) + c;
        if (ptr - start < 64) { out_len[s] = 0xffffffffu; return; }
    }
    for (int i = 0; i < 4; ++i) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
    out_len[s] = (uint32_t)(end - ptr);
}

__global__ __launch_bounds__(64) void k_dec(const uint8_t* __restrict__ in, const uint64_t* __restrict__ in_off,
                                            uint8_t* __restrict__ dev, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                            int nseg, const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                            const int8_t* __restrict__ scl, const int32_t* __restrict__ rowmap,
                                            const int32_t* __restrict__ remap, const uint16_t* __restrict__ freq,
                                            const uint32_t* __restrict__ cum, const uint8_t* __restrict__ lut) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const SG g = sg[s];
    const TB T = tb[g.t];
    uint16_t* W = reinterpret_cast<uint16_t*>(dev + T.doff);
    const uint8_t* ptr = in + in_off[s];
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) x = (x << 8) | *ptr++;
    auto get = [&](int tab) {
        const int tt = remap[tab] < 0 ? 0 : remap[tab];            // unused contexts only on damaged streams
        const uint32_t slot = x & (PSCALE - 1);
        const int v = lut[(size_t)tt * PSCALE + slot];
        x = freq[tt * 256 + v] * (x >> PB) + slot - cum[tt * 257 + v];
        // a valid stream needs at most two bytes here; the cap ends the loop on a damaged one
#pragma unroll
        for (int i = 0; i < 4 && x < RANS_L; ++i) x = (x << 8) | *ptr++;
        return v;
    };
    for (int k = 0; k < g.n; ++k) {
        int64_t orow;
        int j;
        weight_at(dev, T, rowmap, g.i0 + k, orow, j);
        const int pred = rfi[T.rowbase + orow] + cfi[T.colbase + j];
        const int pe = clampi(pred + 256, 0, 511);
        const int ex = get(T.tab + pe);
        const int rlc = clampi(8 * ex - pred - 1016 + 64, 0, 127);
        const int man = get(T.tab + 512 + rlc);
        const int sgn = get(T.tab + 640 + scl[T.colbase + j]);
        W[orow * T.rowlen + j] = (uint16_t)((sgn << 15) | (ex << 7) | man);
    }
}

// rows[pairs[2i]] = rows[pairs[2i+1]] (duplicate rows from their source), one workgroup per pair
__global__ __launch_bounds__(256) void k_copy_rows(uint16_t* __restrict__ w, int rl, const int64_t* __restrict__ pairs, int n) {
    const int p = blockIdx.x;
    if (p >= n) return;
    const int64_t d = pairs[2 * p], s = pairs[2 * p + 1];
    for (int j = threadIdx.x; j < rl; j += 256) w[d * rl + j] = w[s * rl + j];
}

__global__ __launch_bounds__(256) void k_lut(const uint32_t* __restrict__ cum, int ntab, int pb, uint8_t* __restrict__ lut) {
    const int tb = blockIdx.x;
    if (tb >= ntab) return;
    for (int sym = threadIdx.x; sym < 256; sym += blockDim.x)
        for (uint32_t i = cum[tb * 257 + sym]; i < cum[tb * 257 + sym + 1]; ++i) lut[((size_t)tb << pb) + i] = (uint8_t)sym;
}

}  // namespace
}  // namespace r2
}  // namespace spa

using spa::fail;
using namespace spa::r2;

extern "C" {

int spa_r2_stats(const void* w, int64_t nrows, int rowlen, int16_t* rfi, int16_t* cfi, int8_t* scl, uint64_t* row_hash,
                 float* rfa_work, double* rf_out, void* stream) {
    if (nrows <= 0 || rowlen <= 0) return fail(SPA_ERR_ARG, "spa_r2_stats: empty tensor");
    if (!w || !rfi || !cfi || !scl || !rfa_work) return fail(SPA_ERR_ARG, "spa_r2_stats: null pointer");
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_rows, dim3((unsigned)((nrows + RT - 1) / RT)), dim3(RT), 0, st, (const uint16_t*)w, nrows, rowlen, rfi,
                       rfa_work, row_hash, rf_out);
    const int64_t step = (16 << 20) / rowlen > 0 ? (16 << 20) / rowlen : 1;
    hipLaunchKernelGGL(k_cols, dim3((unsigned)((rowlen + 255) / 256)), dim3(256), 0, st, (const uint16_t*)w, nrows, rowlen, step,
                       (const float*)rfa_work, cfi, scl);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_hist(const void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                const int8_t* scl, const int32_t* rowmap, uint32_t* counts, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_r2_hist: negative segment count");
    if (nseg == 0) return SPA_OK;
    hipLaunchKernelGGL(k_hist, dim3((unsigned)nseg), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)dev, (const TB*)tb,
                       (const SG*)sg, rfi, cfi, scl, rowmap, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_encode(const void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                  const int8_t* scl, const int32_t* rowmap, const int32_t* remap, const uint16_t* freq, const uint32_t* cum,
                  uint32_t* fc_work, void* out, uint64_t cap, uint32_t* out_len, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_r2_encode: negative segment count");
    if (cap < 1024) return fail(SPA_ERR_ARG, "spa_r2_encode: segment capacity %llu too small", (unsigned long long)cap);
    if (nseg == 0) return SPA_OK;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_fc, dim3((unsigned)nseg), dim3(256), 0, st, (const uint8_t*)dev, (const TB*)tb, (const SG*)sg, rfi, cfi,
                       scl, rowmap, remap, freq, cum, fc_work);
    hipLaunchKernelGGL(k_enc, dim3((unsigned)((nseg + 63) / 64)), dim3(64), 0, st, (const SG*)sg, nseg, (const uint32_t*)fc_work,
                       (uint8_t*)out, cap, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_decode(const void* in, const uint64_t* in_off, void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi,
                  const int16_t* cfi, const int8_t* scl, const int32_t* rowmap, const int32_t* remap, const uint16_t* freq,
                  const uint32_t* cum, const uint8_t* lut, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_r2_decode: negative segment count");
    if (nseg == 0) return SPA_OK;
    hipLaunchKernelGGL(k_dec, dim3((unsigned)((nseg + 63) / 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)in, in_off,
                       (uint8_t*)dev, (const TB*)tb, (const SG*)sg, nseg, rfi, cfi, scl, rowmap, remap, freq, cum, lut);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_copy_rows(void* w, int rowlen, const int64_t* pairs, int npairs, void* stream) {
    if (npairs < 0 || rowlen <= 0) return fail(SPA_ERR_ARG, "spa_r2_copy_rows: bad arguments");
    if (npairs == 0) return SPA_OK;
    hipLaunchKernelGGL(k_copy_rows, dim3((unsigned)npairs), dim3(256), 0, (hipStream_t)stream, (uint16_t*)w, rowlen, pairs, npairs);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_rans_build_lut_pb(const uint32_t* cum, int ntab, int pb, uint8_t* lut, void* stream) {
    if (pb < 1 || pb > 16) return fail(SPA_ERR_ARG, "spa_rans_build_lut_pb: precision %d", pb);
    if (ntab <= 0) return SPA_OK;
    hipLaunchKernelGGL(k_lut, dim3((unsigned)ntab), dim3(256), 0, (hipStream_t)stream, cum, ntab, pb, lut);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
