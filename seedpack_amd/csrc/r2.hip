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
//   * histogram: weight-parallel, counted in LDS per workgroup (a run of segments) and flushed once
//     per bin with global atomics;
//   * encode: the table lookups are independent of the coder state, so a weight-parallel pass
//     writes each symbol's (frequency << 16 | cumulative) word; the serial coder (one lane per
//     segment, as the format requires) then streams those words;
//   * decode: one lane per segment.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "detmath.h"
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

using dm::dm_exp2;
using dm::dm_log2;
using dm::dm_rint;

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ int16_t to_i16(double v) {
    // clip(rint(v), -32768, 32767) as int16 (NaN, which the statistics do not produce, maps to 0)
    const double r = rint(v);
    return (int16_t)(r < -32768.0 ? -32768 : (r > 32767.0 ? 32767 : (r == r ? (int)r : 0)));
}

// ---- row statistics and fingerprints: a lane per row (its float64 sum and its hash run in index
// order), 64 rows per workgroup staged through LDS in 64 x 64 tiles. With 16-byte aligned rows the
// tile is read as 16-byte vectors (eight lanes per 128-byte row piece) and the next tile's loads are
// issued before the current tile is summed.
constexpr int RT = 64;
__device__ __forceinline__ void row_step(uint32_t u, double& s, uint64_t& h) {
    const double v = (double)__uint_as_float(u << 16);
    s = s + v * v;
    h ^= u;
    h *= 1099511628211ull;
    h ^= h >> 29;
}
__global__ __launch_bounds__(RT) void k_rows(const uint16_t* __restrict__ w, int64_t nr, int rl, int vec, int16_t* __restrict__ rfi,
                                             float* __restrict__ rfa, uint64_t* __restrict__ hash, double* __restrict__ rf_out) {
    __shared__ uint32_t tile[RT][RT / 2 + 1];
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * RT, row = r0 + lane;
    double s = 0.0;
    uint64_t h = 1469598103934665603ull;
    const int nfull = vec ? rl / RT : 0;                 // tiles read as vectors
    uint4 v[8];
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t r = r0 + (lane >> 3) + 8 * k;
            v[k] = r < nr ? *reinterpret_cast<const uint4*>(w + r * rl + c0 + (lane & 7) * 8) : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    if (nfull) load(0);
    for (int t = 0; t < nfull; ++t) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t* d = &tile[(lane >> 3) + 8 * k][(lane & 7) * 4];
            d[0] = v[k].x; d[1] = v[k].y; d[2] = v[k].z; d[3] = v[k].w;
        }
        __syncthreads();
        if (t + 1 < nfull) load((t + 1) * RT);
        if (row < nr) {
#pragma unroll 8
            for (int j = 0; j < RT / 2; ++j) {
                const uint32_t pr = tile[lane][j];
                row_step(pr & 0xFFFFu, s, h);
                row_step(pr >> 16, s, h);
            }
        }
    }
    uint16_t* t16 = reinterpret_cast<uint16_t*>(&tile[0][0]);
    for (int c0 = nfull * RT; c0 < rl; c0 += RT) {       // rows not 16-byte aligned, and the last partial tile
        const int nc = rl - c0 < RT ? rl - c0 : RT;
        __syncthreads();
        for (int i = 0; i < RT; ++i) {
            const int64_t r = r0 + i;
            if (r < nr && lane < nc) t16[i * (RT + 2) + lane] = w[r * rl + c0 + lane];
        }
        __syncthreads();
        if (row < nr)
            for (int j = 0; j < nc; ++j) row_step(t16[lane * (RT + 2) + j], s, h);
    }
    if (row < nr) {
        const double rf = dm_log2(sqrt(s / (double)rl) + 1e-30);
        rfi[row] = to_i16(rf * K);
        rfa[row] = (float)dm_exp2(rf);
        if (hash) hash[row] = h;
        if (rf_out) rf_out[row] = rf;
    }
}

// ---- column statistics (bf16v2.py:234-238): the reference adds each chunk's column sums, taken
// in row order, to running totals in chunk order. The chunks are independent, so one launch takes
// every (chunk, column) pair, a lane summing its column over the chunk's rows with 32 rows'
// loads issued ahead of their adds; a second pass adds the chunk sums in order per column.
constexpr int CPF = 32;
__global__ __launch_bounds__(256) void k_cols_part(const uint16_t* __restrict__ w, int64_t nr, int rl, int64_t step,
                                                   int64_t nch, const float* __restrict__ rfa, double* __restrict__ part) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= rl) return;
    for (int64_t ch = blockIdx.y; ch < nch; ch += gridDim.y) {
        const int64_t r0 = ch * step, r1 = r0 + step < nr ? r0 + step : nr;
        double c2 = 0.0, c1 = 0.0;
        int64_t r = r0;
        for (; r + CPF <= r1; r += CPF) {
            uint32_t u[CPF];
            float a[CPF];
#pragma unroll
            for (int i = 0; i < CPF; ++i) {
                u[i] = w[(r + i) * rl + c];
                a[i] = rfa[r + i];
            }
#pragma unroll
            for (int i = 0; i < CPF; ++i) {
                const double v = (double)(__uint_as_float(u[i] << 16) / a[i]);
                c2 = c2 + v * v;
                c1 = c1 + v;
            }
        }
        for (; r < r1; ++r) {
            const double v = (double)(__uint_as_float((uint32_t)w[r * rl + c] << 16) / rfa[r]);
            c2 = c2 + v * v;
            c1 = c1 + v;
        }
        part[(ch * 2) * rl + c] = c2;
        part[(ch * 2 + 1) * rl + c] = c1;
    }
}

__global__ __launch_bounds__(256) void k_cols_fin(const double* __restrict__ part, int64_t nch, int64_t nr, int rl,
                                                  int16_t* __restrict__ cfi, int8_t* __restrict__ scl) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= rl) return;
    double s2 = 0.0, s1 = 0.0;
    for (int64_t ch = 0; ch < nch; ++ch) {
        s2 = s2 + part[(ch * 2) * rl + c];
        s1 = s1 + part[(ch * 2 + 1) * rl + c];
    }
    const double cf = dm_log2(sqrt(s2 / (double)nr) + 1e-30);
    const int16_t ci = to_i16(cf * K);
    cfi[c] = ci;
    const double bias = (s1 / (double)nr) / dm_exp2((double)ci / K);
    const double fl = floor(bias * 16) + 8;
    scl[c] = (int8_t)(fl < 0.0 ? 0 : (fl > 15.0 ? 15 : (fl == fl ? (int)fl : 0)));
}

// workspace of the statistics: the rows' float scales, then the chunk sums (2 doubles per chunk and column)
__host__ __device__ inline int64_t stats_step(int rl) { return (16 << 20) / rl > 0 ? (16 << 20) / rl : 1; }
inline uint64_t stats_rfa_bytes(int64_t nr) { return ((uint64_t)nr * 4 + 255) / 256 * 256; }
inline uint64_t stats_work_bytes(int64_t nr, int rl) {
    const int64_t nch = (nr + stats_step(rl) - 1) / stats_step(rl);
    return stats_rfa_bytes(nr) + (uint64_t)nch * 2 * (uint64_t)rl * 8;
}

// ---- symbols
// Position of a coded weight: compact row rc and column j (a segment's weights run along the compact
// rows, duplicate rows left out). Set once per thread and segment, then stepped; the division only
// runs when a step crosses a row end.
struct Cursor {
    int64_t rc;
    int j;
    __device__ __forceinline__ void start(int64_t idx, int rl) {
        rc = idx / rl;
        j = (int)(idx - rc * rl);
    }
    __device__ __forceinline__ void step(int s, int rl) {
        j += s;
        if (j >= rl) {
            const int q = j / rl;
            rc += q;
            j -= q * rl;
        }
    }
};
__device__ __forceinline__ int64_t orig_row(const TB& T, const int32_t* rowmap, int64_t rc) {
    return T.rmap >= 0 ? rowmap[T.rmap + rc] : rc;
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

// Histogram: a workgroup takes a run of consecutive segments and counts into LDS (mantissa 128 x 128,
// a window of HEW exponent contexts starting at the tensor's TB.pad, sign 16 x 2), flushing the
// non-zero bins with global atomics when the table block (role, window) changes and at the end.
// Exponent contexts outside the window count straight into global memory, so any window base gives
// the same counts.
constexpr int HT = 1024;            // threads per histogram workgroup
constexpr int HEW = 64;             // exponent contexts held in LDS

__device__ __forceinline__ void hist_flush(uint32_t* hm, uint32_t* he, uint32_t* hs, int tab, int pe0, uint32_t* counts) {
    for (int i = threadIdx.x; i < 128 * 128; i += HT) {
        const uint32_t v = hm[i];
        if (v) { atomicAdd(&counts[(uint32_t)(tab + 512 + (i >> 7)) * 256 + (i & 127)], v); hm[i] = 0; }
    }
    for (int i = threadIdx.x; i < HEW * 256; i += HT) {
        const uint32_t v = he[i];
        if (v) { atomicAdd(&counts[(uint32_t)(tab + pe0 + (i >> 8)) * 256 + (i & 255)], v); he[i] = 0; }
    }
    if (threadIdx.x < 32) {
        const uint32_t v = hs[threadIdx.x];
        if (v) { atomicAdd(&counts[(uint32_t)(tab + 640 + (threadIdx.x >> 1)) * 256 + (threadIdx.x & 1)], v); hs[threadIdx.x] = 0; }
    }
}

__global__ __launch_bounds__(HT) void k_hist(const uint8_t* __restrict__ dev, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                             int nseg, int spw, const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                             const int8_t* __restrict__ scl, const int32_t* __restrict__ rowmap,
                                             uint32_t* __restrict__ counts) {
    __shared__ uint32_t hm[128 * 128];
    __shared__ uint32_t he[HEW * 256];
    __shared__ uint32_t hs[32];
    for (int i = threadIdx.x; i < 128 * 128; i += HT) hm[i] = 0;
    for (int i = threadIdx.x; i < HEW * 256; i += HT) he[i] = 0;
    if (threadIdx.x < 32) hs[threadIdx.x] = 0;
    __syncthreads();
    const int s0 = blockIdx.x * spw, s1 = min(nseg, s0 + spw);
    int tab = -1, pe0 = 0;
    for (int s = s0; s < s1; ++s) {
        const SG g = sg[s];
        const TB T = tb[g.t];
        const int wpe = clampi(T.pad, 0, 512 - HEW);
        if (T.tab != tab || wpe != pe0) {
            if (tab >= 0) {
                __syncthreads();
                hist_flush(hm, he, hs, tab, pe0, counts);
                __syncthreads();
            }
            tab = T.tab;
            pe0 = wpe;
        }
        const uint16_t* W = reinterpret_cast<const uint16_t*>(dev + T.doff);
        Cursor cur;
        cur.start(g.i0 + threadIdx.x, T.rowlen);
        for (int k = threadIdx.x; k < g.n; k += HT, cur.step(HT, T.rowlen)) {
            int ex, man, sgn, pe, rlc, sc;
            const int64_t orow = orig_row(T, rowmap, cur.rc);
            const int j = cur.j;
            contexts(T, orow, j, W[orow * T.rowlen + j], rfi, cfi, scl, ex, man, sgn, pe, rlc, sc);
            atomicAdd(&hm[rlc * 128 + man], 1u);
            const int e = pe - pe0;
            if ((unsigned)e < (unsigned)HEW) atomicAdd(&he[e * 256 + ex], 1u);
            else atomicAdd(&counts[(uint32_t)(T.tab + pe) * 256 + ex], 1u);
            atomicAdd(&hs[sc * 2 + sgn], 1u);
        }
    }
    __syncthreads();
    if (tab >= 0) hist_flush(hm, he, hs, tab, pe0, counts);
}

// Per-context coding words: fcw[c][sym] = freq << 16 | cum of symbol sym in context c's table
// (c over roles x 656; contexts never coded hold zeros), so the symbol pass needs one load per
// symbol and no remap.
__global__ __launch_bounds__(256) void k_fcw(const int32_t* __restrict__ remap, const uint16_t* __restrict__ freq,
                                             const uint32_t* __restrict__ cum, uint32_t* __restrict__ fcw) {
    const int t = remap[blockIdx.x], i = threadIdx.x;
    fcw[(size_t)blockIdx.x * 256 + i] = t < 0 ? 0u : (((uint32_t)freq[(size_t)t * 256 + i] << 16) | cum[(size_t)t * 257 + i]);
}

// The coding word of every symbol, three per weight in forward order, for the coder. Layout: word i
// of batch segment s at fc[((s / 64) * 3 * SEG + i) * 64 + s % 64], so that the 64 lanes of an
// encoding wave read one 256-byte row per step. A workgroup takes 64 segments x FCK weights; lane l
// of wave v takes segment l's weights v*16 .. v*16+15 of the chunk (read as two 16-byte vectors, with
// their column side information, where rows are 16-weight aligned), its 48 words go to an LDS tile
// [word][segment] that is written out row by row.
constexpr int FCK = 64;
__global__ __launch_bounds__(256) void k_fc(const uint8_t* __restrict__ dev, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                            int nseg, const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                            const int8_t* __restrict__ scl, const int32_t* __restrict__ rowmap,
                                            const uint32_t* __restrict__ fcw, uint32_t* __restrict__ fc) {
    __shared__ uint32_t tile[3 * FCK][65];
    const int t = threadIdx.x, ls = t & 63, sub = t >> 6;
    const int s = blockIdx.x * 64 + ls;
    const int k0 = blockIdx.y * FCK + sub * 16;
    if (s < nseg) {
        const SG g = sg[s];
        if (k0 < g.n) {
            const TB T = tb[g.t];
            const uint16_t* W = reinterpret_cast<const uint16_t*>(dev + T.doff);
            const uint32_t* fw = fcw + (size_t)T.tab * 256;
            Cursor cur;
            cur.start(g.i0 + k0, T.rowlen);
            const int kn = g.n - k0 < 16 ? g.n - k0 : 16;
            auto words = [&](int q, uint32_t u, int pred, int scv) {
                const int ex = (u >> 7) & 255, man = u & 127, sgn = u >> 15;
                const int pe = clampi(pred + 256, 0, 511);
                const int rlc = clampi(8 * ex - pred - 1016 + 64, 0, 127);
                const int r = (sub * 16 + q) * 3;
                tile[r][ls] = fw[pe * 256 + ex];
                tile[r + 1][ls] = fw[(512 + rlc) * 256 + man];
                tile[r + 2][ls] = fw[(640 + scv) * 256 + sgn];
            };
            const bool vec = kn == 16 && (T.rowlen & 15) == 0 && (T.colbase & 15) == 0 && (cur.j & 15) == 0 &&
                             ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
            if (vec) {                           // 16 weights of one row
                const int64_t orow = orig_row(T, rowmap, cur.rc);
                const int rf = rfi[T.rowbase + orow];
                const uint4* wp = reinterpret_cast<const uint4*>(W + orow * T.rowlen + cur.j);
                const uint4* cp = reinterpret_cast<const uint4*>(cfi + T.colbase + cur.j);
                const uint4 w0 = wp[0], w1 = wp[1], c0 = cp[0], c1 = cp[1];
                const uint4 s16 = *reinterpret_cast<const uint4*>(scl + T.colbase + cur.j);
                const uint32_t wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                const uint32_t cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                const uint32_t sv[4] = {s16.x, s16.y, s16.z, s16.w};
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const uint32_t u = (wv[q >> 1] >> (16 * (q & 1))) & 0xFFFFu;
                    const int cfv = (int)(int16_t)(uint16_t)(cv[q >> 1] >> (16 * (q & 1)));
                    const int scv = (int)(int8_t)(uint8_t)(sv[q >> 2] >> (8 * (q & 3)));
                    words(q, u, rf + cfv, scv);
                }
            } else {
                for (int q = 0; q < kn; ++q, cur.step(1, T.rowlen)) {
                    const int64_t orow = orig_row(T, rowmap, cur.rc);
                    const int j = cur.j;
                    words(q, W[orow * T.rowlen + j], rfi[T.rowbase + orow] + cfi[T.colbase + j], scl[T.colbase + j]);
                }
            }
        }
    }
    __syncthreads();
    uint32_t* o = fc + ((int64_t)blockIdx.x * 3 * SEG + (int64_t)blockIdx.y * 3 * FCK) * 64;
    for (int i = t; i < 3 * FCK * 64; i += 256) o[i] = tile[i >> 6][i & 63];
}

// One lane per segment, a wave per 64 segments: the words coded backwards (sign, mantissa, exponent
// of the last weight first), the wave stepping down from its longest segment so that its lanes read
// one fc row per step; a lane's output bytes are packed four to a dword and stored downwards from
// the end of its slot (cap bytes, a multiple of 4); 4-byte flush.
__global__ __launch_bounds__(64) void k_enc(const SG* __restrict__ sg, int nseg, const uint32_t* __restrict__ fc,
                                            uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * 64 + threadIdx.x;
    const bool on = s < nseg;
    const int n3 = on ? 3 * sg[s].n : 0;
    int nmax = n3;
    for (int o = 32; o; o >>= 1) nmax = max(nmax, __shfl_xor(nmax, o));
    const uint32_t* in = fc + (int64_t)blockIdx.x * 3 * SEG * 64 + threadIdx.x;
    uint32_t* const start = reinterpret_cast<uint32_t*>(out + (uint64_t)(on ? s : 0) * cap);
    uint32_t* wp = start + cap / 4;
    uint32_t acc = 0, x = RANS_L, nbytes = 0;
    bool ovf = false;
    auto emit = [&](uint32_t v) {
        acc |= v << (8 * (3 - (nbytes & 3)));
        if ((++nbytes & 3) == 0) {
            *--wp = acc;
            acc = 0;
        }
    };
    // words loaded 16 at a time, one group ahead of the coding (their addresses do not depend on it)
    constexpr int PF = 16;
    uint32_t nxt[PF];
#pragma unroll
    for (int q = 0; q < PF; ++q) {
        const int ii = nmax - 1 - q;
        nxt[q] = (ii >= 0 && ii < n3) ? in[(int64_t)ii * 64] : 1u << 16;
    }
    for (int i0 = nmax - 1; i0 >= 0; i0 -= PF) {
        uint32_t cw[PF];
#pragma unroll
        for (int q = 0; q < PF; ++q) {
            cw[q] = nxt[q];
            const int ii = i0 - PF - q;
            nxt[q] = (ii >= 0 && ii < n3) ? in[(int64_t)ii * 64] : 1u << 16;
        }
#pragma unroll
        for (int q = 0; q < PF; ++q) {
            const int i = i0 - q;
            if (i >= 0 && i < n3 && !ovf) {
                const uint32_t f = cw[q] >> 16, c = cw[q] & 0xffffu;
                const uint32_t xm = ((RANS_L >> PB) << 8) * f;
                while (x >= xm) {
                    emit(x & 0xff);
                    x >>= 8;
                }
                x = ((x / f) << PB) + (x % f) + c;
                if (i % 3 == 0) ovf = nbytes > cap - 64;   // after each weight: under 64 bytes left (bf16v2.py:106)
            }
        }
    }
    if (!on) return;
    if (ovf) {
        out_len[s] = 0xffffffffu;
        return;
    }
    for (int i = 0; i < 4; ++i) {
        emit(x & 0xff);
        x >>= 8;
    }
    if (nbytes & 3) *--wp = acc;                 // its top bytes are the stream's first
    out_len[s] = nbytes;
}

// Decode tables, DT_BYTES per context (a role's 656 contexts side by side, so the decoder needs no
// remap): for each of the 256 slot buckets of 128 slots a u64, then every symbol's (cum | freq << 16)
// (u32). A bucket whose slots belong to at most two symbols s0 <= s1 holds them with the bounds
// c0 = cum[s0], c1 = end of s0 = cum[s1], c2 = end of s1:
//   s0 | s1 << 8 | c0 << 16 (15 bits) | c1 << 31 | c2 << 47, bit 63 clear,
// so one 8-byte load decodes the slot (s1 when slot >= c1, else s0). A bucket with slots of three or
// more symbols (only symbols of fewer than 128 slots make one) holds the first and last of them with
// the first one's cum and freq, first | (last - first) << 8 | cum << 16 | freq << 32, bit 63 set; a
// slot past the first symbol is then found by binary search over the bucket's other symbols. Every
// slot gets the symbol a full 2^15-entry lookup table gives; 3 KB per table instead of 32 KB.
// Contexts without a table (never coded) get a one-symbol table, reached only by damaged streams.
constexpr int DT_BYTES = 3072;
__device__ __forceinline__ int dec_sym(const uint8_t* dt, uint32_t slot, uint32_t& c0, uint32_t& f) {
    const uint64_t e = reinterpret_cast<const uint64_t*>(dt)[slot >> 7];
    if (!(e >> 63)) {
        const uint32_t c1 = (uint32_t)(e >> 31) & 0xFFFFu;
        const bool up = slot >= c1;
        c0 = up ? c1 : (uint32_t)(e >> 16) & 0x7FFFu;
        f = (up ? (uint32_t)(e >> 47) & 0xFFFFu : c1) - c0;
        return (int)(up ? (e >> 8) & 255u : e & 255u);
    }
    int s = (int)(e & 255u);
    c0 = (uint32_t)(e >> 16) & 0xFFFFu;
    f = (uint32_t)(e >> 32) & 0xFFFFu;
    const int span = (int)((e >> 8) & 255u);
    if (c0 + f <= slot) {
        // the last symbol in (first, last] whose cumulative frequency is <= slot
        const uint32_t* ps = reinterpret_cast<const uint32_t*>(dt + 2048);
        int lo = s + 1, hi = s + span;
        uint32_t u = ps[hi];
        if ((u & 0xFFFFu) > slot) {
            while (hi - lo > 0) {                 // invariant: cum[lo] <= slot < cum[hi]
                const int mid = (lo + hi + 1) >> 1;
                const uint32_t um = ps[mid];
                if ((um & 0xFFFFu) <= slot) lo = mid;
                else hi = mid - 1;
            }
            hi = lo;
            u = ps[lo];
        }
        s = hi;
        c0 = u & 0xFFFFu;
        f = u >> 16;
    }
    return s;
}

__global__ __launch_bounds__(256) void k_dtab(const uint32_t* __restrict__ cum, const int32_t* __restrict__ remap,
                                              uint8_t* __restrict__ dt) {
    __shared__ uint32_t ps[256];
    __shared__ uint32_t cs[257];
    const int t = remap[blockIdx.x];
    const uint32_t* c = cum + (size_t)(t < 0 ? 0 : t) * 257;
    uint8_t* o = dt + (size_t)blockIdx.x * DT_BYTES;
    const int i = threadIdx.x;
    // cum[0] is 0 and cum never falls (clamped to 16 bits), so every slot has a holder below
    for (int k = i; k < 257; k += 256) cs[k] = t < 0 || k == 0 ? (k ? 32768u : 0u) : (c[k] < 65535u ? c[k] : 65535u);
    __syncthreads();
    const uint32_t fi = cs[i + 1] > cs[i] ? cs[i + 1] - cs[i] : 0u;
    ps[i] = cs[i] | (fi << 16);
    reinterpret_cast<uint32_t*>(o + 2048)[i] = ps[i];
    // the symbol holding a slot: the last s <= 255 with cum[s] <= slot
    auto holder = [&](uint32_t slot) {
        int lo = 0, hi = 256;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (cs[mid] <= slot) lo = mid;
            else hi = mid;
        }
        return lo;
    };
    const int first = holder((uint32_t)i << 7), last = holder(((uint32_t)i << 7) + 127);
    // the second holder: the one of the first slot past the first symbol's (cum[first + 1] lies in
    // the bucket when last > first)
    const int second = last > first ? holder(cs[first + 1]) : first;
    uint64_t e;
    if (second == last) {
        e = (uint64_t)first | ((uint64_t)last << 8) | ((uint64_t)(cs[first] & 0x7FFFu) << 16) | ((uint64_t)cs[first + 1] << 31) |
            ((uint64_t)cs[last + 1] << 47);
    } else {
        const uint32_t u = ps[first];
        e = (uint64_t)first | ((uint64_t)(last - first) << 8) | ((uint64_t)(u & 0xFFFFu) << 16) | ((uint64_t)(u >> 16) << 32) |
            (1ull << 63);
    }
    reinterpret_cast<uint64_t*>(o)[i] = e;
}

// A lane's reader of its segment's bytes: a 16-byte window in registers refilled from the next
// aligned 16-byte block, which is already loaded (its load issued when the window was last refilled),
// so the coded stream is read once from HBM and its latency hides behind the decoding; blocks at or
// past `lim` (the stream's length rounded up to 16 bytes) read as zeros.
struct Reader {
    const uint4* p;
    const uint4* lim;
    uint4 w, nx;                                 // w.x holds the current dword; consumed dwords shift out
    int left, b;                                 // dwords left in the window, byte index in w.x
    __device__ __forceinline__ uint4 fetch() {
        const uint4 v = p < lim ? *p : make_uint4(0u, 0u, 0u, 0u);
        ++p;
        return v;
    }
    __device__ __forceinline__ void next_dword() {
        w.x = w.y;
        w.y = w.z;
        w.z = w.w;
        if (--left == 0) {
            w = nx;
            nx = fetch();
            left = 4;
        }
    }
    __device__ __forceinline__ void start(const uint8_t* base, uint64_t off, uint64_t nblocks) {
        p = reinterpret_cast<const uint4*>(base) + (off >> 4);
        lim = reinterpret_cast<const uint4*>(base) + nblocks;
        w = fetch();
        nx = fetch();
        left = 4;
        for (int q = (int)((off >> 2) & 3); q > 0; --q) next_dword();
        b = (int)(off & 3);
    }
    __device__ __forceinline__ uint32_t byte() {
        const uint32_t v = (w.x >> (8 * b)) & 0xFFu;
        if (++b == 4) {
            b = 0;
            next_dword();
        }
        return v;
    }
};

// One lane per segment (the format's unit of sequential decoding). Where rows and the column
// side information are 16-byte aligned (row length a multiple of 8), a lane decodes its weights in
// groups of 8: the group's cfi / scl read in one 16- and one 8-byte load, its 8 outputs written as
// one 16-byte store; otherwise weight by weight.
__global__ __launch_bounds__(256) void k_dec(const uint8_t* __restrict__ in, uint64_t in_blocks, const uint64_t* __restrict__ in_off,
                                             uint8_t* __restrict__ dev, const TB* __restrict__ tb, const SG* __restrict__ sg,
                                             int nseg, const int16_t* __restrict__ rfi, const int16_t* __restrict__ cfi,
                                             const int8_t* __restrict__ scl, const int32_t* __restrict__ rowmap,
                                             const uint8_t* __restrict__ dtab) {
    const int s = (int)(xcd_block(blockIdx.x, gridDim.x) * blockDim.x + threadIdx.x);
    if (s >= nseg) return;
    const SG g = sg[s];
    const TB T = tb[g.t];
    uint16_t* W = reinterpret_cast<uint16_t*>(dev + T.doff);
    Reader rd;
    rd.start(in, in_off[s], in_blocks);
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) x = (x << 8) | rd.byte();
    const uint8_t* dt = dtab + (size_t)T.tab * DT_BYTES;
    const int16_t* cf = cfi + T.colbase;
    const int8_t* sc = scl + T.colbase;
    auto get = [&](int ctx) {
        const uint32_t slot = x & (PSCALE - 1);
        uint32_t c0, f;
        const int v = dec_sym(dt + (size_t)ctx * DT_BYTES, slot, c0, f);
        x = f * (x >> PB) + slot - c0;
        // a valid stream needs at most two bytes here; the cap ends the loop on a damaged one
#pragma unroll
        for (int i = 0; i < 4 && x < RANS_L; ++i) x = (x << 8) | rd.byte();
        return v;
    };
    auto weight = [&](int pred, int scv) {
        const int ex = get(clampi(pred + 256, 0, 511));
        const int man = get(512 + clampi(8 * ex - pred - 1016 + 64, 0, 127));
        const int sgn = get(640 + scv);
        return (uint32_t)((sgn << 15) | (ex << 7) | man);
    };
    Cursor cur;
    cur.start(g.i0, T.rowlen);
    int64_t orow = orig_row(T, rowmap, cur.rc);
    int rf = rfi[T.rowbase + orow];
    uint16_t* Wr = W + orow * T.rowlen;
    const bool vec = (T.rowlen & 7) == 0 && (T.colbase & 7) == 0 && ((reinterpret_cast<uintptr_t>(W) & 15) == 0) &&
                     ((reinterpret_cast<uintptr_t>(cfi) & 15) == 0) && ((reinterpret_cast<uintptr_t>(scl) & 7) == 0);
    if (vec) {                                   // g.i0, g.n and the row length are multiples of 8
        // the group's column side information (loaded one group ahead) and outputs move through
        // 128-bit shift registers
        uint4 c8n = *reinterpret_cast<const uint4*>(cf + cur.j);
        uint2 s8n = *reinterpret_cast<const uint2*>(sc + cur.j);
        for (int k = 0; k < g.n; k += 8) {
            const int j = cur.j;
            uint4 c8 = c8n;
            uint64_t s64 = (uint64_t)s8n.x | ((uint64_t)s8n.y << 32);
            const int jn = j + 8 < T.rowlen ? j + 8 : 0;
            c8n = *reinterpret_cast<const uint4*>(cf + jn);
            s8n = *reinterpret_cast<const uint2*>(sc + jn);
            uint4 o = make_uint4(0u, 0u, 0u, 0u);
            for (int t = 0; t < 8; ++t) {
                const int cfv = (int)(int16_t)(uint16_t)c8.x;
                c8.x = (c8.x >> 16) | (c8.y << 16);
                c8.y = (c8.y >> 16) | (c8.z << 16);
                c8.z = (c8.z >> 16) | (c8.w << 16);
                c8.w >>= 16;
                const int scv = (int)(int8_t)(uint8_t)s64;
                s64 >>= 8;
                const uint32_t v = weight(rf + cfv, scv);
                o.x = (o.x >> 16) | (o.y << 16);
                o.y = (o.y >> 16) | (o.z << 16);
                o.z = (o.z >> 16) | (o.w << 16);
                o.w = (o.w >> 16) | (v << 16);
            }
            *reinterpret_cast<uint4*>(Wr + j) = o;
            cur.j += 8;
            if (cur.j == T.rowlen && k + 8 < g.n) {
                cur.j = 0;
                ++cur.rc;
                orow = orig_row(T, rowmap, cur.rc);
                rf = rfi[T.rowbase + orow];
                Wr = W + orow * T.rowlen;
            }
        }
        return;
    }
    for (int k = 0; k < g.n; ++k) {
        const int j = cur.j;
        Wr[j] = (uint16_t)weight(rf + cf[j], sc[j]);
        if (++cur.j == T.rowlen && k + 1 < g.n) {
            cur.j = 0;
            ++cur.rc;
            orow = orig_row(T, rowmap, cur.rc);
            rf = rfi[T.rowbase + orow];
            Wr = W + orow * T.rowlen;
        }
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

uint64_t spa_r2_stats_work_bytes(int64_t nrows, int rowlen) {
    return nrows > 0 && rowlen > 0 ? stats_work_bytes(nrows, rowlen) : 0;
}

int spa_r2_stats(const void* w, int64_t nrows, int rowlen, int16_t* rfi, int16_t* cfi, int8_t* scl, uint64_t* row_hash,
                 void* work, uint64_t work_bytes, double* rf_out, void* stream) {
    if (nrows <= 0 || rowlen <= 0) return fail(SPA_ERR_ARG, "spa_r2_stats: empty tensor");
    if (!w || !rfi || !cfi || !scl || !work) return fail(SPA_ERR_ARG, "spa_r2_stats: null pointer");
    if (work_bytes < stats_work_bytes(nrows, rowlen))
        return fail(SPA_ERR_ARG, "spa_r2_stats: workspace of %llu bytes, %llu needed", (unsigned long long)work_bytes,
                    (unsigned long long)stats_work_bytes(nrows, rowlen));
    hipStream_t st = (hipStream_t)stream;
    float* rfa = (float*)work;
    double* part = (double*)((uint8_t*)work + stats_rfa_bytes(nrows));
    const int vec = (rowlen % 8 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    hipLaunchKernelGGL(k_rows, dim3((unsigned)((nrows + RT - 1) / RT)), dim3(RT), 0, st, (const uint16_t*)w, nrows, rowlen, vec,
                       rfi, rfa, row_hash, rf_out);
    const int64_t step = stats_step(rowlen), nch = (nrows + step - 1) / step;
    const unsigned gx = (unsigned)((rowlen + 255) / 256), gy = (unsigned)(nch < 65535 ? nch : 65535);
    hipLaunchKernelGGL(k_cols_part, dim3(gx, gy), dim3(256), 0, st, (const uint16_t*)w, nrows, rowlen, step, nch,
                       (const float*)rfa, part);
    hipLaunchKernelGGL(k_cols_fin, dim3(gx), dim3(256), 0, st, (const double*)part, nch, nrows, rowlen, cfi, scl);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_hist(const void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                const int8_t* scl, const int32_t* rowmap, uint32_t* counts, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_r2_hist: negative segment count");
    if (nseg == 0) return SPA_OK;
    // about 512 workgroups (two per CU) however many segments, each a run of consecutive segments
    const int spw = (nseg + 511) / 512;
    hipLaunchKernelGGL(k_hist, dim3((unsigned)((nseg + spw - 1) / spw)), dim3(HT), 0, (hipStream_t)stream, (const uint8_t*)dev,
                       (const TB*)tb, (const SG*)sg, nseg, spw, rfi, cfi, scl, rowmap, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_encode_tables(const int32_t* remap, int nctx, const uint16_t* freq, const uint32_t* cum, uint32_t* fcw, void* stream) {
    if (nctx < 0) return fail(SPA_ERR_ARG, "spa_r2_encode_tables: negative context count");
    if (nctx == 0) return SPA_OK;
    hipLaunchKernelGGL(k_fcw, dim3((unsigned)nctx), dim3(256), 0, (hipStream_t)stream, remap, freq, cum, fcw);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_encode(const void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                  const int8_t* scl, const int32_t* rowmap, const uint32_t* fcw, uint32_t* fc_work, void* out, uint64_t cap,
                  uint32_t* out_len, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_r2_encode: negative segment count");
    if (cap < 1024 || cap % 16) return fail(SPA_ERR_ARG, "spa_r2_encode: segment capacity %llu (a multiple of 16, >= 1024)", (unsigned long long)cap);
    if (reinterpret_cast<uintptr_t>(out) & 15) return fail(SPA_ERR_ARG, "spa_r2_encode: output not 16-byte aligned");
    if (nseg == 0) return SPA_OK;
    hipStream_t st = (hipStream_t)stream;
    const unsigned ngrp = (unsigned)((nseg + 63) / 64);
    hipLaunchKernelGGL(k_fc, dim3(ngrp, SEG / FCK), dim3(256), 0, st, (const uint8_t*)dev, (const TB*)tb, (const SG*)sg, nseg, rfi,
                       cfi, scl, rowmap, fcw, fc_work);
    hipLaunchKernelGGL(k_enc, dim3(ngrp), dim3(64), 0, st, (const SG*)sg, nseg, (const uint32_t*)fc_work, (uint8_t*)out, cap,
                       out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_r2_decode(const void* in, uint64_t in_bytes, const uint64_t* in_off, void* dev, const void* tb, const void* sg, int nseg,
                  const int16_t* rfi, const int16_t* cfi, const int8_t* scl, const int32_t* rowmap, const uint8_t* dtab,
                  void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_r2_decode: negative segment count");
    if (nseg == 0) return SPA_OK;
    if (reinterpret_cast<uintptr_t>(in) & 15) return fail(SPA_ERR_ARG, "spa_r2_decode: stream not 16-byte aligned");
    hipLaunchKernelGGL(k_dec, dim3((unsigned)((nseg + 255) / 256)), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)in,
                       (in_bytes + 15) / 16, in_off, (uint8_t*)dev, (const TB*)tb, (const SG*)sg, nseg, rfi, cfi, scl, rowmap,
                       dtab);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

uint64_t spa_r2_dec_table_bytes(void) { return DT_BYTES; }

int spa_r2_build_dec_tables(const uint32_t* cum, const int32_t* remap, int nctx, uint8_t* dtab, void* stream) {
    if (nctx < 0) return fail(SPA_ERR_ARG, "spa_r2_build_dec_tables: negative context count");
    if (nctx == 0) return SPA_OK;
    hipLaunchKernelGGL(k_dtab, dim3((unsigned)nctx), dim3(256), 0, (hipStream_t)stream, cum, remap, dtab);
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
