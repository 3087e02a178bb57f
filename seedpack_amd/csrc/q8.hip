// M22: the reference's Q8_0 codec (seedpack/gpu2.py GPU2 + seedpack/gpu3.py GPU3 with the M22Fast
// settings; Q8Parts runs it per part of a file, SeedCodec per seed). Every Q8_0 block (fp16 d, 32
// int8 weights) is coded in up to three phases, each a set of rANS segments (PB 12, RANS_L 2^23,
// byte renormalisation, a segment coded backwards and ended by its 4-byte state):
//   A  per block: the scale's high byte (context: previous block's high byte, block-column factor
//      bin), low byte (context: high byte), the position of the largest |weight| as its rank among
//      the block's columns by column factor (context: spread of the factors), and its value
//      (context: the column's sign class); 4096 blocks per segment;
//   B  the other 31 weights: magnitude in 64 variance bins pbin(cfi[col], row mean - block scale
//      bits - tensor offset), sign in (bin, sign class); 1024 blocks per segment;
//   C  rows of token_embd predicted from up to 4 earlier similar rows (parents in earlier waves of
//      128): symbols (q - prediction) & 255 in bins shifted by the row's residual class, plus the
//      maximum's rank and value by the prediction; 4 rows per segment, decoded wave by wave.
// The planner of phase C (kNN by exact int8 similarities, least squares per row, residual column
// factors) is deterministic: float64 sums in index order, Gaussian elimination, detmath's log2.
//
// MI355X mapping: the per-phase coders are a lane per segment (the rANS state is serial), with the
// division-free encoder step (per-(table, symbol) reciprocals). Histograms of the per-weight phases
// are privatised in LDS per workgroup (one table set per work item), phase A's per-block symbols go
// to global atomics. The kNN search is an int8 MFMA GEMM (v_mfma_i32_32x32x32_i8, exact integer
// dot products) fused with a per-row top-4 merge through LDS, so the n x n similarity matrix never
// reaches HBM. The least-squares fit is a lane per row over the row and its four parents in one
// pass (all 15 float64 sums advance together, each in index order); the column sums of the
// statistics and of the residuals split rows into the reference's own slices and chunks, a thread
// per (column, slice), the slices summed in order on the host.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "detmath.h"
#include "launch.h"

namespace spa {
namespace q8 {
namespace {

constexpr uint32_t PB = 12, PSCALE = 1u << PB, RANS_L = 1u << 23;
constexpr int SEGA = 4096, SEGB = 1024;                       // gpu2.py:35-36
constexpr int A_HI = 0, A_LO = 256 * 16, A_POS = A_LO + 256, A_MX = A_POS + 16, TA = A_MX + 16;   // gpu2.py:47-51
constexpr int Q_SG = 64, TQ = 64 + 1024;                       // gpu2.py:52-53
constexpr int TPC = 64 + 24;                                   // gpu3.py:31 with PREDA
constexpr int KP = 4;                                          // parents per row (M21, gpu3.py:573)

struct Meta { int first, nblocks, nb_row, grp, colbase, rowbase, off, qset; };     // gpu2.py:278 META_DT
struct Item { int t, b0, nb; };                                 // histogram work: blocks [b0, b0+nb) of tensor t
struct CSeg { int t, r0, nr, slot; };                          // phase C segment (gpu3.py:321-335)
struct Slot { int64_t rbase, pbase; int first, nbr, mubase, pad; };   // a predicted tensor
static_assert(sizeof(Meta) == 32 && sizeof(Item) == 12 && sizeof(CSeg) == 16 && sizeof(Slot) == 32, "layouts");

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ int bits_of(const uint8_t* blk) { return blk[0] | (blk[1] << 8); }

__device__ __forceinline__ int tensor_of(const Meta* M, int ntens, int b) {
    int lo = 0, hi = ntens - 1;
    while (lo < hi) {
        const int m = (lo + hi + 1) >> 1;
        if (M[m].first <= b) lo = m; else hi = m - 1;
    }
    return lo;
}

__device__ __forceinline__ int pbin(int cf, int sh) {                 // gpu2.py:182-185
    const int u = (cf * 128 + sh) >> 7;
    return u < 0 ? 0 : (u > 63 ? 63 : u);
}

// ------------------------------------------------------------------ rANS
__device__ __forceinline__ uint32_t rcp_of(uint32_t f) {
    if (f < 2) return 0xffffffffu;
    const uint32_t sh = 32 - __clz(f - 1);
    return (uint32_t)(((1ull << (31 + sh)) + f - 1) / f);
}

__global__ __launch_bounds__(256) void k_rcp(const uint16_t* __restrict__ freq, int ntab, uint32_t* __restrict__ rcp) {
    const int tt = blockIdx.x;
    if (tt < ntab) rcp[tt * 256 + threadIdx.x] = rcp_of(freq[tt * 256 + threadIdx.x]);
}

// x -> C(s, x) = (x / f) * 2^PB + x % f + cum, the quotient by multiply-high (exact for x < 2^31)
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
    __device__ __forceinline__ uint32_t flush(uint8_t* end) {
        for (int i = 0; i < 4; ++i) { *--ptr = (uint8_t)(x & 0xff); x >>= 8; }
        return (uint32_t)(end - ptr);
    }
};

// The decoder's table: per (table, slot) one 32-bit word, symbol | (freq - 1) << 8 | (slot - cum) << 20,
// so that a step is one dependent load (the word) instead of two (symbol, then its freq and cum).
__global__ __launch_bounds__(256) void k_lut32(const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum, int ntab,
                                               uint32_t* __restrict__ lut) {
    const int tt = blockIdx.x;
    if (tt >= ntab) return;
    for (int s = threadIdx.x; s < 256; s += blockDim.x) {
        const uint32_t f = freq[tt * 256 + s], c = cum[tt * 257 + s];
        for (uint32_t k = 0; k < f; ++k) lut[(size_t)tt * PSCALE + c + k] = (uint32_t)s | ((f - 1) << 8) | (k << 20);
    }
}

// reads past the stream's end give zeros (a corrupt stream decodes to garbage inside the buffers)
struct Dec {
    uint32_t x;
    const uint8_t* ptr;
    const uint8_t* endp;
    const int* remap;
    const uint32_t* lut;
    __device__ __forceinline__ uint32_t byte() { const uint32_t b = ptr < endp ? *ptr : 0u; ++ptr; return b; }
    __device__ __forceinline__ void start(const uint8_t* in, uint64_t in_bytes, uint64_t off) {
        ptr = in + (off < in_bytes ? off : in_bytes);
        endp = in + in_bytes;
        x = 0;
        for (int i = 0; i < 4; ++i) x = (x << 8) | byte();
    }
    __device__ __forceinline__ int row(int tab) const { return max(remap[tab], 0); }   // < 0: only in a corrupt stream
    __device__ __forceinline__ int get(int tab) { return get_row(row(tab)); }
    __device__ __forceinline__ int get_row(int tt) {
        const uint32_t e = lut[(size_t)tt * PSCALE + (x & (PSCALE - 1))];
        x = ((e >> 8) & 4095u) * (x >> PB) + (x >> PB) + (e >> 20);     // freq * (x >> PB) + slot - cum
        while (x < RANS_L) x = (x << 8) | byte();
        return (int)(e & 255u);
    }
};

// ------------------------------------------------------------------ block statistics
__global__ __launch_bounds__(256) void k_pos(const uint8_t* __restrict__ blocks, int64_t n, uint8_t* __restrict__ pos) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n) return;
    const int8_t* q = reinterpret_cast<const int8_t*>(blocks + b * 34 + 2);
    int best = -1, p = 0;
    for (int j = 0; j < 32; ++j) {
        const int a = q[j] < 0 ? -q[j] : q[j];
        if (a > best) { best = a; p = j; }
    }
    pos[b] = (uint8_t)p;
}

// row_m[row] = (sum of the row's scale bits) // blocks per row (gpu2.py:555-558)
__global__ __launch_bounds__(256) void k_row_means(const uint8_t* __restrict__ blocks, const Meta* __restrict__ M, int ntens,
                                                   int64_t nrows, int* __restrict__ row_m) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= nrows) return;
    int lo = 0, hi = ntens - 1;
    while (lo < hi) {
        const int m = (lo + hi + 1) >> 1;
        if (M[m].rowbase <= r) lo = m; else hi = m - 1;
    }
    const Meta& T = M[lo];
    const int64_t b0 = T.first + (r - T.rowbase) * T.nb_row;
    int64_t s = 0;
    for (int k = 0; k < T.nb_row; ++k) s += bits_of(blocks + (b0 + k) * 34);
    row_m[r] = (int)(s / T.nb_row);
}

// rel[b] = float(exp2(float(bits - row mean) / 1024)): the block's scale relative to its row
__global__ __launch_bounds__(256) void k_rel(const uint8_t* __restrict__ blocks, int first, int nbr, int64_t nrows,
                                             const int* __restrict__ row_m, float* __restrict__ rel) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * nbr) return;
    const int dv = bits_of(blocks + ((int64_t)first + i) * 34) - row_m[i / nbr];
    rel[i] = (float)dm::dm_exp2((double)((float)dv / 1024.0f));
}

// part[s][c]: sums over the rows of slice s of w and w^2, w = float(q[r][c]) * rel[r][c / 32]
// (gpu2.py:588-597: detmath.cols of each slice of rows_per_slice rows)
__global__ __launch_bounds__(256) void k_col_stats(const uint8_t* __restrict__ blocks, int first, int nbr, int64_t nrows,
                                                   const float* __restrict__ rel, int64_t rows_per_slice,
                                                   double* __restrict__ p1, double* __restrict__ p2) {
    const int C = nbr * 32;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const int64_t r0 = (int64_t)blockIdx.y * rows_per_slice;
    const int64_t r1 = r0 + rows_per_slice < nrows ? r0 + rows_per_slice : nrows;
    const int kk = c >> 5, j = c & 31;
    double a = 0.0, b = 0.0;
    constexpr int AHEAD = 8;
    for (int64_t r = r0; r < r1; r += AHEAD) {
        float w[AHEAD];
#pragma unroll
        for (int u = 0; u < AHEAD; ++u) {
            const int64_t rr = r + u < r1 ? r + u : r1 - 1;
            const int64_t bi = rr * nbr + kk;
            w[u] = (float)(int8_t)blocks[((int64_t)first + bi) * 34 + 2 + j] * rel[bi];
        }
#pragma unroll
        for (int u = 0; u < AHEAD; ++u)
            if (r + u < r1) {
                const double v = (double)w[u];
                a = a + v;
                b = b + v * v;
            }
    }
    p1[blockIdx.y * (int64_t)C + c] = a;
    p2[blockIdx.y * (int64_t)C + c] = b;
}

// duplicate rows: h[r] = sum over the row's 64-bit words of word * mult[word] (mod 2^64)
__global__ __launch_bounds__(64) void k_row_hash(const uint8_t* __restrict__ blocks, int first, int nbr, int64_t nrows,
                                                 const uint64_t* __restrict__ mult, uint64_t* __restrict__ h) {
    const int64_t r = blockIdx.x;
    if (r >= nrows) return;
    const int nw = nbr * 34 / 8;
    const uint64_t* row = reinterpret_cast<const uint64_t*>(blocks + ((int64_t)first + r * nbr) * 34);
    uint64_t s = 0;
    for (int i = threadIdx.x; i < nw; i += 64) s += row[i] * mult[i];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (threadIdx.x == 0) h[r] = s;
}

__global__ __launch_bounds__(64) void k_rows_equal(const uint8_t* __restrict__ blocks, int first, int nbr,
                                                   const int* __restrict__ ra, const int* __restrict__ rb, int n,
                                                   uint8_t* __restrict__ eq) {
    const int i = blockIdx.x;
    if (i >= n) return;
    const int nb = nbr * 34;
    const uint8_t* a = blocks + ((int64_t)first + (int64_t)ra[i] * nbr) * 34;
    const uint8_t* b = blocks + ((int64_t)first + (int64_t)rb[i] * nbr) * 34;
    int diff = 0;
    for (int k = threadIdx.x; k < nb; k += 64) diff |= a[k] != b[k];
    diff = __any(diff);
    if (threadIdx.x == 0) eq[i] = diff ? 0 : 1;
}

// ------------------------------------------------------------------ phase A
struct AArgs {
    const uint8_t* skip; const Meta* M; int ntens, nblocks;
    const uint8_t *bcf, *spread, *perm, *rankof, *scls;
};

__device__ __forceinline__ void a_setup(const Meta& T, int b, int& inrow, int& cb, int& c0, int& base) {
    const int k = b - T.first;
    inrow = k % T.nb_row;
    cb = T.colbase / 32 + inrow;
    c0 = T.colbase + inrow * 32;
    base = T.grp * TA;
}

__global__ __launch_bounds__(64) void k_hist_a(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ pos, AArgs A,
                                               uint32_t* __restrict__ counts) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x, b0 = s * SEGA;
    if (b0 >= A.nblocks) return;
    const int b1 = min(b0 + SEGA, A.nblocks);
    int t = tensor_of(A.M, A.ntens, b0);
    for (int b = b0; b < b1; ++b) {
        while (t + 1 < A.ntens && b >= A.M[t + 1].first) ++t;
        if (A.skip[b] & 1) continue;
        int inrow, cb, c0, base;
        a_setup(A.M[t], b, inrow, cb, c0, base);
        const uint8_t* blk = blocks + (int64_t)b * 34;
        const int prev = (inrow == 0 || b == b0) ? 0 : blocks[(int64_t)(b - 1) * 34 + 1];
        const int hi = blk[1], p = pos[b];
        atomicAdd(&counts[(size_t)(base + A_HI + prev + 256 * A.bcf[cb]) * 256 + hi], 1u);
        atomicAdd(&counts[(size_t)(base + A_LO + hi) * 256 + blk[0]], 1u);
        if (!(A.skip[b] & 4)) {
            atomicAdd(&counts[(size_t)(base + A_POS + A.spread[cb]) * 256 + A.rankof[cb * 32 + p]], 1u);
            atomicAdd(&counts[(size_t)(base + A_MX + A.scls[c0 + p]) * 256 + blk[2 + p]], 1u);
        }
    }
}

__global__ __launch_bounds__(64) void k_enc_a(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ pos, AArgs A,
                                              const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                              const uint32_t* __restrict__ cum, const uint32_t* __restrict__ rcp,
                                              uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x, b0 = s * SEGA;
    if (b0 >= A.nblocks) return;
    const int b1 = min(b0 + SEGA, A.nblocks);
    int t = tensor_of(A.M, A.ntens, b1 - 1);
    uint8_t* const start = out + (uint64_t)s * cap;
    uint8_t* const end = start + cap;
    Enc e{RANS_L, end, remap, freq, cum, rcp};
    for (int b = b1 - 1; b >= b0; --b) {
        while (b < A.M[t].first) --t;
        if (A.skip[b] & 1) continue;
        int inrow, cb, c0, base;
        a_setup(A.M[t], b, inrow, cb, c0, base);
        const uint8_t* blk = blocks + (int64_t)b * 34;
        const int prev = (inrow == 0 || b == b0) ? 0 : blocks[(int64_t)(b - 1) * 34 + 1];
        const int hi = blk[1], p = pos[b];
        if (!(A.skip[b] & 4)) {
            e.put(base + A_MX + A.scls[c0 + p], blk[2 + p]);
            e.put(base + A_POS + A.spread[cb], A.rankof[cb * 32 + p]);
        }
        e.put(base + A_LO + hi, blk[0]);
        e.put(base + A_HI + prev + 256 * A.bcf[cb], hi);
        if (e.ptr - start < 16) { out_len[s] = 0xffffffffu; return; }
    }
    out_len[s] = e.flush(end);
}

__global__ __launch_bounds__(64) void k_dec_a(const uint8_t* __restrict__ in, uint64_t in_bytes,
                                              const uint64_t* __restrict__ in_off, AArgs A, const int* __restrict__ remap,
                                              const uint32_t* __restrict__ lut, uint8_t* __restrict__ blocks,
                                              uint8_t* __restrict__ pos) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x, b0 = s * SEGA;
    if (b0 >= A.nblocks) return;
    const int b1 = min(b0 + SEGA, A.nblocks);
    int t = tensor_of(A.M, A.ntens, b0);
    Dec d{0, nullptr, nullptr, remap, lut};
    d.start(in, in_bytes, in_off[s]);
    int prev = 0;
    for (int b = b0; b < b1; ++b) {
        while (t + 1 < A.ntens && b >= A.M[t + 1].first) ++t;
        if (A.skip[b] & 1) continue;
        int inrow, cb, c0, base;
        a_setup(A.M[t], b, inrow, cb, c0, base);
        uint8_t* blk = blocks + (int64_t)b * 34;
        if (inrow == 0 || b == b0) prev = 0;
        const int hi = d.get(base + A_HI + prev + 256 * A.bcf[cb]);
        const int lo = d.get(base + A_LO + hi);
        blk[0] = (uint8_t)lo;
        blk[1] = (uint8_t)hi;
        prev = hi;
        if (!(A.skip[b] & 4)) {
            const int r = d.get(base + A_POS + A.spread[cb]);
            const int p = A.perm[cb * 32 + (r & 31)];
            const int mx = d.get(base + A_MX + A.scls[c0 + p]);
            blk[2 + p] = (uint8_t)mx;
            pos[b] = (uint8_t)p;
        }
    }
}

// ------------------------------------------------------------------ phase B
struct BArgs {
    const uint8_t* skip; const Meta* M; int ntens, nblocks;
    const int16_t* cfi; const uint8_t* scls; const int* row_m; int qbase;
};

__device__ __forceinline__ int b_shift(const BArgs& B, const Meta& T, int b, const uint8_t* blk, int& c0) {
    const int k = b - T.first, inrow = k % T.nb_row;
    c0 = T.colbase + inrow * 32;
    const int rm = B.row_m[T.rowbase + k / T.nb_row];
    return rm - bits_of(blk) - T.off;
}

// a workgroup per work item (blocks of one tensor): counts of its table set in LDS
__global__ __launch_bounds__(256) void k_hist_b(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ pos, BArgs B,
                                                const Item* __restrict__ items, uint32_t* __restrict__ counts) {
    __shared__ uint32_t cm[64 * 256];
    __shared__ uint32_t cs[1024 * 2];
    for (int i = threadIdx.x; i < 64 * 256; i += 256) cm[i] = 0;
    for (int i = threadIdx.x; i < 2048; i += 256) cs[i] = 0;
    __syncthreads();
    const Item it = items[blockIdx.x];
    const Meta T = B.M[it.t];
    for (int i = threadIdx.x; i < it.nb; i += 256) {
        const int b = it.b0 + i;
        if (B.skip[b]) continue;
        const uint8_t* blk = blocks + (int64_t)b * 34;
        int c0;
        const int sh = b_shift(B, T, b, blk, c0), p = pos[b];
        for (int j = 0; j < 32; ++j) {
            if (j == p) continue;
            const int c = c0 + j, pb = pbin(B.cfi[c], sh), v = (int8_t)blk[2 + j];
            const int mag = v < 0 ? -v : v;
            atomicAdd(&cm[pb * 256 + mag], 1u);
            if (mag) atomicAdd(&cs[(pb * 16 + B.scls[c]) * 2 + (v < 0)], 1u);
        }
    }
    __syncthreads();
    const size_t qb = (size_t)B.qbase + (size_t)T.qset * TQ;
    for (int i = threadIdx.x; i < 64 * 256; i += 256)
        if (cm[i]) atomicAdd(&counts[(qb + i / 256) * 256 + (i % 256)], cm[i]);
    for (int i = threadIdx.x; i < 2048; i += 256)
        if (cs[i]) atomicAdd(&counts[(qb + Q_SG + i / 2) * 256 + (i % 2)], cs[i]);
}

__global__ __launch_bounds__(64) void k_enc_b(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ pos, BArgs B,
                                              const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                              const uint32_t* __restrict__ cum, const uint32_t* __restrict__ rcp,
                                              uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x, b0 = s * SEGB;
    if (b0 >= B.nblocks) return;
    const int b1 = min(b0 + SEGB, B.nblocks);
    int t = tensor_of(B.M, B.ntens, b1 - 1);
    uint8_t* const start = out + (uint64_t)s * cap;
    uint8_t* const end = start + cap;
    Enc e{RANS_L, end, remap, freq, cum, rcp};
    for (int b = b1 - 1; b >= b0; --b) {
        while (b < B.M[t].first) --t;
        if (B.skip[b]) continue;
        const uint8_t* blk = blocks + (int64_t)b * 34;
        int c0;
        const int sh = b_shift(B, B.M[t], b, blk, c0), p = pos[b];
        const int qb = B.qbase + B.M[t].qset * TQ;
        for (int j = 31; j >= 0; --j) {
            if (j == p) continue;
            const int c = c0 + j, pb = pbin(B.cfi[c], sh), v = (int8_t)blk[2 + j];
            const int mag = v < 0 ? -v : v;
            if (mag) e.put(qb + Q_SG + pb * 16 + B.scls[c], v < 0);
            e.put(qb + pb, (uint32_t)mag);
        }
        if (e.ptr - start < 160) { out_len[s] = 0xffffffffu; return; }
    }
    out_len[s] = e.flush(end);
}

__global__ __launch_bounds__(64) void k_dec_b(const uint8_t* __restrict__ in, uint64_t in_bytes,
                                              const uint64_t* __restrict__ in_off, BArgs B, const int* __restrict__ remap,
                                              const uint32_t* __restrict__ lut, uint8_t* __restrict__ blocks,
                                              const uint8_t* __restrict__ pos) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x, b0 = s * SEGB;
    if (b0 >= B.nblocks) return;
    const int b1 = min(b0 + SEGB, B.nblocks);
    int t = tensor_of(B.M, B.ntens, b0);
    const int16_t* __restrict__ cfi = B.cfi;
    const uint8_t* __restrict__ scls = B.scls;
    Dec d{0, nullptr, nullptr, remap, lut};
    d.start(in, in_bytes, in_off[s]);
    for (int b = b0; b < b1; ++b) {
        while (t + 1 < B.ntens && b >= B.M[t + 1].first) ++t;
        if (B.skip[b]) continue;
        uint8_t* blk = blocks + (int64_t)b * 34;
        int c0;
        const int sh = b_shift(B, B.M[t], b, blk, c0), p = pos[b];
        const int qb = B.qbase + B.M[t].qset * TQ;
        // the block's 31 magnitude and sign tables do not depend on the stream: looked up before the
        // serial steps, which then wait on one table load each
        int tm[32], ts[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int c = c0 + j, pb = pbin(cfi[c], sh);
            tm[j] = d.row(qb + pb);
            ts[j] = d.row(qb + Q_SG + pb * 16 + scls[c]);
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            if (j == p) continue;
            const int mag = d.get_row(tm[j]);
            const int sg = mag ? d.get_row(ts[j]) : 0;
            blk[2 + j] = (uint8_t)((sg ? -mag : mag) & 0xff);
        }
    }
}

// ------------------------------------------------------------------ row prediction (phase C)
__device__ __forceinline__ float h2f(uint32_t h) { return f16_to_f32(h); }

// w_hat = mu + sum_k coef_k (w[parent_k] - mu), then clip(rint(w_hat / d), -127, 127) for d > 0
// (gpu3.py:67-87: explicit IEEE operations, in parent order)
__device__ __forceinline__ int8_t pred1(const uint8_t* blocks, int first, int nbr, int r, int j, const int* par,
                                        const float* coef, const float* mu) {
    float acc = 0.0f;
    for (int k = 0; k < KP; ++k) {
        const int p = par[(size_t)r * KP + k];
        if (p < 0) continue;
        const uint8_t* pb = blocks + ((size_t)first + (size_t)p * nbr + j / 32) * 34;
        const float w = __fmul_rn((float)(int8_t)pb[2 + j % 32], h2f(bits_of(pb)));
        acc = __fadd_rn(acc, __fmul_rn(coef[(size_t)r * KP + k], __fsub_rn(w, mu[j])));
    }
    const float m = __fadd_rn(acc, mu[j]);
    const uint8_t* tb = blocks + ((size_t)first + (size_t)r * nbr + j / 32) * 34;
    const float d = h2f(bits_of(tb));
    int v = 0;
    if (d > 0.0f) {
        const float t = rintf(__fdiv_rn(m, d));
        v = (int)fmaxf(-127.0f, fminf(127.0f, t));
    }
    return (int8_t)v;
}

__global__ __launch_bounds__(256) void k_predict(const uint8_t* __restrict__ blocks, int first, int nbr, int64_t nrows,
                                                 const int* __restrict__ par, const float* __restrict__ coef,
                                                 const float* __restrict__ mu, int8_t* __restrict__ pint) {
    const int64_t C = (int64_t)nbr * 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * C) return;
    const int r = (int)(i / C), j = (int)(i % C);
    pint[i] = pred1(blocks, first, nbr, r, j, par, coef, mu);
}

// one wave of the decoder: entry e = row ent_row[e] of slot ent_slot[e] (gpu3.py:90-104)
__global__ __launch_bounds__(256) void k_predict_multi(const uint8_t* __restrict__ blocks, const int* __restrict__ ent_slot,
                                                       const int* __restrict__ ent_row, int nent, int cmax,
                                                       const Slot* __restrict__ slots, const int* __restrict__ par,
                                                       const float* __restrict__ coef, const float* __restrict__ mu,
                                                       int8_t* __restrict__ pint) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)nent * cmax) return;
    const int e = (int)(i / cmax), j = (int)(i % cmax);
    const Slot S = slots[ent_slot[e]];
    const int C = S.nbr * 32, r = ent_row[e];
    if (j >= C) return;
    pint[S.pbase + (int64_t)r * C + j] = pred1(blocks, S.first, S.nbr, r, j, par + S.rbase * KP, coef + S.rbase * KP,
                                               mu + S.mubase);
}

// The maximum's rank among the block's 32 predictions (|prediction| descending, ties by position) and
// the rank context min(max |prediction| / 16, 7) (gpu3.py:48-60), per block before the serial coders:
// prk[b][j] = rank of position j, pinv[b][rank] = position, rctx[b]. A workgroup per 8 blocks, a lane
// per (block, position) over the block's predictions in LDS.
__global__ __launch_bounds__(256) void k_ranks(const int8_t* __restrict__ pint, int64_t nblk, int8_t* __restrict__ prk,
                                               int8_t* __restrict__ pinv, int8_t* __restrict__ rctx) {
    __shared__ int a[256];
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int j = threadIdx.x & 31, base = threadIdx.x & ~31;
    const bool in = i < nblk * 32;
    const int v = in ? pint[i] : 0;
    a[threadIdx.x] = v < 0 ? -v : v;
    __syncthreads();
    if (!in) return;
    const int aj = a[threadIdx.x];
    int r = 0, m = 0;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int ak = a[base + k];
        r += (ak > aj) || (ak == aj && k < j);
        m = ak > m ? ak : m;
    }
    prk[i] = (int8_t)r;
    pinv[(i & ~(int64_t)31) + r] = (int8_t)j;
    if (j == 0) rctx[i >> 5] = (int8_t)min(m / 16, 7);
}

__device__ __forceinline__ int mx_ctx(const int8_t* pr, int p) { const int v = pr[p]; return (v < 0) * 8 + min(abs(v) / 16, 7); }

struct CArgs {
    const uint8_t* skip; const Meta* M; const CSeg* seg; int nseg; const Slot* slots;
    const int16_t* cfi; const int* row_m; const int8_t* fbin; const int8_t* pint;
    const int8_t* prk; const int8_t* pinv; const int8_t* rctx;       // k_ranks' tables, laid out as pint
};

__device__ __forceinline__ int c_ctx(int cf, int sh, int fb) { return clampi(pbin(cf, sh) + fb, 0, 63); }

// a workgroup per 16 segments; counts of the first segment's slot in LDS, other slots to global
constexpr int HC_SEGS = 16;
__global__ __launch_bounds__(256) void k_hist_c(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ pos, CArgs A,
                                                uint32_t* __restrict__ counts) {
    __shared__ uint32_t h[TPC * 256];
    for (int i = threadIdx.x; i < TPC * 256; i += 256) h[i] = 0;
    __syncthreads();
    const int s0 = blockIdx.x * HC_SEGS, s1 = min(s0 + HC_SEGS, A.nseg);
    const int lslot = A.seg[s0].slot;
    for (int s = s0; s < s1; ++s) {
        const CSeg g = A.seg[s];
        const Meta T = A.M[g.t];
        const Slot S = A.slots[g.slot];
        const int nbr = T.nb_row, C = nbr * 32;
        uint32_t* const gl = counts + (size_t)g.slot * TPC * 256;
        const bool local = g.slot == lslot;
        for (int i = threadIdx.x; i < g.nr * nbr; i += 256) {
            const int r = g.r0 + i / nbr, kk = i % nbr;
            const size_t b = (size_t)T.first + (size_t)r * nbr + kk;
            if (A.skip[b] & 1) continue;
            const uint8_t* blk = blocks + b * 34;
            const int sh = A.row_m[T.rowbase + r] - bits_of(blk) - T.off, p = pos[b];
            const size_t q0 = S.pbase + (size_t)r * C + kk * 32;
            const int8_t* pr = A.pint + q0;
            const int fb = A.fbin[S.rbase + r];
            int idx = (64 + A.rctx[q0 >> 5]) * 256 + A.prk[q0 + p];
            if (local) atomicAdd(&h[idx], 1u); else atomicAdd(&gl[idx], 1u);
            idx = (72 + mx_ctx(pr, p)) * 256 + blk[2 + p];
            if (local) atomicAdd(&h[idx], 1u); else atomicAdd(&gl[idx], 1u);
            for (int j = 0; j < 32; ++j) {
                if (j == p) continue;
                const int ctx = c_ctx(A.cfi[T.colbase + kk * 32 + j], sh, fb);
                idx = ctx * 256 + (((int8_t)blk[2 + j] - pr[j]) & 255);
                if (local) atomicAdd(&h[idx], 1u); else atomicAdd(&gl[idx], 1u);
            }
        }
    }
    __syncthreads();
    uint32_t* const gl = counts + (size_t)lslot * TPC * 256;
    for (int i = threadIdx.x; i < TPC * 256; i += 256)
        if (h[i]) atomicAdd(&gl[i], h[i]);
}

__global__ __launch_bounds__(64) void k_enc_c(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ pos, CArgs A,
                                              const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                              const uint32_t* __restrict__ cum, const uint32_t* __restrict__ rcp,
                                              uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= A.nseg) return;
    const CSeg g = A.seg[s];
    const Meta T = A.M[g.t];
    const Slot S = A.slots[g.slot];
    const int nbr = T.nb_row, C = nbr * 32, tb = g.slot * TPC;
    uint8_t* const start = out + (uint64_t)s * cap;
    uint8_t* const end = start + cap;
    Enc e{RANS_L, end, remap, freq, cum, rcp};
    for (int r = g.r0 + g.nr - 1; r >= g.r0; --r) {
        const int fb = A.fbin[S.rbase + r];
        for (int kk = nbr - 1; kk >= 0; --kk) {
            const size_t b = (size_t)T.first + (size_t)r * nbr + kk;
            if (A.skip[b] & 1) continue;
            const uint8_t* blk = blocks + b * 34;
            const int sh = A.row_m[T.rowbase + r] - bits_of(blk) - T.off, p = pos[b];
            const size_t q0 = S.pbase + (size_t)r * C + kk * 32;
            const int8_t* pr = A.pint + q0;
            for (int j = 31; j >= 0; --j) {
                if (j == p) continue;
                const int ctx = c_ctx(A.cfi[T.colbase + kk * 32 + j], sh, fb);
                e.put(tb + ctx, (uint32_t)(((int8_t)blk[2 + j] - pr[j]) & 255));
            }
            e.put(tb + 72 + mx_ctx(pr, p), blk[2 + p]);
            e.put(tb + 64 + A.rctx[q0 >> 5], (uint32_t)A.prk[q0 + p]);
            if (e.ptr - start < 160) { out_len[s] = 0xffffffffu; return; }
        }
    }
    out_len[s] = e.flush(end);
}

__global__ __launch_bounds__(64) void k_dec_c(const uint8_t* __restrict__ in, uint64_t in_bytes,
                                              const uint64_t* __restrict__ in_off, int seg0, int seg1, CArgs A,
                                              const int* __restrict__ remap, const uint32_t* __restrict__ lut,
                                              uint8_t* __restrict__ blocks, uint8_t* __restrict__ pos) {
    const int s = seg0 + blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= seg1) return;
    const CSeg g = A.seg[s];
    const Meta T = A.M[g.t];
    const Slot S = A.slots[g.slot];
    const int nbr = T.nb_row, C = nbr * 32, tb = g.slot * TPC;
    const int16_t* __restrict__ cfi = A.cfi;
    const int8_t* __restrict__ pint = A.pint;
    Dec d{0, nullptr, nullptr, remap, lut};
    d.start(in, in_bytes, in_off[s]);
    for (int r = g.r0; r < g.r0 + g.nr; ++r) {
        const int fb = A.fbin[S.rbase + r];
        for (int kk = 0; kk < nbr; ++kk) {
            const size_t b = (size_t)T.first + (size_t)r * nbr + kk;
            if (A.skip[b] & 1) continue;
            uint8_t* blk = blocks + b * 34;
            const int sh = A.row_m[T.rowbase + r] - bits_of(blk) - T.off;
            const size_t q0 = S.pbase + (size_t)r * C + kk * 32;
            // the block's predictions and its 31 residual tables, before the serial steps
            int4 pw[2];
            pw[0] = *reinterpret_cast<const int4*>(pint + q0);
            pw[1] = *reinterpret_cast<const int4*>(pint + q0 + 16);
            int tt[32];
#pragma unroll
            for (int j = 0; j < 32; ++j) tt[j] = d.row(tb + c_ctx(cfi[T.colbase + kk * 32 + j], sh, fb));
            const int rk = d.get(tb + 64 + A.rctx[q0 >> 5]);
            const int p = rk < 32 ? A.pinv[q0 + rk] : 0;          // a rank past 31: only in a corrupt stream
            const int mx = d.get(tb + 72 + mx_ctx(pint + q0, p));
            blk[2 + p] = (uint8_t)mx;
            pos[b] = (uint8_t)p;
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                if (j == p) continue;
                const int w = (j < 16 ? (&pw[0].x)[(j & 15) >> 2] : (&pw[1].x)[(j & 15) >> 2]);
                const int prj = (int)(int8_t)(w >> (8 * (j & 3)));
                const int sym = d.get_row(tt[j]);
                blk[2 + j] = (uint8_t)((prj + sym) & 255);
            }
        }
    }
}

// ------------------------------------------------------------------ planner (encoder only)
// W[r][c] = float(q) * float(d): exact (gpu3.py:263-270)
__global__ __launch_bounds__(256) void k_row_matrix(const uint8_t* __restrict__ blocks, int first, int nbr, int64_t nrows,
                                                    float* __restrict__ W) {
    const int64_t C = (int64_t)nbr * 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * C) return;
    const uint8_t* blk = blocks + ((int64_t)first + i / 32) * 34;
    W[i] = (float)(int8_t)blk[2 + (i & 31)] * h2f(bits_of(blk));
}

__global__ __launch_bounds__(256) void k_center(float* __restrict__ W, const float* __restrict__ mu, int64_t nrows, int C) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nrows * C) W[i] = __fsub_rn(W[i], mu[i % C]);
}

// Wq = clip(rint(x / nrm * 127), -127, 127) in float64, 0 for rows that are not valid (gpu3.py:289-295)
__global__ __launch_bounds__(256) void k_norm_i8(const float* __restrict__ W, const double* __restrict__ nrm,
                                                 const uint8_t* __restrict__ valid, int64_t nrows, int C,
                                                 int8_t* __restrict__ Wq) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * C) return;
    const int64_t r = i / C;
    int v = 0;
    if (valid[r]) {
        double t = rint((double)W[i] / nrm[r] * 127.0);
        t = t < -127.0 ? -127.0 : (t > 127.0 ? 127.0 : t);
        v = t == t ? (int)t : 0;                    // NaN (rows of infinite scales) -> 0, numpy's cast
    }
    Wq[i] = (int8_t)v;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i load16(const int8_t* base, int64_t row, int64_t lim, int C, int k) {
    if (row >= lim) return v4i{0, 0, 0, 0};
    return *reinterpret_cast<const v4i*>(base + row * C + k);
}

// a wave's 32 x 32 block of A B^T (rows a0.., b0..; rows past the limits read as zeros). Lane l
// holds rows a0 + l % 32 / b0 + l % 32 and 16 of each 32 columns (half l / 32): the same columns
// for A and B, so every product pairs equal columns. Result: lane l, element v is row
// a0 + 8 (v / 4) + 4 (l / 32) + v % 4, column b0 + l % 32.
__device__ __forceinline__ v16i tile_dot(const int8_t* A, int64_t alim, int64_t a0, const int8_t* B, int64_t blim,
                                         int64_t b0, int C) {
    const int lane = threadIdx.x & 63;
    const int64_t ar = a0 + (lane & 31), br = b0 + (lane & 31);
    const int kh = (lane >> 5) * 16;
    v16i acc = {};
    for (int k0 = 0; k0 < C; k0 += 32) {
        const v4i a = load16(A, ar, alim, C, k0 + kh);
        const v4i b = load16(B, br, blim, C, k0 + kh);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
    }
    return acc;
}
__device__ __forceinline__ int tile_row(int v) { return 8 * (v >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (v & 3); }

// S = A B^T exactly (int32), a wave per 32 x 32 block (detmath.sim8, detmath.py:250-259)
__global__ __launch_bounds__(64) void k_sim8(const int8_t* __restrict__ A, int64_t ra, const int8_t* __restrict__ B,
                                             int64_t rb, int C, int32_t* __restrict__ S) {
    const int64_t a0 = (int64_t)blockIdx.x * 32, b0 = (int64_t)blockIdx.y * 32;
    const v16i acc = tile_dot(A, ra, a0, B, rb, b0, C);
    const int64_t col = b0 + (threadIdx.x & 31);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t row = a0 + tile_row(v);
        if (row < ra && col < rb) S[row * rb + col] = acc[v];
    }
}

// per row r: the 4 rows c < wstart[r] with valid[c] of largest similarity Wq[r].Wq[c], ties to the
// lower index, -1 where fewer exist (gpu3.py:296-310). An LDS-staged int8 GEMM fused with the top-4
// merge: a workgroup takes 128 query rows and walks the candidate rows 128 at a time; per 64-column
// chunk the 256 lanes stage the query and candidate tiles in LDS (double-buffered, the next chunk's
// loads in flight during the MFMAs), each wave computes 32 query rows x 128 candidates as four
// v_mfma_i32_32x32x32_i8 tiles; the 128 x 128 similarities then go through LDS to lanes 0..127,
// which merge their row's values in ascending column order into a running top 4.
constexpr int NQ = 128, NCAND = 128, KC = 64, KPITCH = KC + 16;
__global__ __launch_bounds__(256) void k_neighbours(const int8_t* __restrict__ Wq, int64_t n, int C,
                                                    const int* __restrict__ wstart, const uint8_t* __restrict__ valid,
                                                    int* __restrict__ cand) {
    __shared__ __align__(16) int8_t As[2][NQ][KPITCH];
    __shared__ __align__(16) int8_t Bs[2][NCAND][KPITCH];
    __shared__ int32_t S[NQ][NCAND + 1];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int64_t q0 = (int64_t)blockIdx.x * NQ;
    const int64_t qlast = q0 + NQ - 1 < n ? q0 + NQ - 1 : n - 1;
    // candidates are earlier rows: wstart[r] <= r is the contract, and no read goes past row n - 1
    const int64_t cmax = min(max((int64_t)wstart[qlast], (int64_t)0), n);
    const int64_t q = q0 + tid;
    const int ws = (tid < NQ && q < n) ? (int)min(max((int64_t)wstart[q], (int64_t)0), cmax) : 0;
    int v0 = -2147483647 - 1, v1 = v0, v2 = v0, v3 = v0, i0 = -1, i1 = -1, i2 = -1, i3 = -1;
    const int nk = (C + KC - 1) / KC;
    // this lane's two 16-byte pieces of a 128-row x 64-byte chunk: row p / 4, bytes 16 (p % 4)
    const int pr0 = tid >> 2, pc0 = (tid & 3) * 16, pr1 = (tid + 256) >> 2, pc1 = ((tid + 256) & 3) * 16;
    auto piece = [&](int64_t row, int64_t lim, int k) -> v4i {
        if (row >= lim || k >= C) return v4i{0, 0, 0, 0};
        return *reinterpret_cast<const v4i*>(Wq + row * C + k);
    };
    for (int64_t j0 = 0; j0 < cmax; j0 += NCAND) {
        v16i acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = v16i{};
        v4i ra0 = piece(q0 + pr0, n, pc0), ra1 = piece(q0 + pr1, n, pc1);
        v4i rb0 = piece(j0 + pr0, cmax, pc0), rb1 = piece(j0 + pr1, cmax, pc1);
        *reinterpret_cast<v4i*>(&As[0][pr0][pc0]) = ra0;
        *reinterpret_cast<v4i*>(&As[0][pr1][pc1]) = ra1;
        *reinterpret_cast<v4i*>(&Bs[0][pr0][pc0]) = rb0;
        *reinterpret_cast<v4i*>(&Bs[0][pr1][pc1]) = rb1;
        __syncthreads();
        for (int kc = 0; kc < nk; ++kc) {
            const int cur = kc & 1;
            const bool more = kc + 1 < nk;
            if (more) {
                const int k = (kc + 1) * KC;
                ra0 = piece(q0 + pr0, n, k + pc0);
                ra1 = piece(q0 + pr1, n, k + pc1);
                rb0 = piece(j0 + pr0, cmax, k + pc0);
                rb1 = piece(j0 + pr1, cmax, k + pc1);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int kk = ks * 32 + (lane >> 5) * 16;
                const v4i a = *reinterpret_cast<const v4i*>(&As[cur][32 * w + (lane & 31)][kk]);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const v4i b = *reinterpret_cast<const v4i*>(&Bs[cur][32 * t + (lane & 31)][kk]);
                    acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[t], 0, 0, 0);
                }
            }
            if (more) {
                *reinterpret_cast<v4i*>(&As[cur ^ 1][pr0][pc0]) = ra0;
                *reinterpret_cast<v4i*>(&As[cur ^ 1][pr1][pc1]) = ra1;
                *reinterpret_cast<v4i*>(&Bs[cur ^ 1][pr0][pc0]) = rb0;
                *reinterpret_cast<v4i*>(&Bs[cur ^ 1][pr1][pc1]) = rb1;
            }
            __syncthreads();
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) S[32 * w + tile_row(v)][32 * t + (lane & 31)] = acc[t][v];
        __syncthreads();
        if (tid < NQ) {
            const int lim = (int)((int64_t)ws - j0 < NCAND ? (int64_t)ws - j0 : NCAND);
            for (int c = 0; c < lim; ++c) {
                const int cj = (int)j0 + c;
                if (!valid[cj]) continue;
                const int val = S[tid][c];
                if (val > v3) {
                    if (val > v2) {
                        v3 = v2; i3 = i2;
                        if (val > v1) {
                            v2 = v1; i2 = i1;
                            if (val > v0) { v1 = v0; i1 = i0; v0 = val; i0 = cj; }
                            else { v1 = val; i1 = cj; }
                        } else { v2 = val; i2 = cj; }
                    } else { v3 = val; i3 = cj; }
                }
            }
        }
        __syncthreads();
    }
    if (tid < NQ && q < n) {
        int* o = cand + q * KP;
        o[0] = i0; o[1] = i1; o[2] = i2; o[3] = i3;
    }
}

// Gaussian elimination with partial pivoting in float64 (detmath.py:122-152), K unknowns
template <int K>
__device__ __forceinline__ void solve_k(const float (&A)[KP][KP], const float (&b)[KP], float (&x)[KP]) {
    double M[K][K + 1];
#pragma unroll
    for (int i = 0; i < K; ++i) {
#pragma unroll
        for (int j = 0; j < K; ++j) M[i][j] = A[i][j];
        M[i][K] = b[i];
    }
#pragma unroll
    for (int col = 0; col < K; ++col) {
        int piv = col;
        double pv = fabs(M[col][col]);
#pragma unroll
        for (int i = col + 1; i < K; ++i) {
            const double a = fabs(M[i][col]);
            if (a > pv) { pv = a; piv = i; }
        }
#pragma unroll
        for (int i = col + 1; i < K; ++i) {
            if (piv == i) {
#pragma unroll
                for (int j = 0; j <= K; ++j) { const double t = M[col][j]; M[col][j] = M[i][j]; M[i][j] = t; }
            }
        }
        const double p = M[col][col];
#pragma unroll
        for (int i = col + 1; i < K; ++i) {
            const double f = M[i][col] / p;
#pragma unroll
            for (int j = col; j <= K; ++j) M[i][j] = M[i][j] - f * M[col][j];
        }
    }
#pragma unroll
    for (int i = K - 1; i >= 0; --i) {
        double s = M[i][K];
#pragma unroll
        for (int j = i + 1; j < K; ++j) s = s - M[i][j] * M[j][K];
        M[i][K] = s / M[i][i];
    }
#pragma unroll
    for (int i = 0; i < KP; ++i) x[i] = i < K ? (float)M[i][K] : 0.0f;
}

__device__ __forceinline__ float clipf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ double clipd(double v, double lo, double hi) { return v < lo ? lo : (v > hi ? hi : v); }

// a row's least-squares fit on its (up to) four parents for k = 1..4 parents, the choice of k by
// estimated bits (gpu3.py:312-343). Parent slots without a parent read row 0 times zero, as the
// reference's gather does. Lane per row.
__global__ __launch_bounds__(64) void k_fit(const float* __restrict__ W, const int* __restrict__ cand, int64_t n, int C,
                                            float* __restrict__ frac, int* __restrict__ kuse, float* __restrict__ coefs) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const float4* y = reinterpret_cast<const float4*>(W + r * C);
    const float4* x[KP];
    float z[KP];
#pragma unroll
    for (int a = 0; a < KP; ++a) {
        const int p = cand[r * KP + a];
        x[a] = reinterpret_cast<const float4*>(W + (int64_t)(p >= 0 ? p : 0) * C);
        z[a] = p >= 0 ? 1.0f : 0.0f;
    }
    double yy = 0.0, g[KP][KP], bd[KP];
#pragma unroll
    for (int a = 0; a < KP; ++a) {
        bd[a] = 0.0;
#pragma unroll
        for (int b = 0; b < KP; ++b) g[a][b] = 0.0;
    }
    const int C4 = C / 4;
    for (int t = 0; t < C4; ++t) {
        const float4 yv = y[t];
        float4 xv[KP];
#pragma unroll
        for (int a = 0; a < KP; ++a) {
            const float4 u = x[a][t];
            xv[a] = make_float4(__fmul_rn(u.x, z[a]), __fmul_rn(u.y, z[a]), __fmul_rn(u.z, z[a]), __fmul_rn(u.w, z[a]));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const double yd = e == 0 ? yv.x : e == 1 ? yv.y : e == 2 ? yv.z : yv.w;
            double xd[KP];
#pragma unroll
            for (int a = 0; a < KP; ++a) xd[a] = e == 0 ? xv[a].x : e == 1 ? xv[a].y : e == 2 ? xv[a].z : xv[a].w;
            yy = yy + yd * yd;
#pragma unroll
            for (int a = 0; a < KP; ++a) {
                bd[a] = bd[a] + xd[a] * yd;
#pragma unroll
                for (int b = a; b < KP; ++b) g[a][b] = g[a][b] + xd[a] * xd[b];
            }
        }
    }
    yy = yy > 1e-12 ? yy : (yy != yy ? yy : 1e-12);
    float A[KP][KP], bv[KP], c[KP + 1][KP];
#pragma unroll
    for (int a = 0; a < KP; ++a) {
        bv[a] = (float)bd[a];
#pragma unroll
        for (int b = 0; b < KP; ++b) A[a][b] = __fadd_rn((float)g[a < b ? a : b][a < b ? b : a], a == b ? 1e-3f : 0.0f);
    }
#pragma unroll
    for (int a = 0; a < KP; ++a) c[0][a] = 0.0f;
    solve_k<1>(A, bv, c[1]);
    solve_k<2>(A, bv, c[2]);
    solve_k<3>(A, bv, c[3]);
    solve_k<4>(A, bv, c[4]);
#pragma unroll
    for (int k = 1; k <= KP; ++k)
#pragma unroll
        for (int a = 0; a < KP; ++a) c[k][a] = __fdiv_rn(clipf(rintf(__fmul_rn(c[k][a], 64.0f)), -127.0f, 127.0f), 64.0f);
    double s[KP + 1] = {0.0, 0.0, 0.0, 0.0, 0.0};
    for (int t = 0; t < C4; ++t) {
        const float4 yv = y[t];
        float4 xv[KP];
#pragma unroll
        for (int a = 0; a < KP; ++a) {
            const float4 u = x[a][t];
            xv[a] = make_float4(__fmul_rn(u.x, z[a]), __fmul_rn(u.y, z[a]), __fmul_rn(u.z, z[a]), __fmul_rn(u.w, z[a]));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float yf = e == 0 ? yv.x : e == 1 ? yv.y : e == 2 ? yv.z : yv.w;
            float xf[KP];
#pragma unroll
            for (int a = 0; a < KP; ++a) xf[a] = e == 0 ? xv[a].x : e == 1 ? xv[a].y : e == 2 ? xv[a].z : xv[a].w;
#pragma unroll
            for (int k = 1; k <= KP; ++k) {
                float res = yf;
#pragma unroll
                for (int a = 0; a < k; ++a) res = __fsub_rn(res, __fmul_rn(c[k][a], xf[a]));
                s[k] = s[k] + (double)res * (double)res;
            }
        }
    }
    const double ncol = (double)(C - C / 32);
    double best_cost = 0.0, best = 1.0;
    int bk = 0;
#pragma unroll
    for (int k = 1; k <= KP; ++k) {
        const double f = clipd(s[k] / yy, 1e-3, 4.0);
        const double cost = 0.5 * dm::dm_log2(f) * ncol + (double)(k * 25);
        if (cost < best_cost) { best_cost = cost; best = f; bk = k; }
    }
    frac[r] = (float)best;
    kuse[r] = bk;
#pragma unroll
    for (int a = 0; a < KP; ++a) {
        float v = 0.0f;
#pragma unroll
        for (int k = 1; k <= KP; ++k) if (bk == k) v = c[k][a];
        coefs[r * KP + a] = v;
    }
}

// part[ch][c] = sum over the valid rows of chunk ch (chunk rows, in order) of the chosen residual^2
// (gpu3.py:343: detmath.cols(res_best, True, mask) per chunk of 2048 rows)
__global__ __launch_bounds__(256) void k_col_res(const float* __restrict__ W, const int* __restrict__ cand,
                                                 const float* __restrict__ coefs, const int* __restrict__ kuse,
                                                 const uint8_t* __restrict__ valid, int64_t n, int C, int64_t chunk,
                                                 double* __restrict__ part) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const int64_t r0 = (int64_t)blockIdx.y * chunk, r1 = r0 + chunk < n ? r0 + chunk : n;
    double s = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
        if (!valid[r]) continue;
        float res = W[r * C + c];
        const int k = kuse[r];
        for (int a = 0; a < k; ++a) {
            const int p = cand[r * KP + a];
            const float xf = __fmul_rn(W[(int64_t)(p >= 0 ? p : 0) * C + c], p >= 0 ? 1.0f : 0.0f);
            res = __fsub_rn(res, __fmul_rn(coefs[r * KP + a], xf));
        }
        s = s + (double)res * (double)res;
    }
    part[blockIdx.y * (int64_t)C + c] = s;
}

unsigned nblk(int64_t n, int wg) { return (unsigned)((n + wg - 1) / wg); }

}  // namespace
}  // namespace q8
}  // namespace spa

using spa::fail;
using namespace spa::q8;

#define Q8_NONNULL(...)                                                              \
    do {                                                                             \
        const void* ps_[] = {__VA_ARGS__};                                           \
        for (const void* p_ : ps_)                                                   \
            if (!p_) return fail(SPA_ERR_ARG, "%s: null pointer", __func__);         \
    } while (0)

extern "C" {

int spa_q8_pos(const void* blocks, int64_t n, uint8_t* pos, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_q8_pos: %lld blocks", (long long)n);
    if (!n) return SPA_OK;
    Q8_NONNULL(blocks, pos);
    hipLaunchKernelGGL(k_pos, dim3(nblk(n, 256)), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks, n, pos);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_row_means(const void* blocks, const void* meta, int ntens, int64_t nrows, int* row_m, void* stream) {
    if (ntens <= 0 || nrows < 0) return fail(SPA_ERR_ARG, "spa_q8_row_means: %d tensors, %lld rows", ntens, (long long)nrows);
    if (!nrows) return SPA_OK;
    Q8_NONNULL(blocks, meta, row_m);
    hipLaunchKernelGGL(k_row_means, dim3(nblk(nrows, 256)), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks,
                       (const Meta*)meta, ntens, nrows, row_m);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_col_stats(const void* blocks, int first, int nbr, int64_t nrows, const int* row_m, float* rel,
                     int64_t rows_per_slice, double* part1, double* part2, void* stream) {
    if (first < 0 || nbr <= 0 || nrows <= 0 || rows_per_slice <= 0)
        return fail(SPA_ERR_ARG, "spa_q8_col_stats: first %d, %d blocks per row, %lld rows, %lld rows per slice", first,
                    nbr, (long long)nrows, (long long)rows_per_slice);
    Q8_NONNULL(blocks, row_m, rel, part1, part2);
    const int64_t nsl = (nrows + rows_per_slice - 1) / rows_per_slice;
    if (nsl > 65535) return fail(SPA_ERR_ARG, "spa_q8_col_stats: %lld slices", (long long)nsl);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_rel, dim3(nblk(nrows * nbr, 256)), dim3(256), 0, st, (const uint8_t*)blocks, first, nbr, nrows,
                       row_m, rel);
    hipLaunchKernelGGL(k_col_stats, dim3(nblk(nbr * 32, 256), (unsigned)nsl), dim3(256), 0, st, (const uint8_t*)blocks,
                       first, nbr, nrows, (const float*)rel, rows_per_slice, part1, part2);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_row_hash(const void* blocks, int first, int nbr, int64_t nrows, const uint64_t* mult, uint64_t* h, void* stream) {
    if (first < 0 || nbr <= 0 || nrows < 0 || (nbr * 34) % 8)
        return fail(SPA_ERR_ARG, "spa_q8_row_hash: %d blocks per row (rows must be whole 64-bit words)", nbr);
    if (!nrows) return SPA_OK;
    Q8_NONNULL(blocks, mult, h);
    if (nrows > 0x7fffffff) return fail(SPA_ERR_ARG, "spa_q8_row_hash: %lld rows", (long long)nrows);
    hipLaunchKernelGGL(k_row_hash, dim3((unsigned)nrows), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)blocks, first,
                       nbr, nrows, mult, h);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_rows_equal(const void* blocks, int first, int nbr, const int* ra, const int* rb, int n, uint8_t* eq,
                      void* stream) {
    if (first < 0 || nbr <= 0 || n < 0) return fail(SPA_ERR_ARG, "spa_q8_rows_equal: bad arguments");
    if (!n) return SPA_OK;
    Q8_NONNULL(blocks, ra, rb, eq);
    hipLaunchKernelGGL(k_rows_equal, dim3((unsigned)n), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)blocks, first, nbr,
                       ra, rb, n, eq);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_rcp(const uint16_t* freq, int ntab, uint32_t* rcp, void* stream) {
    if (ntab < 0) return fail(SPA_ERR_ARG, "spa_q8_rcp: %d tables", ntab);
    if (!ntab) return SPA_OK;
    Q8_NONNULL(freq, rcp);
    hipLaunchKernelGGL(k_rcp, dim3((unsigned)ntab), dim3(256), 0, (hipStream_t)stream, freq, ntab, rcp);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

static int check_a(const char* fn, int ntens, int nblocks) {
    if (ntens <= 0 || nblocks < 0) return fail(SPA_ERR_ARG, "%s: %d tensors, %d blocks", fn, ntens, nblocks);
    return SPA_OK;
}

int spa_q8_hist_a(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                  const uint8_t* bcf, const uint8_t* spread, const uint8_t* rankof, const uint8_t* scls, uint32_t* counts,
                  void* stream) {
    if (int e = check_a(__func__, ntens, nblocks)) return e;
    if (!nblocks) return SPA_OK;
    Q8_NONNULL(blocks, pos, skip, meta, bcf, spread, rankof, scls, counts);
    AArgs A{skip, (const Meta*)meta, ntens, nblocks, bcf, spread, nullptr, rankof, scls};
    const int nseg = (nblocks + SEGA - 1) / SEGA;
    hipLaunchKernelGGL(k_hist_a, dim3(nblk(nseg, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)blocks, pos, A, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_enc_a(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                 const uint8_t* bcf, const uint8_t* spread, const uint8_t* rankof, const uint8_t* scls, const int* remap,
                 const uint16_t* freq, const uint32_t* cum, const uint32_t* rcp, void* out, uint64_t cap, uint32_t* out_len,
                 void* stream) {
    if (int e = check_a(__func__, ntens, nblocks)) return e;
    if (cap < 64) return fail(SPA_ERR_ARG, "spa_q8_enc_a: slot capacity %llu", (unsigned long long)cap);
    if (!nblocks) return SPA_OK;
    Q8_NONNULL(blocks, pos, skip, meta, bcf, spread, rankof, scls, remap, freq, cum, rcp, out, out_len);
    AArgs A{skip, (const Meta*)meta, ntens, nblocks, bcf, spread, nullptr, rankof, scls};
    const int nseg = (nblocks + SEGA - 1) / SEGA;
    hipLaunchKernelGGL(k_enc_a, dim3(nblk(nseg, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)blocks, pos, A, remap,
                       freq, cum, rcp, (uint8_t*)out, cap, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_lut32(const uint16_t* freq, const uint32_t* cum, int ntab, uint32_t* lut, void* stream) {
    if (ntab < 0) return fail(SPA_ERR_ARG, "spa_q8_lut32: %d tables", ntab);
    if (!ntab) return SPA_OK;
    Q8_NONNULL(freq, cum, lut);
    hipLaunchKernelGGL(k_lut32, dim3((unsigned)ntab), dim3(256), 0, (hipStream_t)stream, freq, cum, ntab, lut);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_dec_a(const void* in, uint64_t in_bytes, const uint64_t* in_off, const uint8_t* skip, const void* meta, int ntens,
                 int nblocks, const uint8_t* bcf, const uint8_t* spread, const uint8_t* perm, const uint8_t* scls,
                 const int* remap, const uint32_t* lut, void* blocks, uint8_t* pos, void* stream) {
    if (int e = check_a(__func__, ntens, nblocks)) return e;
    if (!nblocks) return SPA_OK;
    Q8_NONNULL(in, in_off, skip, meta, bcf, spread, perm, scls, remap, lut, blocks, pos);
    AArgs A{skip, (const Meta*)meta, ntens, nblocks, bcf, spread, perm, nullptr, scls};
    const int nseg = (nblocks + SEGA - 1) / SEGA;
    hipLaunchKernelGGL(k_dec_a, dim3(nblk(nseg, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)in, in_bytes, in_off,
                       A, remap, lut, (uint8_t*)blocks, pos);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_hist_b(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                  const void* items, int nitems, const int16_t* cfi, const uint8_t* scls, const int* row_m, int qbase,
                  uint32_t* counts, void* stream) {
    if (int e = check_a(__func__, ntens, nblocks)) return e;
    if (nitems < 0) return fail(SPA_ERR_ARG, "spa_q8_hist_b: %d work items", nitems);
    if (!nitems) return SPA_OK;
    Q8_NONNULL(blocks, pos, skip, meta, items, cfi, scls, row_m, counts);
    BArgs B{skip, (const Meta*)meta, ntens, nblocks, cfi, scls, row_m, qbase};
    hipLaunchKernelGGL(k_hist_b, dim3((unsigned)nitems), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks, pos, B,
                       (const Item*)items, counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_enc_b(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                 const int16_t* cfi, const uint8_t* scls, const int* row_m, int qbase, const int* remap, const uint16_t* freq,
                 const uint32_t* cum, const uint32_t* rcp, void* out, uint64_t cap, uint32_t* out_len, void* stream) {
    if (int e = check_a(__func__, ntens, nblocks)) return e;
    if (cap < 256) return fail(SPA_ERR_ARG, "spa_q8_enc_b: slot capacity %llu", (unsigned long long)cap);
    if (!nblocks) return SPA_OK;
    Q8_NONNULL(blocks, pos, skip, meta, cfi, scls, row_m, remap, freq, cum, rcp, out, out_len);
    BArgs B{skip, (const Meta*)meta, ntens, nblocks, cfi, scls, row_m, qbase};
    const int nseg = (nblocks + SEGB - 1) / SEGB;
    hipLaunchKernelGGL(k_enc_b, dim3(nblk(nseg, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)blocks, pos, B, remap,
                       freq, cum, rcp, (uint8_t*)out, cap, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_dec_b(const void* in, uint64_t in_bytes, const uint64_t* in_off, const uint8_t* skip, const void* meta, int ntens,
                 int nblocks, const int16_t* cfi, const uint8_t* scls, const int* row_m, int qbase, const int* remap,
                 const uint32_t* lut, void* blocks, const uint8_t* pos, void* stream) {
    if (int e = check_a(__func__, ntens, nblocks)) return e;
    if (!nblocks) return SPA_OK;
    Q8_NONNULL(in, in_off, skip, meta, cfi, scls, row_m, remap, lut, blocks, pos);
    BArgs B{skip, (const Meta*)meta, ntens, nblocks, cfi, scls, row_m, qbase};
    const int nseg = (nblocks + SEGB - 1) / SEGB;
    hipLaunchKernelGGL(k_dec_b, dim3(nblk(nseg, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)in, in_bytes, in_off,
                       B, remap, lut, (uint8_t*)blocks, pos);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_predict(const void* blocks, int first, int nbr, int64_t nrows, const int* par, const float* coef, const float* mu,
                   int8_t* pint, void* stream) {
    if (first < 0 || nbr <= 0 || nrows < 0) return fail(SPA_ERR_ARG, "spa_q8_predict: bad shape");
    if (!nrows) return SPA_OK;
    Q8_NONNULL(blocks, par, coef, mu, pint);
    hipLaunchKernelGGL(k_predict, dim3(nblk(nrows * nbr * 32, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blocks, first, nbr, nrows, par, coef, mu, pint);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_predict_multi(const void* blocks, const int* ent_slot, const int* ent_row, int nent, int cmax, const void* slots,
                         const int* par, const float* coef, const float* mu, int8_t* pint, void* stream) {
    if (nent < 0 || cmax <= 0 || cmax % 32) return fail(SPA_ERR_ARG, "spa_q8_predict_multi: %d entries, %d columns", nent, cmax);
    if (!nent) return SPA_OK;
    Q8_NONNULL(blocks, ent_slot, ent_row, slots, par, coef, mu, pint);
    hipLaunchKernelGGL(k_predict_multi, dim3(nblk((int64_t)nent * cmax, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blocks, ent_slot, ent_row, nent, cmax, (const Slot*)slots, par, coef, mu, pint);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_ranks(const int8_t* pint, int64_t nb, int8_t* prk, int8_t* pinv, int8_t* rctx, void* stream) {
    if (nb < 0) return fail(SPA_ERR_ARG, "spa_q8_ranks: %lld blocks", (long long)nb);
    if (!nb) return SPA_OK;
    Q8_NONNULL(pint, prk, pinv, rctx);
    hipLaunchKernelGGL(k_ranks, dim3(nblk(nb * 32, 256)), dim3(256), 0, (hipStream_t)stream, pint, nb, prk, pinv, rctx);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_hist_c(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, const void* segs, int nseg,
                  const void* slots, const int16_t* cfi, const int* row_m, const int8_t* fbin, const int8_t* pint,
                  const int8_t* prk, const int8_t* pinv, const int8_t* rctx, uint32_t* counts, void* stream) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "spa_q8_hist_c: %d segments", nseg);
    if (!nseg) return SPA_OK;
    Q8_NONNULL(blocks, pos, skip, meta, segs, slots, cfi, row_m, fbin, pint, prk, pinv, rctx, counts);
    CArgs A{skip, (const Meta*)meta, (const CSeg*)segs, nseg, (const Slot*)slots, cfi, row_m, fbin, pint, prk, pinv, rctx};
    hipLaunchKernelGGL(k_hist_c, dim3(nblk(nseg, HC_SEGS)), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks, pos, A,
                       counts);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_enc_c(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, const void* segs, int nseg,
                 const void* slots, const int16_t* cfi, const int* row_m, const int8_t* fbin, const int8_t* pint,
                 const int8_t* prk, const int8_t* pinv, const int8_t* rctx, const int* remap, const uint16_t* freq,
                 const uint32_t* cum, const uint32_t* rcp, void* out, uint64_t cap, uint32_t* out_len, void* stream) {
    if (nseg < 0 || cap < 256) return fail(SPA_ERR_ARG, "spa_q8_enc_c: %d segments, slot capacity %llu", nseg, (unsigned long long)cap);
    if (!nseg) return SPA_OK;
    Q8_NONNULL(blocks, pos, skip, meta, segs, slots, cfi, row_m, fbin, pint, prk, pinv, rctx, remap, freq, cum, rcp, out,
               out_len);
    CArgs A{skip, (const Meta*)meta, (const CSeg*)segs, nseg, (const Slot*)slots, cfi, row_m, fbin, pint, prk, pinv, rctx};
    hipLaunchKernelGGL(k_enc_c, dim3(nblk(nseg, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)blocks, pos, A, remap,
                       freq, cum, rcp, (uint8_t*)out, cap, out_len);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_dec_c(const void* in, uint64_t in_bytes, const uint64_t* in_off, int seg0, int seg1, const uint8_t* skip,
                 const void* meta, const void* segs, int nseg, const void* slots, const int16_t* cfi, const int* row_m,
                 const int8_t* fbin, const int8_t* pint, const int8_t* prk, const int8_t* pinv, const int8_t* rctx,
                 const int* remap, const uint32_t* lut, void* blocks, uint8_t* pos, void* stream) {
    if (seg0 < 0 || seg1 > nseg || seg0 > seg1) return fail(SPA_ERR_ARG, "spa_q8_dec_c: segments [%d, %d) of %d", seg0, seg1, nseg);
    if (seg0 == seg1) return SPA_OK;
    Q8_NONNULL(in, in_off, skip, meta, segs, slots, cfi, row_m, fbin, pint, prk, pinv, rctx, remap, lut, blocks, pos);
    CArgs A{skip, (const Meta*)meta, (const CSeg*)segs, nseg, (const Slot*)slots, cfi, row_m, fbin, pint, prk, pinv, rctx};
    hipLaunchKernelGGL(k_dec_c, dim3(nblk(seg1 - seg0, 64)), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)in, in_bytes,
                       in_off, seg0, seg1, A, remap, lut, (uint8_t*)blocks, pos);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_row_matrix(const void* blocks, int first, int nbr, int64_t nrows, float* W, void* stream) {
    if (first < 0 || nbr <= 0 || nrows < 0) return fail(SPA_ERR_ARG, "spa_q8_row_matrix: bad shape");
    if (!nrows) return SPA_OK;
    Q8_NONNULL(blocks, W);
    hipLaunchKernelGGL(k_row_matrix, dim3(nblk(nrows * nbr * 32, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blocks, first, nbr, nrows, W);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_center(float* W, const float* mu, int64_t nrows, int C, void* stream) {
    if (nrows < 0 || C <= 0) return fail(SPA_ERR_ARG, "spa_q8_center: bad shape");
    if (!nrows) return SPA_OK;
    Q8_NONNULL(W, mu);
    hipLaunchKernelGGL(k_center, dim3(nblk(nrows * C, 256)), dim3(256), 0, (hipStream_t)stream, W, mu, nrows, C);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_norm_i8(const float* W, const double* nrm, const uint8_t* valid, int64_t nrows, int C, int8_t* Wq, void* stream) {
    if (nrows < 0 || C <= 0) return fail(SPA_ERR_ARG, "spa_q8_norm_i8: bad shape");
    if (!nrows) return SPA_OK;
    Q8_NONNULL(W, nrm, valid, Wq);
    hipLaunchKernelGGL(k_norm_i8, dim3(nblk(nrows * C, 256)), dim3(256), 0, (hipStream_t)stream, W, nrm, valid, nrows, C, Wq);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_sim8(const int8_t* A, int64_t ra, const int8_t* B, int64_t rb, int C, int32_t* S, void* stream) {
    if (ra < 0 || rb < 0 || C <= 0 || C % 32) return fail(SPA_ERR_ARG, "spa_q8_sim8: %lld x %lld rows of %d (a multiple of 32)",
                                                          (long long)ra, (long long)rb, C);
    if ((ra + 31) / 32 > 0x7fffffff || (rb + 31) / 32 > 65535) return fail(SPA_ERR_ARG, "spa_q8_sim8: too many rows");
    if (!ra || !rb) return SPA_OK;
    Q8_NONNULL(A, B, S);
    if (((uintptr_t)A | (uintptr_t)B) & 15) return fail(SPA_ERR_ARG, "spa_q8_sim8: operands must be 16-byte aligned");
    hipLaunchKernelGGL(k_sim8, dim3((unsigned)((ra + 31) / 32), (unsigned)((rb + 31) / 32)), dim3(64), 0, (hipStream_t)stream,
                       A, ra, B, rb, C, S);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_neighbours(const int8_t* Wq, int64_t n, int C, const int* wstart, const uint8_t* valid, int* cand, void* stream) {
    if (n < 0 || C <= 0 || C % 32) return fail(SPA_ERR_ARG, "spa_q8_neighbours: %lld rows of %d (a multiple of 32)", (long long)n, C);
    if (!n) return SPA_OK;
    Q8_NONNULL(Wq, wstart, valid, cand);
    if ((uintptr_t)Wq & 15) return fail(SPA_ERR_ARG, "spa_q8_neighbours: rows must be 16-byte aligned");
    hipLaunchKernelGGL(k_neighbours, dim3(nblk(n, NQ)), dim3(256), 0, (hipStream_t)stream, Wq, n, C, wstart, valid, cand);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_fit_rows(const float* W, const int* cand, int64_t n, int C, float* frac, int* kuse, float* coefs, void* stream) {
    if (n < 0 || C <= 0 || C % 4) return fail(SPA_ERR_ARG, "spa_q8_fit_rows: %lld rows of %d", (long long)n, C);
    if (!n) return SPA_OK;
    Q8_NONNULL(W, cand, frac, kuse, coefs);
    hipLaunchKernelGGL(k_fit, dim3(nblk(n, 64)), dim3(64), 0, (hipStream_t)stream, W, cand, n, C, frac, kuse, coefs);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_q8_col_res(const float* W, const int* cand, const float* coefs, const int* kuse, const uint8_t* valid, int64_t n,
                   int C, int64_t chunk, double* part, void* stream) {
    if (n < 0 || C <= 0 || chunk <= 0) return fail(SPA_ERR_ARG, "spa_q8_col_res: bad shape");
    if (!n) return SPA_OK;
    Q8_NONNULL(W, cand, coefs, kuse, valid, part);
    const int64_t nch = (n + chunk - 1) / chunk;
    if (nch > 65535) return fail(SPA_ERR_ARG, "spa_q8_col_res: %lld chunks", (long long)nch);
    hipLaunchKernelGGL(k_col_res, dim3(nblk(C, 256), (unsigned)nch), dim3(256), 0, (hipStream_t)stream, W, cand, coefs, kuse,
                       valid, n, C, chunk, part);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
