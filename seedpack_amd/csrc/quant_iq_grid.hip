// Grid i-quants: IQ2_XXS, IQ2_XS, IQ2_S (8-dimensional lattice groups), IQ3_XXS, IQ3_S
// (4-dimensional groups), IQ1_S, IQ1_M (8-dimensional ternary groups), bit-exact with
// ggml-quants.c (cited per type).
//
// Mapping: one lane per sub-block (32 or 16 weights), G = 256/sub lanes per super-block, 256-lane
// workgroups. Per workgroup the lattice codebook is copied to LDS; the level-index map and the
// neighbour lists stay in global memory (43,692 x int32 and up to 1.4 M x uint16: L2-resident).
// The super-block sum of squares (and IQ1_M's final scale refit) is one left-to-right float sum:
// it is handed from lane to lane of the group by shuffles. Every sub-block search (trial scales,
// lattice lookups, neighbour searches; IQ1: sorting and the exhaustive split search) runs in its own
// lane. Lane 0 of each group packs the block from the per-lane results parked in LDS.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "iq_tables.h"
#include "launch.h"
#include "search.h"

namespace spa {
namespace {

constexpr int WG = 256;
constexpr float FLT_BIG = 3.402823466e+38F;   // FLT_MAX

// ---------------------------------------------------------------- shared helpers

// sum of v[] over the G lanes of a group, lane 0's terms first: one left-to-right float sum
template <int G, int N>
__device__ __forceinline__ float group_sum(const float (&v)[N], int sub) {
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (sub == g) {
#pragma unroll
            for (int i = 0; i < N; ++i) s += v[i];
        }
        s = __shfl(s, g, G);
    }
    return s;
}

template <int D>
struct LIdx {
    static constexpr int B = D == 8 ? 2 : 3, M = (1 << B) - 1;
    __device__ __forceinline__ static int level(int u, int i) { return (u >> (B * i)) & M; }
};

// grid point j's coordinate values (2l+1) from the LDS codebook
template <int D>
__device__ __forceinline__ void grid_point(const uint8_t* grid, int j, int (&q)[D]) {
    if constexpr (D == 8) {
        const uint2 v = reinterpret_cast<const uint2*>(grid)[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) { q[i] = (v.x >> (8 * i)) & 0xff; q[4 + i] = (v.y >> (8 * i)) & 0xff; }
    } else {
        const uint32_t v = reinterpret_cast<const uint32_t*>(grid)[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = (v >> (8 * i)) & 0xff;
    }
}

// ------------------------------------------------------- wave-balanced neighbour search
//
// A lattice group off the grid is snapped to the best point of its neighbour list
// (iq2_find_best_neighbour / iq3_find_best_neighbour, ggml-quants.c:3271-3293, :3915-3937): among the
// listed points, the first with the smallest weighted squared error sum_i sqrt(w_i) (s q_i - x_i)^2
// at the trial scale s. The lists hold 1 to ~300 points; one lane per list would leave the wave
// waiting for its longest list (3-4x the useful work on the configuration-3 tensors). Instead, for
// one group index k at a time, the lists of all the wave's off-grid groups are cut into pieces of
// a few consecutive entries and the pieces are dealt to the 64 lanes in rounds, so every lane
// evaluates the same number of entries per round. A piece's owner (its group's |x|, scale, list) is read from the owner's LDS
// record and its sqrt(w) from the owner's LDS row. Each list's winner is kept in an LDS slot as the
// 64-bit key (d2 bits, position, point) lowered by atomic min: d2 >= +0 orders as its bit pattern, so
// the least key is the smallest d2 at the smallest position -- the reference's first strict minimum.
// Entries are kept only when d2 < FLT_MAX (the reference's initial best); a list with none keeps its
// first point (the reference asserts there instead).
// Entries per piece (measured per type on the configuration-3 tensors): long lists (the
// 8-dimensional lattices, 35 entries on average when off the grid) take 8, the 4-dimensional ones
// (about 14) take 4; IQ2_S takes 4 and IQ3_S 6.
template <int D> constexpr int nb_piece() { return D == 8 ? 8 : 4; }

template <int D>
struct NbWave {
    // per owner lane: |x| of the group, scale, list offset, first piece, length; rows of 12 words put
    // the records of 8 consecutive owners on distinct banks
    __align__(16) float rec[64][12];
    unsigned long long slot[64];          // per owner lane: least key so far
    int mark[D == 4 ? 64 : 1];            // (D = 4) per round: the lane whose pieces start at this slot, else -1
};

struct NbCtx {
    void* w;               // this wave's NbWave
    const float* wrows;    // per-lane rows of sqrt(w) (N floats each, rotated: wrow_at), the workgroup's
    int wbase;             // the wave's first thread in the workgroup
};

// LDS writes of the wave's lanes complete before its later LDS reads, and no compiler reordering
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// inclusive prefix maximum over the 64 lanes (-1 is the identity): shifts by 1, 2, 4, 8 inside each
// row of 16 lanes, then lane 15 of rows 0 and 2 into rows 1 and 3, then lane 31 into rows 2 and 3
__device__ __forceinline__ int wave_prefix_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x111, 0xf, 0xf, false));   // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x112, 0xf, 0xf, false));   // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x114, 0xf, 0xf, false));   // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x118, 0xf, 0xf, false));   // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x142, 0xa, 0xf, false));   // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x143, 0xc, 0xf, false));   // row_bcast:31
    return v;
}

// The device map holds, for a point off the grid, -1 - (list offset << 9 | list length)
__device__ __forceinline__ int nb_offset(int gi) { return (-1 - gi) >> 9; }
__device__ __forceinline__ int nb_length(int gi) { return (-1 - gi) & 511; }

// Thread t's row of sqrt(w) holds its 4-weight group v at float4 slot (v + t) mod N/4: the rows of
// different owners read in one instruction start on different banks.
template <int N>
__device__ __forceinline__ int wrow_at(int t, int v) { return (v + t) % (N / 4); }

// The level index of the best neighbour of group k for the lanes with `off` set (gi: the map's
// negative entry for the group's rounded point); called by all lanes of the wave together.
template <int D, int N, int R = nb_piece<D>()>
__device__ int wave_best_neighbour(const NbCtx& c, int k, bool off, int gi, const float (&xval)[N], float scale,
                                   const uint16_t* __restrict__ nbt, const uint8_t* grid) {
    NbWave<D>& W = *reinterpret_cast<NbWave<D>*>(c.w);
    constexpr unsigned long long INIT = (unsigned long long)0x7f7fffffu << 32;   // (FLT_MAX, position 0)
    const int lane = (int)__lane_id();
    const int ptr = off ? nb_offset(gi) : 0;
    const int len = off ? nb_length(gi) : 0;
    const int np = (len + R - 1) / R;
    // inclusive prefix of the piece counts over the wave (the scan of wave_prefix_max with +)
    int incl = np;
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xf, 0xf, false);   // row_shr:1
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xf, 0xf, false);   // row_shr:2
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xf, 0xf, false);   // row_shr:4
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xf, 0xf, false);   // row_shr:8
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xa, 0xf, false);   // row_bcast:15
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x143, 0xc, 0xf, false);   // row_bcast:31
    const int first = incl - np;
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (np > 0) {
        float4* r = reinterpret_cast<float4*>(W.rec[lane]);
#pragma unroll
        for (int v = 0; v < D / 4; ++v)
            r[v] = make_float4(xval[D * k + 4 * v], xval[D * k + 4 * v + 1], xval[D * k + 4 * v + 2], xval[D * k + 4 * v + 3]);
        r[D / 4] = make_float4(scale, __int_as_float(ptr), __int_as_float(first), __int_as_float(len));
        W.slot[lane] = INIT;
    }
    if constexpr (D == 4) W.mark[lane] = -1;
    wave_lds_sync();
    for (int base = 0; base < total; base += 64) {
        const int q = base + lane;
        // the owner of piece q, the lane whose pieces [first, incl) hold q
        int o = 0;
        if constexpr (D == 4) {
            // short lists, many owners per round: each lane whose pieces meet this round marks the
            // slot of its first one in it (distinct slots; slot 0 always has one, the owner of piece
            // `base`), and the owner of q is the last mark at or before q; each lane resets its slot
            // after reading it
            if (np > 0 && first < base + 64 && incl > base) W.mark[(first > base ? first : base) - base] = lane;
            wave_lds_sync();
            const int m = W.mark[lane];
            W.mark[lane] = -1;
            o = max(wave_prefix_max(m), 0);
        } else {
            // long lists, few owners per round: the number of lanes whose pieces end at or before q
            // (incl rises with lane), by binary search
#pragma unroll
            for (int st = 32; st >= 1; st >>= 1) {
                const int probe = __shfl(incl, o + st - 1);
                if (probe <= q) o += st;
            }
        }
        if (q < total) {
            const float4* r = reinterpret_cast<const float4*>(W.rec[o]);
            const float4* wr = reinterpret_cast<const float4*>(c.wrows + (c.wbase + o) * N);
            float xg[D], wv[D];
#pragma unroll
            for (int v = 0; v < D / 4; ++v) {
                const float4 a = r[v], b = wr[wrow_at<N>(c.wbase + o, D * k / 4 + v)];
                xg[4 * v] = a.x; xg[4 * v + 1] = a.y; xg[4 * v + 2] = a.z; xg[4 * v + 3] = a.w;
                wv[4 * v] = b.x; wv[4 * v + 1] = b.y; wv[4 * v + 2] = b.z; wv[4 * v + 3] = b.w;
            }
            const float4 meta = r[D / 4];
            const float s = meta.x;
            const int p = __float_as_int(meta.y), L = __float_as_int(meta.w);
            const int pos0 = (q - __float_as_int(meta.z)) * R;
            float best = FLT_BIG;
            uint32_t bj = 0;
            // the piece's list entries, then their codebook points, are all requested before the
            // first distance is formed (one wait each instead of a load chain per entry); positions
            // past the list end re-read its last entry and are left out of the minimum
            int jj[R];
#pragma unroll
            for (int e = 0; e < R; ++e) jj[e] = nbt[p + 1 + min(pos0 + e, L - 1)];
            int qg[R][D];
#pragma unroll
            for (int e = 0; e < R; ++e) grid_point<D>(grid, jj[e], qg[e]);
#pragma unroll
            for (int e = 0; e < R; ++e) {
                const int pos = pos0 + e;
                float d2 = 0;
#pragma unroll
                for (int i = 0; i < D; ++i) {
                    const float diff = s * (float)qg[e][i] - xg[i];
                    d2 += wv[i] * diff * diff;
                }
                if (pos < L && d2 < best) { best = d2; bj = ((uint32_t)pos << 16) | (uint32_t)jj[e]; }
            }
            if (best < FLT_BIG) atomicMin(&W.slot[o], ((unsigned long long)__float_as_uint(best) << 32) | bj);
        }
    }
    wave_lds_sync();
    int u = 0;
    if (np > 0) {
        const unsigned long long key = W.slot[lane];
        const int j = key == INIT ? (int)nbt[ptr + 1] : (int)(key & 0xffffu);
        int qg[D];
        grid_point<D>(grid, j, qg);
#pragma unroll
        for (int i = 0; i < D; ++i) u |= ((qg[i] - 1) / 2) << (LIdx<D>::B * i);
    }
    wave_lds_sync();
    return u;
}

// |x| per group of 8 and the sign bits; with PARITY (IQ2_XXS, IQ2_XS, IQ3_XXS) an odd count of
// negatives leaves the least important weight's sign flipped and keeps 7 bits
// (ggml-quants.c:3336-3356); without it (IQ2_S, IQ3_S) all 8 bits are kept (:4222-4231)
template <int N, bool PARITY>
__device__ __forceinline__ void make_signs(const float (&x)[N], const float (&w)[N], float (&xval)[N], uint32_t (&sg)[N / 8]) {
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
        int nflip = 0;
        uint32_t s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (x[8 * k + i] >= 0) xval[8 * k + i] = x[8 * k + i];
            else { xval[8 * k + i] = -x[8 * k + i]; ++nflip; s |= 1u << i; }
        }
        if (PARITY && (nflip % 2)) {
            int imin = 0;
            float mn = w[8 * k] * x[8 * k] * x[8 * k];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
                const float ax = w[8 * k + i] * x[8 * k + i] * x[8 * k + i];
                if (ax < mn) { mn = ax; imin = i; }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (i == imin) xval[8 * k + i] = -xval[8 * k + i];
            s ^= 1u << imin;
        }
        sg[k] = PARITY ? (s & 127) : s;
    }
}

// level index of a lattice group (2 bits per coordinate for D = 8, 3 bits for D = 4)
template <int D, int N>
__device__ __forceinline__ int level_index(const int (&L)[N], int off) {
    constexpr int B = D == 8 ? 2 : 3;
    int u = 0;
#pragma unroll
    for (int i = 0; i < D; ++i) u |= L[off + i] << (B * i);
    return u;
}

template <int N>
__device__ __forceinline__ void sums_2l1(const float (&xval)[N], const float (&w)[N], const int (&L)[N], float& sumqx, float& sumq2) {
    sumqx = 0; sumq2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float q = (float)(2 * L[i] + 1);
        sumqx += w[i] * xval[i] * q;
        sumq2 += w[i] * q * q;
    }
}

// A lattice group's levels are kept as its level index (B bits per coordinate: the map's key), one
// register per group instead of one per weight; the search states of the 32-weight sub-blocks
// otherwise do not fit the register file twice over.
// the group at `off` rounded at inverse scale id: nearest_int(0.5 (id x - 1)) clamped to the levels
template <int D, int N, int KMAXQ>
__device__ __forceinline__ int round_group(const float (&xval)[N], int off, float id) {
    int u = 0;
#pragma unroll
    for (int i = 0; i < D; ++i) {
        const int l = nearest_int(0.5f * (id * xval[off + i] - 1));
        u |= tmax(0, tmin(KMAXQ - 1, l)) << (LIdx<D>::B * i);
    }
    return u;
}

// sums_2l1 over groups held as level indices (element order)
template <int D, int N>
__device__ __forceinline__ void sums_idx(const float (&xval)[N], const float (&w)[N], const int (&idx)[N / D], float& sumqx,
                                         float& sumq2) {
    sumqx = 0; sumq2 = 0;
#pragma unroll
    for (int k = 0; k < N / D; ++k) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const float q = (float)(2 * LIdx<D>::level(idx[k], i) + 1);
            // w passes an empty asm so that w*xval is not hoisted out of the trial loop (N live
            // registers more, one wave less per SIMD)
            float wi = w[D * k + i];
            asm volatile("" : "+v"(wi));
            sumqx += wi * xval[D * k + i] * q;
            sumq2 += wi * q * q;
        }
    }
}

// ---------------------------------------------------------------- the lattice types (IQ2_*, IQ3_*)

// Result of one sub-block. An empty sub-block (its early exit in the reference) writes no bytes:
// gidx and signs stay zero and `empty` is set.
struct SubOut {
    float scale;
    int shift;          // IQ1_S: +1 / -1; IQ1_M: sign combination 0..3
    bool empty;
    int gidx[8];        // grid point per lattice group
    uint32_t signs[4];  // per 8 weights
};

// The trial search of IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S: trial scales id = (2 kMaxQ - 1 + is*step)/max,
// levels by rounding, groups off the grid snapped to their best neighbour; the best trial's levels
// are kept; then the groups that were off the grid (REFIT_ALL: every group) are requantized at the
// best scale and the scale refitted (ggml-quants.c:3540-3616, :5176-5252, :4014-4086, :4250-4322).
// SET_L_IN_REFIT: the refit writes the rounded levels before the map lookup (IQ2_XS, IQ2_S);
// otherwise the levels come from the grid point (IQ3_*): the same values either way.
// All lanes of the wave run it (the neighbour searches are wave-wide); a lane whose sub-block is
// empty (`live` false) searches nothing and its result is not used.
template <int N, int D, int KMAXQ, int IS_LO, int IS_HI, bool ONGRID_INIT, bool REFIT_ALL, bool SET_L_IN_REFIT,
          int R = nb_piece<D>()>
__device__ __forceinline__ float lattice_search(bool live, const float (&xval)[N], const float (&w)[N], const NbCtx& nc,
                                                float max, float step, const IqDeviceTable& tab, const uint8_t* grid,
                                                int (&idx)[N / D]) {
    constexpr int NG = N / D;
    bool on[NG];
#pragma unroll
    for (int k = 0; k < NG; ++k) on[k] = ONGRID_INIT;
    float scale = max / (float)(2 * KMAXQ - 1);
    float best = 0;
    for (int is = IS_LO; is <= IS_HI; ++is) {
        const float id = ((float)(2 * KMAXQ - 1) + (float)is * step) / max;
        const float this_scale = 1 / id;
        int ia[NG], ga[NG];
        bool ona[NG];
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            ia[k] = round_group<D, N, KMAXQ>(xval, D * k, id);
            ga[k] = tab.map[ia[k]];
        }
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            ona[k] = ga[k] >= 0;
            const int nu = wave_best_neighbour<D, N, R>(nc, k, live && ga[k] < 0, ga[k], xval, this_scale, tab.nb, grid);
            if (ga[k] < 0) ia[k] = nu;
        }
        float sumqx, sumq2;
        sums_idx<D, N>(xval, w, ia, sumqx, sumq2);
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            scale = sumqx / sumq2;
            best = scale * sumqx;
#pragma unroll
            for (int k = 0; k < NG; ++k) { idx[k] = ia[k]; on[k] = ona[k]; }
        }
    }
    int n_off = 0;
#pragma unroll
    for (int k = 0; k < NG; ++k) n_off += on[k] ? 0 : 1;
    const bool refit = live && n_off > 0 && scale > 0;
    const float id = 1 / scale;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
        // the rounded levels, or the best neighbour's when off the grid (SET_L_IN_REFIT only
        // changes when the levels are written, not their values)
        const bool redo = refit && (REFIT_ALL || !on[k]);
        const int u = round_group<D, N, KMAXQ>(xval, D * k, id);
        const int gi = tab.map[u];
        const int nu = wave_best_neighbour<D, N, R>(nc, k, redo && gi < 0, gi, xval, scale, tab.nb, grid);
        if (redo) idx[k] = gi < 0 ? nu : u;
    }
    if (refit) {
        float sumqx, sumq2;
        sums_idx<D, N>(xval, w, idx, sumqx, sumq2);
        if (sumq2 > 0) scale = sumqx / sumq2;
    }
    return scale;
}

// sqrt(w) of the sub-block into this lane's LDS row, read by the neighbour searches
template <int N>
__device__ __forceinline__ void put_sqrt_w(const NbCtx& nc, const float (&w)[N]) {
    float4* row = reinterpret_cast<float4*>(const_cast<float*>(nc.wrows) + threadIdx.x * N);
#pragma unroll
    for (int v = 0; v < N / 4; ++v) row[wrow_at<N>((int)threadIdx.x, v)] = make_float4(sqrtf(w[4 * v]), sqrtf(w[4 * v + 1]), sqrtf(w[4 * v + 2]), sqrtf(w[4 * v + 3]));
}

// A lattice group's levels are kept as its level index (B bits per coordinate: the map's key), one
// register per group instead of one per weight; the search states of the 32-weight sub-blocks
// otherwise do not fit the register file twice over.
// IQ2_XXS -- quantize_row_iq2_xxs_impl (ggml-quants.c:3295-3471): 32-weight sub-blocks, 4 groups of 8
__device__ __forceinline__ SubOut iq2_xxs_sub(const float (&x)[32], const float (&w)[32], const IqDeviceTable& tab,
                                              const uint8_t* grid, const NbCtx& nc) {
    constexpr int KMAXQ = 3;
    SubOut o{};
    float xval[32];
    put_sqrt_w<32>(nc, w);
    uint32_t sg[4];
    make_signs<32, true>(x, w, xval, sg);
    float max = xval[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) max = tmax(max, xval[i]);
    float scale;
    {
        int Lq[32];     // make_qp_quants' levels never reach the output: scale > 0 below refits every group
        scale = make_qp_quants<32>(KMAXQ + 1, xval, Lq, w);
    }
    const float eff_max = scale * KMAXQ;
    // the reference's early exits (max < GROUP_MAX_EPS, eff_max <= 0) leave the sub-block empty
    const bool live = !(max < GROUP_MAX_EPS) && eff_max > 0;
    o.empty = !live;
    float best = 0;
    int idx[4] = {0, 0, 0, 0};
    for (int is = -6; is <= 6; ++is) {
        const float id = ((float)(2 * KMAXQ - 1) + (float)is * 0.1f) / eff_max;
        const float this_scale = 1 / id;
        int ia[4], ga[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ia[k] = round_group<8, 32, KMAXQ>(xval, 8 * k, id);
            ga[k] = tab.map[ia[k]];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int nu = wave_best_neighbour<8, 32>(nc, k, live && ga[k] < 0, ga[k], xval, this_scale, tab.nb, grid);
            if (ga[k] < 0) ia[k] = nu;
        }
        float sumqx, sumq2;
        sums_idx<8, 32>(xval, w, ia, sumqx, sumq2);
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            scale = sumqx / sumq2;
            best = scale * sumqx;
#pragma unroll
            for (int k = 0; k < 4; ++k) idx[k] = ia[k];
        }
    }
    // every group requantized at the best scale (ggml-quants.c:3411-3432)
    const bool refit = live && scale > 0;
    const float id = 1 / scale;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int u = round_group<8, 32, KMAXQ>(xval, 8 * k, id);
        const int gi = tab.map[u];
        const int nu = wave_best_neighbour<8, 32>(nc, k, refit && gi < 0, gi, xval, scale, tab.nb, grid);
        if (refit) idx[k] = gi < 0 ? nu : u;
    }
    if (refit) {
        float sumqx, sumq2;
        sums_idx<8, 32>(xval, w, idx, sumqx, sumq2);
        if (sumq2 > 0) scale = sumqx / sumq2;
    }
    if (!live) return o;
    if (scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 4; ++k) sg[k] = (~sg[k]) & 127;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) { o.gidx[k] = tab.map[idx[k]]; o.signs[k] = sg[k]; }
    o.scale = scale;
    return o;
}

// IQ2_XS -- quantize_row_iq2_xs_impl (ggml-quants.c:3473-3651); IQ2_S -- quantize_row_iq2_s_impl
// (:5114-5280): 16-weight sub-blocks, 2 lattice groups of 8
template <bool XS>
__device__ __forceinline__ SubOut iq2_16_sub(const float (&x)[16], const float (&w)[16], const IqDeviceTable& tab,
                                             const uint8_t* grid, const NbCtx& nc) {
    SubOut o{};
    float xval[16];
    put_sqrt_w<16>(nc, w);
    uint32_t sg[2];
    make_signs<16, XS>(x, w, xval, sg);
    float max = xval[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) max = tmax(max, xval[i]);
    const bool live = !(max < (XS ? GROUP_MAX_EPS : 1e-8f));   // GROUP_MAX_EPS_IQ2_S = 1e-8f
    o.empty = !live;
    int idx[2] = {0, 0};
    float scale = lattice_search<16, 8, 3, -9, 9, true, false, true, XS ? 8 : 4>(live, xval, w, nc, max, 0.1f, tab, grid, idx);
    if (!live) return o;
    if (scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 2; ++k) sg[k] = XS ? ((~sg[k]) & 127) : ((~sg[k]) & 255);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) { o.gidx[k] = tab.map[idx[k]]; o.signs[k] = sg[k]; }
    o.scale = scale;
    return o;
}

// IQ3_XXS -- quantize_row_iq3_xxs_impl(256) (ggml-quants.c:3939-4151); IQ3_S -- quantize_row_iq3_s_impl
// (:4170-4353): 32-weight sub-blocks, 8 lattice groups of 4
template <bool XXS>
__device__ __forceinline__ SubOut iq3_sub(const float (&x)[32], const float (&w)[32], const IqDeviceTable& tab,
                                          const uint8_t* grid, const NbCtx& nc) {
    SubOut o{};
    float xval[32];
    put_sqrt_w<32>(nc, w);
    uint32_t sg[4];
    make_signs<32, XXS>(x, w, xval, sg);
    float max = xval[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) max = tmax(max, xval[i]);
    const bool live = !(XXS ? (max < 1e-8f) : (max == 0.f));   // GROUP_MAX_EPS_IQ3_XXS = 1e-8f; IQ3_S: !max
    o.empty = !live;
    int idx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float scale;
    if constexpr (XXS) scale = lattice_search<32, 4, 8, -15, 15, true, false, false>(live, xval, w, nc, max, 0.2f, tab, grid, idx);
    else scale = lattice_search<32, 4, 8, -9, 9, false, true, false, 6>(live, xval, w, nc, max, 0.2f, tab, grid, idx);
    if (!live) return o;
    if (scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 4; ++k) sg[k] = XXS ? ((~sg[k]) & 127) : ((~sg[k]) & 255);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) o.gidx[k] = tab.map[idx[k]];
#pragma unroll
    for (int k = 0; k < 4; ++k) o.signs[k] = sg[k];
    o.scale = scale;
    return o;
}

// ---------------------------------------------------------------- IQ1_S / IQ1_M

// Ascending order of (x, original index): a bitonic network on the composite key. This is the order
// of a stable sort by x, which is what glibc's qsort (a merge sort) gives the reference
// (ggml-quants.c:4567, :4761); -0 and +0 compare equal. w travels with its x.
template <int N>
__device__ __forceinline__ void sort_pairs(float (&x)[N], int (&ix)[N], float (&w)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const bool up = (i & k) == 0;
                    const bool gt = x[i] > x[l] || (x[i] == x[l] && ix[i] > ix[l]);
                    if (gt == up) {
                        const float tx = x[i]; x[i] = x[l]; x[l] = tx;
                        const int ti = ix[i]; ix[i] = ix[l]; ix[l] = ti;
                        const float tw = w[i]; w[i] = w[l]; w[l] = tw;
                    }
                }
            }
        }
    }
}

// level (0, 1, 2) of every weight from the split points b1 <= b2 of the sorted order: weight i's
// position in the stable order is the count of weights before it
template <int N>
__device__ __forceinline__ void split_levels(const float (&x)[N], int b1, int b2, int (&L)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int rank = 0;
#pragma unroll
        for (int j = 0; j < N; ++j) rank += (x[j] < x[i] || (x[j] == x[i] && j < i)) ? 1 : 0;
        L[i] = rank < b1 ? 0 : (rank < b2 ? 1 : 2);
    }
}

constexpr float IQ1S_DELTA = 0.125f;    // ggml-common.h IQ1S_DELTA
constexpr float IQ1M_DELTA = 0.125f;    // ggml-common.h IQ1M_DELTA

__device__ __forceinline__ float pick3(int lv, float a, float b, float c) { return lv == 0 ? a : (lv == 1 ? b : c); }

// iq1_find_best_neighbour2 (ggml-quants.c:4444-4499) over the listed neighbours. A point's coordinate
// value q (1, 3, 5 for levels 0, 1, 2) selects the level value g = -1 + d, d, 1 + d (d = +-delta);
// here g is formed as 0.5 q + gc with gc = d - 1.5, which is exact (the values are small dyadic
// rationals), so the distance sees the reference's constants. The reference scans the whole grid
// when no listed point gives a distance below FLT_MAX and aborts if that scan finds none; with finite
// inputs a listed point always wins.
#ifndef IQ1_RUN
#define IQ1_RUN 4
#endif
__device__ __forceinline__ int iq1_neighbour(const uint16_t* __restrict__ nb, const uint8_t* grid, const float (&xv)[8],
                                             const float (&wv)[8], float scale, float gc, int (&Lg)[8]) {
    const int n = nb[0];
    float best = FLT_BIG;
    int gi = nb[1];
    // the list in runs of IQ1_RUN entries: a run's entries and codebook points are all requested
    // before its distances are formed (the lists hold ~300 points); entries past the end re-read the
    // last one and are left out, and the first strict minimum in list order wins as in the reference
    for (int j0 = 1; j0 <= n; j0 += IQ1_RUN) {
        int jj[IQ1_RUN];
#pragma unroll
        for (int e = 0; e < IQ1_RUN; ++e) jj[e] = nb[min(j0 + e, n)];
        uint2 gp[IQ1_RUN];   // the points stay packed (one byte per coordinate) until used
#pragma unroll
        for (int e = 0; e < IQ1_RUN; ++e) gp[e] = reinterpret_cast<const uint2*>(grid)[jj[e]];
#pragma unroll
        for (int e = 0; e < IQ1_RUN; ++e) {
            float d2 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float q = (float)(((i < 4 ? gp[e].x : gp[e].y) >> (8 * (i & 3))) & 0xff);
                const float diff = scale * (0.5f * q + gc) - xv[i];
                d2 += wv[i] * diff * diff;
            }
            if (j0 + e <= n && d2 < best) { best = d2; gi = jj[e]; }
        }
    }
    int q[8];
    grid_point<8>(grid, gi, q);
#pragma unroll
    for (int i = 0; i < 8; ++i) Lg[i] = (q[i] - 1) / 2;
    return gi;
}

// snap the groups of 8 to the grid, then refit the scale if any group was off the grid
// (ggml-quants.c:4602-4629 for IQ1_S, :4824-4852 for IQ1_M, where each group has its own signs)
template <int N>
__device__ __forceinline__ float iq1_snap(const float (&x)[N], const float (&w)[N], int (&L)[N], float scale, const bool (&pos)[N / 8],
                                          const IqDeviceTable& tab, const uint8_t* grid, int (&gidx)[8]) {
    constexpr float XP0 = -1 + IQ1S_DELTA, XP1 = IQ1S_DELTA, XP2 = 1 + IQ1S_DELTA;
    constexpr float XM0 = -1 - IQ1S_DELTA, XM1 = -IQ1S_DELTA, XM2 = 1 - IQ1S_DELTA;
    bool all_on = true;
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
        int gi = tab.map[level_index<8, N>(L, 8 * k)];
        if (gi < 0) {
            all_on = false;
            float xv[8], wv[8];
            int Lg[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) { xv[i] = x[8 * k + i]; wv[i] = w[8 * k + i]; }
            gi = iq1_neighbour(tab.nb + nb_offset(gi), grid, xv, wv, scale, pos[k] ? IQ1S_DELTA - 1.5f : -IQ1S_DELTA - 1.5f, Lg);
#pragma unroll
            for (int i = 0; i < 8; ++i) L[8 * k + i] = Lg[i];
        }
        gidx[k] = gi;
    }
    if (!all_on) {
        float sumqx = 0, sumq2 = 0;
#pragma unroll
        for (int k = 0; k < N / 8; ++k) {
            int q[8];
            grid_point<8>(grid, gidx[k], q);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int lv = (q[j] - 1) / 2;
                const float qq = pos[k] ? pick3(lv, XP0, XP1, XP2) : pick3(lv, XM0, XM1, XM2);
                sumqx += w[8 * k + j] * qq * x[8 * k + j];
                sumq2 += w[8 * k + j] * qq * qq;
            }
        }
        if (sumqx > 0 && sumq2 > 0) scale = sumqx / sumq2;
    }
    return scale;
}

// IQ1_S sub-block of 32 -- quantize_row_iq1_s_impl (ggml-quants.c:4509-4671)
template <class R>
__device__ __forceinline__ SubOut iq1_s_sub(const float (&x)[32], const float (&w)[32], const IqDeviceTable& tab,
                                            const uint8_t* grid, const R& reload) {
    constexpr float XP0 = -1 + IQ1S_DELTA, XP1 = IQ1S_DELTA, XP2 = 1 + IQ1S_DELTA;
    constexpr float XM0 = -1 - IQ1S_DELTA, XM1 = -IQ1S_DELTA, XM2 = 1 - IQ1S_DELTA;
    SubOut o{};
    o.empty = true;
    o.shift = 1;
    float max = fabsf(x[0]);
#pragma unroll
    for (int i = 1; i < 32; ++i) max = tmax(max, fabsf(x[i]));
    if (max < 1e-12f) return o;   // GROUP_MAX_EPS_IQ1_S
    float sx[32], sw[32];
    int si[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) { sx[i] = x[i]; si[i] = i; sw[i] = w[i]; }
    sort_pairs<32>(sx, si, sw);
    float sumx[33], sumw[33];
    sumx[0] = sumw[0] = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) { sumx[j + 1] = sumx[j] + sw[j] * sx[j]; sumw[j + 1] = sumw[j] + sw[j]; }
    float best_score = -FLT_BIG, scale = max;
    int b1 = -1, b2 = -1, best_shift = 0;
    // every split i1 <= i2 in the reference's order; i1 is the same in every lane, so the prefix
    // sums at i1 are picked once per i1 and the inner loop indexes registers by constants
    for (int i1 = 0; i1 <= 32; ++i1) {
        // the prefix sums pass through an empty asm each step: otherwise the i1-invariant products of
        // the unrolled i2 loop are hoisted out as ~130 extra live registers (half the occupancy)
#pragma unroll
        for (int t = 0; t <= 32; ++t) {
            asm volatile("" : "+v"(sumx[t]));
            asm volatile("" : "+v"(sumw[t]));
        }
        float x1 = 0, w1 = 0;
#pragma unroll
        for (int t = 0; t <= 32; ++t)
            if (t == i1) { x1 = sumx[t]; w1 = sumw[t]; }
#pragma unroll
        for (int i2 = 0; i2 <= 32; ++i2) {
            if (i2 < i1) continue;
            float sumqx = (x1 - sumx[0]) * XP0 + (sumx[i2] - x1) * XP1 + (sumx[32] - sumx[i2]) * XP2;
            float sumq2 = (w1 - sumw[0]) * XP0 * XP0 + (sumw[i2] - w1) * XP1 * XP1 + (sumw[32] - sumw[i2]) * XP2 * XP2;
            if (sumq2 > 0 && sumqx * sumqx > best_score * sumq2) {
                scale = sumqx / sumq2; best_score = scale * sumqx; b1 = i1; b2 = i2; best_shift = 1;
            }
            sumqx = (x1 - sumx[0]) * XM0 + (sumx[i2] - x1) * XM1 + (sumx[32] - sumx[i2]) * XM2;
            sumq2 = (w1 - sumw[0]) * XM0 * XM0 + (sumw[i2] - w1) * XM1 * XM1 + (sumw[32] - sumw[i2]) * XM2 * XM2;
            if (sumq2 > 0 && sumqx * sumqx > best_score * sumq2) {
                scale = sumqx / sumq2; best_score = scale * sumqx; b1 = i1; b2 = i2; best_shift = -1;
            }
        }
    }
    if (b1 < 0 || b2 < 0 || best_shift == 0) return o;
    o.empty = false;
    float xr[32], wr[32];
    reload(xr, wr);
    int L[32];
    split_levels<32>(xr, b1, b2, L);
    if (scale < 0) {
#pragma unroll
        for (int j = 0; j < 32; ++j) L[j] = 2 - L[j];
        scale = -scale;
        best_shift = -best_shift;
    }
    const bool p = best_shift == 1;
    const bool pos[4] = {p, p, p, p};
    o.scale = iq1_snap<32>(xr, wr, L, scale, pos, tab, grid, o.gidx);
    o.shift = best_shift;
    return o;
}

// IQ1_M sub-block of 16 -- quantize_row_iq1_m_impl (ggml-quants.c:4693-4916); VARIANT 1 is the
// earlier search that sums every split directly (variants/ggml-quants.pre-f95b0d9539.c:4773-4860)
template <int VARIANT, class R>
__device__ __forceinline__ SubOut iq1_m_sub(const float (&x)[16], const float (&w)[16], const IqDeviceTable& tab,
                                            const uint8_t* grid, const R& reload) {
    constexpr float XP0 = -1 + IQ1M_DELTA, XP1 = IQ1M_DELTA, XP2 = 1 + IQ1M_DELTA;
    constexpr float XM0 = -1 - IQ1M_DELTA, XM1 = -IQ1M_DELTA, XM2 = 1 - IQ1M_DELTA;
    SubOut o{};
    o.empty = true;
    o.shift = 0;
    float max = fabsf(x[0]);
#pragma unroll
    for (int i = 1; i < 16; ++i) max = tmax(max, fabsf(x[i]));
    if (max < 1e-7f) return o;   // GROUP_MAX_EPS_IQ1_M
    float sx[16], sw[16];
    int si[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) { sx[i] = x[i]; si[i] = i; sw[i] = w[i]; }
    sort_pairs<16>(sx, si, sw);
    float best_score = -FLT_BIG, scale = max;
    int b1 = -1, b2 = -1, best_k = -1;
    float sumqx[4], sumq2[4];
    if constexpr (VARIANT == 0) {
        // prefix sums per half of the sub-block (ggml-quants.c:4774-4820)
        float px0[17], px1[17], pw0[17], pw1[17];
        px0[0] = px1[0] = pw0[0] = pw1[0] = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool h1 = si[j] >= 8;
            const float a = sw[j] * sx[j];
            px0[j + 1] = h1 ? px0[j] : px0[j] + a;
            px1[j + 1] = h1 ? px1[j] + a : px1[j];
            pw0[j + 1] = h1 ? pw0[j] : pw0[j] + sw[j];
            pw1[j + 1] = h1 ? pw1[j] + sw[j] : pw1[j];
        }
        const float tx0 = px0[16], tx1 = px1[16], tw0 = pw0[16], tw1 = pw1[16];
        constexpr float P2 = XP2, M2 = XM2;
        const float cp1 = XP0 * XP0 - XP1 * XP1, cp2 = XP1 * XP1 - XP2 * XP2;
        const float cm1 = XM0 * XM0 - XM1 * XM1, cm2 = XM1 * XM1 - XM2 * XM2;
        for (int i1 = 0; i1 <= 16; ++i1) {
            // (as in the IQ1_S search: no hoisting of the i1-invariant terms)
#pragma unroll
            for (int t = 0; t <= 16; ++t) {
                asm volatile("" : "+v"(px0[t]));
                asm volatile("" : "+v"(px1[t]));
                asm volatile("" : "+v"(pw0[t]));
                asm volatile("" : "+v"(pw1[t]));
            }
            float a0 = 0, a1 = 0, c0 = 0, c1 = 0;
#pragma unroll
            for (int t = 0; t <= 16; ++t)
                if (t == i1) { a0 = px0[t]; a1 = px1[t]; c0 = pw0[t]; c1 = pw1[t]; }
#pragma unroll
            for (int i2 = 0; i2 <= 16; ++i2) {
                if (i2 < i1) continue;
                const float s0 = a0 + px0[i2], s1 = a1 + px1[i2];
                const float qx_p0 = tx0 * P2 - s0, qx_m0 = tx0 * M2 - s0;
                const float qx_p1 = tx1 * P2 - s1, qx_m1 = tx1 * M2 - s1;
                const float q2_p0 = tw0 * P2 * P2 + c0 * cp1 + pw0[i2] * cp2;
                const float q2_m0 = tw0 * M2 * M2 + c0 * cm1 + pw0[i2] * cm2;
                const float q2_p1 = tw1 * P2 * P2 + c1 * cp1 + pw1[i2] * cp2;
                const float q2_m1 = tw1 * M2 * M2 + c1 * cm1 + pw1[i2] * cm2;
                sumqx[0] = qx_p0 + qx_p1; sumqx[1] = qx_p0 + qx_m1;
                sumqx[2] = qx_m0 + qx_p1; sumqx[3] = qx_m0 + qx_m1;
                sumq2[0] = q2_p0 + q2_p1; sumq2[1] = q2_p0 + q2_m1;
                sumq2[2] = q2_m0 + q2_p1; sumq2[3] = q2_m0 + q2_m1;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (sumq2[k] > 0 && sumqx[k] * sumqx[k] > best_score * sumq2[k]) {
                        scale = sumqx[k] / sumq2[k]; best_score = scale * sumqx[k];
                        b1 = i1; b2 = i2; best_k = k;
                    }
                }
            }
        }
    } else {
        // Every split's four sums run over the sorted weights j = 0..15 in order, level 0 below i1,
        // 1 below i2, 2 from i2 on. The running sums after the level-0 run depend on i1 only (p0),
        // and after the level-1 run on (i1, i2), growing by one term per i2 (p1); only the level-2
        // tail is added per split. The additions and their order are those of the direct sums.
        // term(j, l, k): the contribution of sorted weight j at level l to sum k (sums 0 and 3 take
        // the +delta / -delta value in both halves, 1 and 2 swap them in the second half)
        auto add_terms = [&](float (&qx)[4], float (&q2)[4], int j, float gp, float gm) {
            const float ap = sw[j] * gp * sx[j], am = sw[j] * gm * sx[j];
            const float bp = sw[j] * gp * gp, bm = sw[j] * gm * gm;
            const bool h0 = si[j] < 8;
            qx[0] += ap; q2[0] += bp;
            qx[3] += am; q2[3] += bm;
            if (h0) { qx[1] += ap; q2[1] += bp; qx[2] += am; q2[2] += bm; }
            else    { qx[1] += am; q2[1] += bm; qx[2] += ap; q2[2] += bp; }
        };
        float p0x[4] = {0, 0, 0, 0}, p0q[4] = {0, 0, 0, 0};
        for (int i1 = 0; i1 <= 16; ++i1) {
            float p1x[4], p1q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) { p1x[k] = p0x[k]; p1q[k] = p0q[k]; }
            for (int i2 = i1; i2 <= 16; ++i2) {
                // sw passes an empty asm each split: otherwise the split-invariant products of every
                // weight and level are hoisted out of the loops and spill
#pragma unroll
                for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(sw[j]));
#pragma unroll
                for (int k = 0; k < 4; ++k) { sumqx[k] = p1x[k]; sumq2[k] = p1q[k]; }
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j >= i2) add_terms(sumqx, sumq2, j, XP2, XM2);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (sumq2[k] > 0 && sumqx[k] * sumqx[k] > best_score * sumq2[k]) {
                        scale = sumqx[k] / sumq2[k]; best_score = scale * sumqx[k];
                        b1 = i1; b2 = i2; best_k = k;
                    }
                }
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j == i2) add_terms(p1x, p1q, j, XP1, XM1);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j == i1) add_terms(p0x, p0q, j, XP0, XM0);
        }
    }
    if (b1 < 0 || b2 < 0 || best_k < 0) return o;
    o.empty = false;
    float xr[16], wr[16];
    reload(xr, wr);
    int L[16];
    split_levels<16>(xr, b1, b2, L);
    if (scale < 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) L[j] = 2 - L[j];
        scale = -scale;
        best_k = 3 - best_k;
    }
    const bool pos[2] = {best_k < 2, best_k % 2 == 0};
    o.scale = iq1_snap<16>(xr, wr, L, scale, pos, tab, grid, o.gidx);
    o.shift = best_k;
    return o;
}

// ---------------------------------------------------------------- kernels

// per-lane results parked for the packing lane
struct Park {
    float scale;
    int l;              // sub-block scale code
    int shift;
    int empty;
    int gidx[8];
    uint32_t signs[4];
};

enum Kind { K_IQ2_XXS, K_IQ2_XS, K_IQ2_S, K_IQ3_XXS, K_IQ3_S, K_IQ1_S, K_IQ1_M0, K_IQ1_M1 };

// D: lattice group size; N: sub-block; BS: block bytes; GBYTES: codebook bytes; TWO: sigma2 = 2 sumx2 / 256
// (else sumx2 / 256)
template <int K> struct Cfg;
// WPE: the waves per SIMD the register allocation is held to. The 32-weight lattice searches need
// ~200 registers; at 3 waves (168) a few spill, which costs less than the lost latency hiding at 2
// (measured: IQ3_XXS 7.6 -> 9.4 GB/s, IQ2_XXS 8.5 -> 10.9); 4 spills them by the thousand. The
// 16-weight and IQ1_S searches fit 128 with few spills (IQ1_S 21.5 -> 23.8 at 4); IQ1_M keeps 3
// (23.1 at 4, 24.0 at 3).
template <> struct Cfg<K_IQ2_XXS> { static constexpr int D = 8, N = 32, BS = 66, GBYTES = 256 * 8, WPE = 3; static constexpr bool TWO = false; };
template <> struct Cfg<K_IQ2_XS> { static constexpr int D = 8, N = 16, BS = 74, GBYTES = 512 * 8, WPE = 4; static constexpr bool TWO = false; };
template <> struct Cfg<K_IQ2_S> { static constexpr int D = 8, N = 16, BS = 82, GBYTES = 1024 * 8, WPE = 4; static constexpr bool TWO = true; };
template <> struct Cfg<K_IQ3_XXS> { static constexpr int D = 4, N = 32, BS = 98, GBYTES = 256 * 4, WPE = 3; static constexpr bool TWO = true; };
template <> struct Cfg<K_IQ3_S> { static constexpr int D = 4, N = 32, BS = 110, GBYTES = 512 * 4, WPE = 3; static constexpr bool TWO = true; };
template <> struct Cfg<K_IQ1_S> { static constexpr int D = 8, N = 32, BS = 50, GBYTES = 2048 * 8, WPE = 4; static constexpr bool TWO = true; };
template <> struct Cfg<K_IQ1_M0> { static constexpr int D = 8, N = 16, BS = 56, GBYTES = 2048 * 8, WPE = 3; static constexpr bool TWO = true; };
template <> struct Cfg<K_IQ1_M1> { static constexpr int D = 8, N = 16, BS = 56, GBYTES = 2048 * 8, WPE = 3; static constexpr bool TWO = true; };

template <int K>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(Cfg<K>::WPE))) void k_iqgrid(const void* __restrict__ src, int kind, uint8_t* __restrict__ dst, int64_t nsb,
                                               int64_t sbpr, const float* __restrict__ imx, IqDeviceTable tab) {
    using C = Cfg<K>;
    constexpr int N = C::N, G = 256 / N, SBW = WG / G;
    constexpr bool IQ1 = K == K_IQ1_S || K == K_IQ1_M0 || K == K_IQ1_M1;
    __shared__ __align__(16) uint8_t grid[C::GBYTES];
    __shared__ __align__(16) uint16_t otile[SBW * C::BS / 2];
    // sqrt(w) of the lattice types' neighbour searches in per-lane LDS rows; once the searches are
    // done the same bytes hold the parked per-lane results
    constexpr int WA_BYTES = IQ1 ? 0 : N * WG * 4, PARK_BYTES = SBW * G * (int)sizeof(Park);
    __shared__ __align__(16) uint8_t wa_park[WA_BYTES > PARK_BYTES ? WA_BYTES : PARK_BYTES];
    __shared__ NbWave<C::D> nbw[IQ1 ? 1 : WG / 64];
    Park (*park)[G] = reinterpret_cast<Park (*)[G]>(wa_park);
    const NbCtx nc{&nbw[IQ1 ? 0 : threadIdx.x / 64], reinterpret_cast<const float*>(wa_park), (int)(threadIdx.x & ~63u)};
    for (int i = threadIdx.x; i < C::GBYTES / 16; i += WG)
        reinterpret_cast<uint4*>(grid)[i] = reinterpret_cast<const uint4*>(tab.grid)[i];
    if constexpr (!IQ1) {
        // every owner record starts as an empty list at offset 0 (scale, offset, first piece, length
        // all zero), so a record is never read before it names a list of the table
        reinterpret_cast<float4*>(nbw[threadIdx.x / 64].rec[threadIdx.x % 64])[C::D / 4] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    // the thread's index rebuilt from the wave's index (a scalar) and the lane where it is needed again
    // after the searches, so that no register holds it through them
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    auto tid = [&] { return wave * 64 + (int)__lane_id(); };
    const int lsb = threadIdx.x / G, sub = threadIdx.x % G;
    const int64_t sb0 = (int64_t)blockIdx.x * SBW;
    const int64_t sb = sb0 + lsb;
    const bool active = sb < nsb;
    const int64_t sbc = active ? sb : nsb - 1;
    float x[N];
    load_weights<N>(src, kind, sbc * 256 + sub * N, x);
    float sq[N];
#pragma unroll
    for (int i = 0; i < N; ++i) sq[i] = x[i] * x[i];
    const float sumx2 = group_sum<G, N>(sq, sub);
    const float sigma2 = C::TWO ? 2 * sumx2 / 256 : sumx2 / 256;
    auto weights = [&](const float (&xv)[N], float (&wv)[N]) {
        if (imx) {
            const float* qw = imx + (sbc % sbpr) * 256 + sub * N;
#pragma unroll
            for (int i = 0; i < N; ++i) wv[i] = qw[i] * sqrtf(sigma2 + xv[i] * xv[i]);
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) wv[i] = K == K_IQ2_S ? 0.25f * sigma2 + xv[i] * xv[i] : xv[i] * xv[i];
        }
    };
    // the IQ1 searches hold sorted copies and prefix sums: x and w are read again afterwards (same
    // values) rather than kept in registers through them, from the element offset, importance offset
    // and sigma^2 parked in this thread's LDS slot (no register holds them through the search). With
    // a 16-bit source the sub-block's raw values (2N bytes, at most a Park) wait in the thread's own
    // park slot, which its parked result overwrites only after the last reload; an f32 source is
    // read again from global memory.
    static_assert(!IQ1 || 2 * N <= (int)sizeof(Park), "a sub-block's 16-bit values fit a park slot");
    __shared__ uint4 stash[IQ1 ? WG : 1];
    const bool raw16 = kind != SRC_F32;
    if constexpr (IQ1) {
        const uint64_t eo = (uint64_t)(sbc * 256 + sub * N);
        stash[threadIdx.x] = make_uint4((uint32_t)eo, (uint32_t)(eo >> 32), (uint32_t)((sbc % sbpr) * 256 + sub * N),
                                        __float_as_uint(sigma2));
        if (raw16) {
            const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + eo);
            uint4* slot = reinterpret_cast<uint4*>(&park[lsb][sub]);
#pragma unroll
            for (int k = 0; k < N / 8; ++k) slot[k] = p[k];
        }
    }
    auto reload = [&](float (&xv)[N], float (&wv)[N]) {
        const uint4 st = stash[tid()];
        if (raw16) {
            // the same widening as load_weights, from the raw values in the park slot
            const uint4* slot = reinterpret_cast<const uint4*>(&park[tid() / G][tid() % G]);
            const bool bf = kind == SRC_BF16;
#pragma unroll
            for (int k = 0; k < N / 8; ++k) {
                const uint4 v = slot[k];
                const uint32_t c[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t h = (j & 1) ? (c[j / 2] >> 16) : (c[j / 2] & 0xffffu);
                    xv[8 * k + j] = bf ? bf16_to_f32(h) : f16_to_f32(h);
                }
            }
        } else {
            load_weights<N>(src, kind, (int64_t)(((uint64_t)st.y << 32) | st.x), xv);
        }
        const float s2 = __uint_as_float(st.w);
        if (imx) {
            const float* qw = imx + st.z;
#pragma unroll
            for (int i = 0; i < N; ++i) wv[i] = qw[i] * sqrtf(s2 + xv[i] * xv[i]);
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) wv[i] = xv[i] * xv[i];
        }
    };
    float w[N];
    weights(x, w);
    SubOut r;
    if constexpr (K == K_IQ2_XXS) r = iq2_xxs_sub(x, w, tab, grid, nc);
    else if constexpr (K == K_IQ2_XS) r = iq2_16_sub<true>(x, w, tab, grid, nc);
    else if constexpr (K == K_IQ2_S) r = iq2_16_sub<false>(x, w, tab, grid, nc);
    else if constexpr (K == K_IQ3_XXS) r = iq3_sub<true>(x, w, tab, grid, nc);
    else if constexpr (K == K_IQ3_S) r = iq3_sub<false>(x, w, tab, grid, nc);
    else if constexpr (K == K_IQ1_S) r = iq1_s_sub(x, w, tab, grid, reload);
    else r = iq1_m_sub<K == K_IQ1_M1 ? 1 : 0>(x, w, tab, grid, reload);
    // super-block scale: MAX over the sub-block scales in sub-block order (empty ones count as 0)
    const float s_own = r.empty ? 0.f : r.scale;
    float max_scale = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) max_scale = tmax(max_scale, __shfl(s_own, g, G));
    const bool nz = max_scale != 0.f;   // the reference's `if (!max_scale)` exit
    constexpr float DIV = IQ1 ? 15.f : 31.f;
    constexpr int LMAX = IQ1 ? 7 : 15;
    const float d = max_scale / DIV;
    int l = 0;
    if (nz) {
        const float id = 1 / d;
        l = tmax(0, tmin(LMAX, nearest_int(0.5f * (id * s_own - 1))));
    }
    float dfinal = d;
    if constexpr (K == K_IQ1_M0 || K == K_IQ1_M1) {
        // refit of the super-scale over all 256 weights in order, empty sub-blocks included as grid
        // point 0 with signs (+, +) (ggml-quants.c:4884-4910)
        constexpr float XP0 = -1 + IQ1M_DELTA, XP1 = IQ1M_DELTA, XP2 = 1 + IQ1M_DELTA;
        constexpr float XM0 = -1 - IQ1M_DELTA, XM1 = -IQ1M_DELTA, XM2 = 1 - IQ1M_DELTA;
        float xr[N], wr[N];
        reload(xr, wr);
        float aqx[16], aq2[16];
        const int shift = r.empty ? 0 : r.shift;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const bool p = k == 0 ? shift < 2 : shift % 2 == 0;
            int q[8];
            grid_point<8>(grid, r.empty ? 0 : r.gidx[k], q);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int lv = (q[j] - 1) / 2;
                const float qq = (p ? pick3(lv, XP0, XP1, XP2) : pick3(lv, XM0, XM1, XM2)) * (float)(2 * l + 1);
                aqx[8 * k + j] = wr[8 * k + j] * qq * xr[8 * k + j];
                aq2[8 * k + j] = wr[8 * k + j] * qq * qq;
            }
        }
        float sqx = 0.f, sq2 = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (sub == g) {
#pragma unroll
                for (int i = 0; i < 16; ++i) { sqx += aqx[i]; sq2 += aq2[i]; }
            }
            sqx = __shfl(sqx, g, G);
            sq2 = __shfl(sq2, g, G);
        }
        if (sq2 > 0) dfinal = sqx / sq2;
    }
    Park pk;
    pk.scale = s_own;
    pk.l = l;
    pk.shift = r.empty ? (K == K_IQ1_S ? 1 : 0) : r.shift;
    pk.empty = r.empty ? 1 : 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) pk.gidx[k] = r.empty ? 0 : r.gidx[k];
#pragma unroll
    for (int k = 0; k < 4; ++k) pk.signs[k] = r.empty ? 0u : r.signs[k];
    if constexpr (!IQ1) __syncthreads();   // every lane's search has read its sqrt(w) column
    const int lsb2 = tid() / G, sub2 = tid() % G;
    park[lsb2][sub2] = pk;
    __syncthreads();
    if (sb0 + lsb2 < nsb && sub2 == 0) {
        TileOut o{otile + lsb2 * (C::BS / 2)};
        const Park* P = park[lsb2];
        for (int j = 0; j < C::BS; j += 2) o.put16(j, 0);
        if constexpr (K == K_IQ2_XXS) {
            // d, then per 32 weights: u32 of 4 grid indices, u32 of 4 x 7 sign bits | scale << 28
            if (nz) {
                o.put16(0, f32_to_f16(d));
                for (int ib = 0; ib < 8; ++ib) {
                    const uint32_t a = (uint32_t)P[ib].gidx[0] | ((uint32_t)P[ib].gidx[1] << 8) |
                                       ((uint32_t)P[ib].gidx[2] << 16) | ((uint32_t)P[ib].gidx[3] << 24);
                    const uint32_t b = P[ib].signs[0] | (P[ib].signs[1] << 7) | (P[ib].signs[2] << 14) |
                                       (P[ib].signs[3] << 21) | ((uint32_t)P[ib].l << 28);
                    o.put16(2 + 8 * ib, a & 0xffff); o.put16(4 + 8 * ib, a >> 16);
                    o.put16(6 + 8 * ib, b & 0xffff); o.put16(8 + 8 * ib, b >> 16);
                }
            }
        } else if constexpr (K == K_IQ2_XS) {
            // d, per 16 weights two u16 (9-bit grid index | 7 sign bits << 9), scale nibbles
            if (nz) {
                o.put16(0, f32_to_f16(d));
                for (int ib = 0; ib < 16; ++ib)
                    for (int k = 0; k < 2; ++k) o.put16(2 + 4 * ib + 2 * k, (uint32_t)P[ib].gidx[k] | (P[ib].signs[k] << 9));
                for (int ib = 0; ib < 16; ib += 4)
                    o.put2(66 + ib / 2, P[ib].l | (P[ib + 1].l << 4), P[ib + 2].l | (P[ib + 3].l << 4));
            }
        } else if constexpr (K == K_IQ2_S) {
            // d, qs[32] grid low bytes, qs[32] signs, qh[8] (2 high bits per group), scales[8]
            if (nz) o.put16(0, f32_to_f16(d * 0.9875f));
            for (int ib = 0; ib < 16; ++ib) {
                o.put2(2 + 2 * ib, P[ib].gidx[0] & 255, P[ib].gidx[1] & 255);
                o.put2(34 + 2 * ib, P[ib].signs[0], P[ib].signs[1]);
            }
            for (int q = 0; q < 8; q += 2) {
                uint32_t h[2] = {0, 0};
                for (int t = 0; t < 2; ++t)
                    for (int i8 = 4 * (q + t); i8 < 4 * (q + t) + 4; ++i8)
                        h[t] |= (uint32_t)(P[i8 / 2].gidx[i8 % 2] >> 8) << (2 * (i8 % 4));
                o.put2(66 + q, h[0], h[1]);
            }
            if (nz)
                for (int ib = 0; ib < 16; ib += 4)
                    o.put2(74 + ib / 2, P[ib].l | (P[ib + 1].l << 4), P[ib + 2].l | (P[ib + 3].l << 4));
        } else if constexpr (K == K_IQ3_XXS) {
            // d, 64 grid indices, per 32 weights u32 of 4 x 7 sign bits | scale << 28
            if (nz) {
                o.put16(0, f32_to_f16(d * 1.0125f));
                for (int ib = 0; ib < 8; ++ib)
                    for (int k = 0; k < 8; k += 2) o.put2(2 + 8 * ib + k, P[ib].gidx[k], P[ib].gidx[k + 1]);
                for (int ib = 0; ib < 8; ++ib) {
                    const uint32_t v = P[ib].signs[0] | (P[ib].signs[1] << 7) | (P[ib].signs[2] << 14) |
                                       (P[ib].signs[3] << 21) | ((uint32_t)P[ib].l << 28);
                    o.put16(66 + 4 * ib, v & 0xffff);
                    o.put16(68 + 4 * ib, v >> 16);
                }
            }
        } else if constexpr (K == K_IQ3_S) {
            // d, qs[64], qh[8], signs[32], scales[4]. The reference advances its qs and signs cursors
            // only past sub-blocks that were not empty (ggml-quants.c:4336-4339 sit after the
            // `continue` of :4237), so later sub-blocks land in the earlier free slots; qh is indexed
            // by position.
            if (nz) o.put16(0, f32_to_f16(d * 1.033f));
            int slot = 0;
            for (int ib = 0; ib < 8; ++ib) {
                if (P[ib].empty) continue;
                for (int k = 0; k < 8; k += 2) o.put2(2 + 8 * slot + k, P[ib].gidx[k] & 255, P[ib].gidx[k + 1] & 255);
                for (int k = 0; k < 4; k += 2) o.put2(74 + 4 * slot + k, P[ib].signs[k], P[ib].signs[k + 1]);
                ++slot;
            }
            for (int ib = 0; ib < 8; ib += 2) {
                uint32_t h[2] = {0, 0};
                for (int t = 0; t < 2; ++t)
                    for (int k = 0; k < 8; ++k) h[t] |= (uint32_t)(P[ib + t].gidx[k] >> 8) << k;
                o.put2(66 + ib, h[0], h[1]);
            }
            if (nz)
                for (int ib = 0; ib < 8; ib += 4)
                    o.put2(106 + ib / 2, P[ib].l | (P[ib + 1].l << 4), P[ib + 2].l | (P[ib + 3].l << 4));
        } else if constexpr (K == K_IQ1_S) {
            // d, qs[32] grid low bytes, qh[8] u16: 3 high bits per group | (scale | 8 if shift -1) << 12
            if (nz) o.put16(0, f32_to_f16(d * 1.125f));
            for (int ib = 0; ib < 8; ++ib)
                for (int k = 0; k < 4; k += 2) o.put2(2 + 4 * ib + k, P[ib].gidx[k] & 255, P[ib].gidx[k + 1] & 255);
            for (int ib = 0; ib < 8; ++ib) {
                uint32_t h = 0;
                for (int k = 0; k < 4; ++k) h |= (uint32_t)(P[ib].gidx[k] >> 8) << (3 * k);
                if (nz) h |= (uint32_t)(P[ib].l | (P[ib].shift == -1 ? 8 : 0)) << 12;
                o.put16(34 + 2 * ib, h);
            }
        } else {
            // IQ1_M: qs[32], qh[16] (3 high bits per group, sign masks), scales: 3-bit codes and the
            // f16 super-scale in the top nibbles
            for (int ib = 0; ib < 16; ++ib) o.put2(2 * ib, P[ib].gidx[0] & 255, P[ib].gidx[1] & 255);
            const uint32_t masks[4] = {0x00, 0x80, 0x08, 0x88};
            for (int ib = 0; ib < 16; ib += 2) {
                uint32_t h[2];
                for (int t = 0; t < 2; ++t)
                    h[t] = (uint32_t)((P[ib + t].gidx[0] >> 8) | ((P[ib + t].gidx[1] >> 8) << 4)) |
                           (nz ? masks[P[ib + t].shift & 3] : 0u);
                o.put2(32 + ib, h[0], h[1]);
            }
            if (nz) {
                const uint32_t s16 = f32_to_f16(dfinal * 1.1125f);
                uint32_t sc[4] = {0, 0, 0, 0};
                for (int ib = 0; ib < 16; ++ib) sc[ib / 4] |= (uint32_t)P[ib].l << (3 * (ib % 4));
                sc[0] |= (s16 & 0x000f) << 12;
                sc[1] |= (s16 & 0x00f0) << 8;
                sc[2] |= (s16 & 0x0f00) << 4;
                sc[3] |= (s16 & 0xf000);
                for (int i = 0; i < 4; ++i) o.put16(48 + 2 * i, sc[i] & 0xffff);
            }
        }
    }
    __syncthreads();
    const int nb = (int)(nsb - sb0 < SBW ? nsb - sb0 : SBW);
    store_tile(otile, dst + sb0 * C::BS, nb * C::BS, tid());
}

template <int K>
int run(const QuantArgs& a, int table) {
    IqDeviceTable tab;
    if (int e = iq_device_table(table, &tab, a.stream)) return e;
    constexpr int D = (K == K_IQ3_XXS || K == K_IQ3_S) ? 4 : 8;
    if ((int64_t)tab.size * D != Cfg<K>::GBYTES)
        return fail(SPA_ERR_ASSERT, "grid i-quant type %d: codebook of %d points does not fit the kernel", a.type, tab.size);
    if (a.n_per_row % 256) return fail(SPA_ERR_ARG, "grid i-quant type %d: n_per_row %% 256", a.type);
    const int64_t nsb = a.nrows * a.n_per_row / 256;
    if (nsb == 0) return 0;
    constexpr int SBW = WG / (256 / Cfg<K>::N);
    hipLaunchKernelGGL(k_iqgrid<K>, dim3((unsigned)((nsb + SBW - 1) / SBW)), dim3(WG), 0, a.stream, a.src, a.src_kind,
                       (uint8_t*)a.dst, nsb, a.n_per_row / 256, a.imatrix, tab);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

int launch_iqgrid(const QuantArgs& a) {
    const int t = iq_table_index(a.type);
    switch (a.type) {
        case 16: return run<K_IQ2_XXS>(a, t);
        case 17: return run<K_IQ2_XS>(a, t);
        case 22: return run<K_IQ2_S>(a, t);
        case 18: return run<K_IQ3_XXS>(a, t);
        case 21: return run<K_IQ3_S>(a, t);
        case 19: return run<K_IQ1_S>(a, t);
        case 29: return a.variant == 1 ? run<K_IQ1_M1>(a, t) : run<K_IQ1_M0>(a, t);
    }
    return fail(SPA_ERR_TYPE, "launch_iqgrid: type %d", a.type);
}

}  // namespace spa
