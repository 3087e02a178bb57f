// QR residual coder kernels for the non-grid quant types (grid types: qr_grid.hip): histogram, interleaved-segment rANS
// encode and decode, segment gather and decode lookup tables (seedpack/qr.py:674-895 semantics).
//
// Stream format (fixed by the archive): a batch of blocks is cut into segments of
// max(16, 16384/QK) blocks; each segment is one rANS stream (PB = 12, RANS_L = 2^23, byte-wise
// renormalisation) coded backwards, ending with the 4-byte state; decoding reads forward.
//
// Mapping on the MI355X:
//   * histogram: block equality and the flag symbols of all blocks first (qr_flags.h), then one
//     lane per differing block from the list, so every such block is modelled in parallel with all
//     lanes busy; counts are integer sums (order-free), aggregated across the wave before each
//     global atomic (one atomic per distinct counter per wave step);
//   * encode / decode: one lane per segment -- the coder state is inherently serial within a
//     segment; the decoder assembles each block in a per-lane LDS slot and stores it whole.
#include <stdio.h>

#include <mutex>

#include "../../include/seedpack_amd.h"
#include "launch.h"
#include "qr_flags.h"
#include "qr_model.h"

namespace spa {
namespace qr {
namespace {

// one lane per differing block of the list (slot = segment * SEG_BLOCKS + block), all lanes of the
// grid striding over it; the flag symbols were counted with the list
template <int T>
__global__ __launch_bounds__(256) void k_qr_hist(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                                 const uint8_t* __restrict__ seed, const TM* __restrict__ tm,
                                                 const SG* __restrict__ sg, const uint32_t* __restrict__ list,
                                                 const uint32_t* __restrict__ nlist, uint32_t* __restrict__ counts, int mv) {
    using Y = Ty<T>;
    constexpr int SEG = SEG_BLOCKS<T>;
    const uint32_t n = *nlist;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t slot = list[i];
        const SG g = sg[slot / SEG];
        const TM m = tm[g.t];
        const int64_t b = g.b0 + (int)(slot % SEG);
        const uint8_t* fb = F + b * Y::BS;
        const uint8_t* pb = P + b * Y::BS;
        int tv[Y::NF];
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) tv[k] = get_field<T>(fb, k);
        int any = 0;
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) {
            const int kd = fkind<T>(k);
            const int pr = fpred<T>(mv, pb, k, tv[0], Y::NF > 1 ? tv[1] : 0), dlt = tv[k] - pr;
            if (kd < 2 && (dlt < -127 || dlt > 127)) {
                hadd(counts, (uint32_t)((kd * 2 + any) * 256 + 128));
                hadd(counts, (uint32_t)(FESC_LO * 256 + (tv[k] & 255)));
                hadd(counts, (uint32_t)(FESC_HI * 256 + (tv[k] >> 8)));
            } else {
                hadd(counts, (uint32_t)((kd * 2 + any) * 256 + (dlt & 255)));
            }
            any |= dlt != 0;
        }
        const uint8_t* sbase = seed + m.seed_off;
        const int64_t gw0 = (b - m.blk0) * Y::QK;
        const int64_t col0 = m.cols > 0 ? gw0 % m.cols : 0;
        float a = 0.f, c = 0.f;
        for (int w = 0; w < Y::QK; ++w) {
            if (w % Y::SUBLEN == 0) wscale<T>(fb, w, a, c);
            float x, h;
            seed_val(m.seed_type, sbase, gw0 + w, m.cols, x, h);
            int r, sg_, ctx;
            predict<T>(a, c, pb, w, x, h, mv, pos8(col0 + w, m.cols), hboff_of(m), r, sg_, ctx);
            hadd(counts, (uint32_t)(ctx * 256 + ((sg_ * (get_code<T>(fb, w) - r)) & 255)));
        }
    }
}

// The encoder's step x -> (x / f) * 2^PB + x % f + c without a division (Giesen's rans_byte
// reciprocal form): for f >= 2 with s = ceil(log2 f), r = ceil(2^(31+s) / f) and
// q = (x * r) >> (31 + s) equal floor(x / f) for every x < 2^31 (the error term x * (r - 2^(31+s)/f)
// / 2^(31+s) stays below 2^-s <= 1/f); then x' = x + c + q * (2^PB - f). For f = 1, r = 2^32 - 1 gives
// q = x - 1 and the bias 2^PB - 1 makes up the difference. The state before a step is below
// ((RANS_L >> PB) << 8) * f <= 2^31.
__device__ __forceinline__ uint32_t enc_rcp(uint32_t f) {
    if (f < 2) return 0xffffffffu;
    const uint32_t sh = 32 - __clz(f - 1);
    return (uint32_t)(((1ull << (31 + sh)) + f - 1) / f);
}

__global__ __launch_bounds__(256) void k_qr_rcp(const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                                uint32_t* __restrict__ rcp) {
    const int tt = remap[blockIdx.x];
    if (tt >= 0) rcp[tt * 256 + threadIdx.x] = enc_rcp(freq[tt * 256 + threadIdx.x]);
}

struct Enc {
    uint32_t x;
    uint8_t* ptr;
    const int* remap;
    const uint16_t* freq;
    const uint32_t* cum;
    const uint32_t* rcp;
    __device__ __forceinline__ void put_fc(uint32_t f, uint32_t c, uint32_t r) {
        // x < 2^31 before a step and xm >= 2^19, so at most two bytes go out
        const uint32_t xm = ((RANS_L >> PB) << 8) * f;
        if (x >= xm) {
            *--ptr = (uint8_t)(x & 0xff);
            x >>= 8;
            if (x >= xm) {
                *--ptr = (uint8_t)(x & 0xff);
                x >>= 8;
            }
        }
        const uint32_t sh = f < 2 ? 0u : 31u - __clz(f - 1);
        const uint32_t q = __umulhi(x, r) >> sh;
        x = x + c + (f < 2 ? PSCALE - 1 : 0u) + q * (PSCALE - f);
    }
    __device__ __forceinline__ void put(int tab, uint32_t sym) {
        const int tt = remap[tab];
        put_fc(freq[tt * 256 + sym], cum[tt * 257 + sym], rcp[tt * 256 + sym]);
    }
};

// bytes kept free below the coder's write pointer while coding codes: the block's fields (up to three
// symbols each) and its flag, at most two bytes per symbol
template <int T> constexpr int64_t FIELD_ROOM = 6 * Ty<T>::NF + 16;
// symbols of a differing block besides its flag: its codes and up to three per field
template <int T> constexpr int MAXSYM = Ty<T>::QK + 3 * Ty<T>::NF;

// The symbols of a differing block in the encoder's order -- codes last to first, then the fields
// last to first (an escaped field as HI, LO, mark) -- handed to put(table, symbol); put returns false
// to stop (the coder's room check after each code). The flag symbol is not included.
template <int T, class Put>
__device__ __forceinline__ bool block_syms(Put&& put, const uint8_t* fb, const uint8_t* pb, const uint8_t* sbase,
                                           const TM& m, int64_t b, int mv) {
    using Y = Ty<T>;
    const int64_t gw0 = (b - m.blk0) * Y::QK;
    const int64_t col0 = m.cols > 0 ? gw0 % m.cols : 0;
    float a = 0.f, c = 0.f;
    int sub = -1;
    for (int w = Y::QK - 1; w >= 0; --w) {
        if (w / Y::SUBLEN != sub) { sub = w / Y::SUBLEN; wscale<T>(fb, w, a, c); }
        float x, h;
        seed_val(m.seed_type, sbase, gw0 + w, m.cols, x, h);
        int r, sg_, ctx;
        predict<T>(a, c, pb, w, x, h, mv, pos8(col0 + w, m.cols), hboff_of(m), r, sg_, ctx);
        if (!put(ctx, (uint32_t)((sg_ * (get_code<T>(fb, w) - r)) & 255), true)) return false;
    }
    int tv[Y::NF], dl[Y::NF], anyk[Y::NF];
#pragma unroll
    for (int k = 0; k < Y::NF; ++k) tv[k] = get_field<T>(fb, k);
    int any = 0;
#pragma unroll
    for (int k = 0; k < Y::NF; ++k) {
        dl[k] = tv[k] - fpred<T>(mv, pb, k, tv[0], Y::NF > 1 ? tv[1] : 0);
        anyk[k] = any;
        any |= dl[k] != 0;
    }
#pragma unroll
    for (int k = Y::NF - 1; k >= 0; --k) {
        const int kd = fkind<T>(k);
        if (kd < 2 && (dl[k] < -127 || dl[k] > 127)) {
            put(FESC_HI, (uint32_t)(tv[k] >> 8), false);
            put(FESC_LO, (uint32_t)(tv[k] & 255), false);
            put(kd * 2 + anyk[k], 128, false);
        } else {
            put(kd * 2 + anyk[k], (uint32_t)(dl[k] & 255), false);
        }
    }
    return true;
}

// The symbols of the listed differing blocks (the first `cap` of the list), one lane per block, all
// lanes busy: words (table << 8 | symbol) in the encoder's order and their count. The serial coder
// then only replays them (one lane per segment would otherwise model each of its blocks while the
// wave's other lanes wait).
template <int T>
__global__ __launch_bounds__(256) void k_qr_syms(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                                 const uint8_t* __restrict__ seed, const TM* __restrict__ tm,
                                                 const SG* __restrict__ sg, const uint32_t* __restrict__ list,
                                                 const uint32_t* __restrict__ nlist, uint32_t cap,
                                                 uint16_t* __restrict__ nsym, uint32_t* __restrict__ syms, int mv) {
    using Y = Ty<T>;
    constexpr int SEG = SEG_BLOCKS<T>;
    const uint32_t n = *nlist < cap ? *nlist : cap;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t slot = list[i];
        const SG g = sg[slot / SEG];
        const TM m = tm[g.t];
        const int64_t b = g.b0 + (int)(slot % SEG);
        uint32_t* out = syms + (size_t)i * MAXSYM<T>;
        int k = 0;
        block_syms<T>([&](int tab, uint32_t sym, bool) { out[k++] = ((uint32_t)tab << 8) | sym; return true; },
                      F + b * Y::BS, P + b * Y::BS, seed + m.seed_off, m, b, mv);
        nsym[i] = (uint16_t)k;
    }
}

// One lane per segment, blocks last to first. The lane's block flags come from the equality pass as a
// bit mask in LDS. Work goes in rounds: each lane codes the flags of its run of equal blocks up to its
// next differing block, then the lanes that stopped at one code its symbols together -- so the wave
// runs the symbol loop once per round rather than once per block any of its lanes differs in. Each
// lane codes its own symbols in the same order as a block-by-block walk: the stream is the same.
template <int T>
__global__ __launch_bounds__(64) void k_qr_enc(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                               const uint8_t* __restrict__ seed, const TM* __restrict__ tm,
                                               const SG* __restrict__ sg, int nseg, const int* __restrict__ remap,
                                               const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                               const uint32_t* __restrict__ rcp,
                                               uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len,
                                               const uint8_t* __restrict__ neq, const uint32_t* __restrict__ idx_of,
                                               const uint16_t* __restrict__ nsym, const uint32_t* __restrict__ syms,
                                               int mv) {
    using Y = Ty<T>;
    constexpr int NW = SEG_BLOCKS<T> / 32;
    __shared__ uint32_t nbits[64][NW + 1];
    const int lane = threadIdx.x;
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const SG g = sg[s];
    const TM m = tm[g.t];
    const int nb = g.nb < SEG_BLOCKS<T> ? g.nb : SEG_BLOCKS<T>;
    // 32 flags per word: unconditional loads (indices clamped into the segment), so each word's loads
    // are in flight together instead of one branch and one wait per flag
    for (int w = 0; w < NW; ++w) {
        uint32_t v = 0;
        if (32 * w < nb) {
            uint8_t f[32];
#pragma unroll
            for (int j = 0; j < 32; ++j) f[j] = neq[g.b0 + min(32 * w + j, nb - 1)];
#pragma unroll
            for (int j = 0; j < 32; ++j) v |= (uint32_t)(f[j] != 0 && 32 * w + j < nb) << j;
        }
        nbits[lane][w] = v;
    }
    // the last differing block at or below i (-1 if none), from the flag words
    auto differing_at_or_below = [&](int i) {
        while (i >= 0) {
            const uint32_t w = nbits[lane][i >> 5] & (0xffffffffu >> (31 - (i & 31)));
            if (w) return (i & ~31) + 31 - (int)__clz(w);
            i = (i & ~31) - 1;
        }
        return -1;
    };
    const uint8_t* sbase = seed + m.seed_off;
    uint8_t* const base = out + (uint64_t)s * cap;
    uint8_t* const end = base + cap;
    Enc e{RANS_L, end, remap, freq, cum, rcp};
    FlagTab ft;
    ft.load(remap, freq, cum);
    ft.load_rcp(remap, rcp);
    auto put = [&](int tab, uint32_t sym, bool code) {
        e.put(tab, sym);
        return !(code && e.ptr - base < FIELD_ROOM<T>);
    };
    // an equal block's flag is coded in the context of its predecessor (block i - 1 equal: 1,
    // differing: 0; block 0: 1). A run of equal blocks i .. j + 1 above the differing block j thus
    // codes i - j - 1 flags in context 1 and then one in context 0 (context 1 when the run reaches
    // block 0): the run is found from the flag words and coded in one register loop
    const uint32_t fA = ft.freq_of(1, 1), cA = ft.cum_of(1, 1), rA = ft.rcp_of(1, 1);
    const uint32_t fB = ft.freq_of(0, 1), cB = ft.cum_of(0, 1), rB = ft.rcp_of(0, 1);
    int i = nb - 1;                              // block g.b0 + i
    for (;;) {
        const int j = differing_at_or_below(i);
        const int n = i - j;                     // equal blocks in the run (two bytes at most each)
        if (e.ptr - base < 8 + 2 * (int64_t)n) { out_len[s] = 0xffffffffu; return; }
        for (int k = j >= 0 ? n - 1 : n; k > 0; --k) e.put_fc(fA, cA, rA);
        if (j >= 0 && n > 0) e.put_fc(fB, cB, rB);
        i = j;
        const bool pend = i >= 0;
        if (__ballot(pend) == 0) break;
        if (!pend) continue;
        const int64_t b = g.b0 + i;
        const uint32_t k = idx_of[b];
        if (k != 0xffffffffu) {
            // the block's symbols from the parallel pass: the codes (checked for room) first. Eight
            // symbols' table entries are fetched together ahead of their coding steps, so the coder's
            // chain waits on memory once per eight symbols
            const uint32_t* q = syms + (size_t)k * MAXSYM<T>;
            const int n = nsym[k];
            for (int j0 = 0; j0 < n; j0 += 8) {
                uint32_t fq[8], cq[8], rq[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    fq[t] = 1u;
                    cq[t] = 0u;
                    rq[t] = 0xffffffffu;
                    if (j0 + t < n) {
                        const uint32_t wd = q[j0 + t];
                        const int tt = remap[wd >> 8];
                        fq[t] = freq[tt * 256 + (wd & 255u)];
                        cq[t] = cum[tt * 257 + (wd & 255u)];
                        rq[t] = rcp[tt * 256 + (wd & 255u)];
                    }
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (j0 + t >= n) break;
                    e.put_fc(fq[t], cq[t], rq[t]);
                    if (j0 + t < Y::QK && e.ptr - base < FIELD_ROOM<T>) { out_len[s] = 0xffffffffu; return; }
                }
            }
        } else if (!block_syms<T>(put, F + b * Y::BS, P + b * Y::BS, sbase, m, b, mv)) {
            out_len[s] = 0xffffffffu;
            return;
        }
        const int prev = i > 0 ? (((nbits[lane][(i - 1) >> 5] >> ((i - 1) & 31)) & 1u) ? 0 : 1) : 1;
        e.put_fc(ft.freq_of(prev, 0), ft.cum_of(prev, 0), ft.rcp_of(prev, 0));
        --i;
    }
    for (int j = 0; j < 4; ++j) { *--e.ptr = (uint8_t)(e.x & 0xff); e.x >>= 8; }
    out_len[s] = (uint32_t)(end - e.ptr);
}

struct Dec {
    uint32_t x;
    ByteQ bq;
    const int* remap;
    const uint16_t* freq;
    const uint32_t* cum;
    const uint32_t* lut;
    __device__ __forceinline__ int get(int tab) { return get_tt(remap[tab]); }
    __device__ __forceinline__ int get_tt(int tt) {
        // one load per symbol: its LUT32 entry holds the symbol, freq - 1 and slot - cum
        const uint32_t slot = x & (PSCALE - 1);
        const uint32_t e = lut[(size_t)tt * PSCALE + slot];
        const int v = (int)(e & 255u);
        x = (((e >> 8) & (PSCALE - 1)) + 1) * (x >> PB) + (e >> 20);
        // a valid stream needs at most two bytes here (x >= 2^11 before them); the cap ends the
        // loop on a damaged stream instead of spinning on zero bytes
#pragma unroll
        for (int i = 0; i < 4 && x < RANS_L; ++i) x = (x << 8) | bq.next();
        return v;
    }
};

constexpr int DEC_WG = 64;

// One lane per segment; the flags are decoded from the register flag table. Work goes in rounds, as in
// the encoder:
// each lane decodes flags up to its next differing block, then the lanes that stopped at one decode
// and model it together, so one lane's differing block does not hold the other 63.
template <int T>
__global__ __launch_bounds__(DEC_WG) void k_qr_dec(const uint8_t* __restrict__ in, uint64_t in_bytes,
                                                   const uint64_t* __restrict__ in_off,
                                                   const uint8_t* __restrict__ P, const uint8_t* __restrict__ seed,
                                                   const TM* __restrict__ tm, const SG* __restrict__ sg, int nseg,
                                                   const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                                   const uint32_t* __restrict__ cum, const uint32_t* __restrict__ lut,
                                                   uint8_t* __restrict__ F, int mv) {
    using Y = Ty<T>;
    constexpr int BSP = (Y::BS + 3) & ~3;
    __shared__ __align__(4) uint8_t blk[DEC_WG * BSP];
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    FlagTab ft;
    ft.load(remap, freq, cum);
    uint8_t* fb = blk + threadIdx.x * BSP;
    const SG g = sg[s];
    const TM m = tm[g.t];
    const uint8_t* sbase = seed + m.seed_off;
    const uint8_t* const in_end = in + in_bytes;
    Dec d{0, {}, remap, freq, cum, lut};
    d.bq.start(in + (in_off[s] < in_bytes ? in_off[s] : in_bytes), in_end);
    for (int i = 0; i < 4; ++i) d.x = (d.x << 8) | d.bq.next();
    int prev = 1;
    int64_t b = g.b0;
    const int64_t bend = g.b0 + g.nb;
    for (;;) {
        bool pend = false;
        for (; b < bend; ++b) {
            prev = ft.get(d.x, d.bq, prev);
            if (!prev) { pend = true; break; }     // F holds P's bytes for the equal blocks (qr_prefill)
        }
        if (__ballot(pend) == 0) break;
        if (!pend) continue;
        const uint8_t* pb = P + b * Y::BS;
        uint8_t* dst = F + b * Y::BS;
        for (int i = 0; i < Y::BS; ++i) fb[i] = 0;
        int vals[Y::NF];
        int any = 0;
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) {
            const int kd = fkind<T>(k);
            const int pr = fpred<T>(mv, pb, k, k > 0 ? vals[0] : 0, k > 1 ? vals[Y::NF > 1 ? 1 : 0] : 0);
            const int sym = d.get(kd * 2 + any);
            int t;
            if (kd < 2 && sym == 128) {
                const int lo = d.get(FESC_LO), hi = d.get(FESC_HI);
                t = lo | (hi << 8);
            } else {
                t = pr + s8((uint32_t)sym);
                if (kd < 2) t &= 0xffff;
                else if (T == 14) t = s8((uint32_t)t);
            }
            vals[k] = t;
            any |= t != pr;
        }
        set_fields<T>(fb, vals);
        const int64_t gw0 = (b - m.blk0) * Y::QK;
        const int64_t col0 = m.cols > 0 ? gw0 % m.cols : 0;
        // the codes' contexts depend on the decoded fields, the seed and P only: eight weights' contexts
        // and table numbers are made ahead of their decoding steps, so the chain waits on the seed and
        // the remap table once per eight weights
        static_assert(Y::SUBLEN % 8 == 0, "weight groups of eight within a sub-block");
        float a = 0.f, c = 0.f;
        for (int w0 = 0; w0 < Y::QK; w0 += 8) {
            if (w0 % Y::SUBLEN == 0) wscale<T>(fb, w0, a, c);
            int r8[8], sg8[8], tt8[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                float x, h;
                seed_val(m.seed_type, sbase, gw0 + w0 + t, m.cols, x, h);
                int ctx;
                predict<T>(a, c, pb, w0 + t, x, h, mv, pos8(col0 + w0 + t, m.cols), hboff_of(m), r8[t], sg8[t], ctx);
                tt8[t] = remap[ctx];
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int v = d.get_tt(tt8[t]);
                int q = r8[t] + sg8[t] * s8((uint32_t)v);
                if (T == 8) q = s8((uint32_t)q);
                put_code<T>(fb, w0 + t, q);
            }
        }
        for (int i = 0; i < Y::BS; ++i) dst[i] = fb[i];
        ++b;
        prev = 0;
    }
}

__global__ __launch_bounds__(256) void k_qr_gather(const uint8_t* __restrict__ src, uint64_t cap, const uint32_t* __restrict__ len,
                                                   const uint64_t* __restrict__ off, int nseg, uint8_t* __restrict__ dst) {
    const int s = blockIdx.x;
    if (s >= nseg) return;
    const uint8_t* a = src + (uint64_t)(s + 1) * cap - len[s];
    uint8_t* d = dst + off[s];
    for (uint32_t i = threadIdx.x; i < len[s]; i += blockDim.x) d[i] = a[i];
}

// LUT32 entries, slot by slot: the symbol s whose range [cum[s], cum[s + 1]) holds the slot (the last
// s with cum[s] <= slot), its frequency - 1 (bits 8-19) and slot - cum[s] (bits 20-31); a table not
// summing to 2^12 gives entries that keep a damaged stream's decoding in bounds
__global__ __launch_bounds__(256) void k_build_lut32(const uint32_t* __restrict__ cum, int ntab, uint32_t* __restrict__ lut) {
    __shared__ uint32_t cs[257];
    const int tb = blockIdx.x;
    if (tb >= ntab) return;
    for (int k = threadIdx.x; k < 257; k += blockDim.x) cs[k] = cum[tb * 257 + k];
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < PSCALE; i += blockDim.x) {
        int lo = 0, hi = 256;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (cs[mid] <= i) lo = mid;
            else hi = mid;
        }
        const uint32_t f = cs[lo + 1] > cs[lo] ? cs[lo + 1] - cs[lo] : 1u;
        lut[(size_t)tb * PSCALE + i] = (uint32_t)lo | (((f - 1) & (PSCALE - 1)) << 8) | (((i - cs[lo]) & (PSCALE - 1)) << 20);
    }
}

__global__ __launch_bounds__(256) void k_build_lut(const uint32_t* __restrict__ cum, int ntab, uint8_t* __restrict__ lut) {
    const int tb = blockIdx.x;
    if (tb >= ntab) return;
    for (int sym = threadIdx.x; sym < 256; sym += blockDim.x)
        for (uint32_t i = cum[tb * 257 + sym]; i < cum[tb * 257 + sym + 1]; ++i) lut[(size_t)tb * PSCALE + i] = (uint8_t)sym;
}

template <template <int> class K, class... A>
int dispatch(int T, A&&... args) {
    switch (T) {
        case 2: return K<2>::run(args...);
        case 3: return K<3>::run(args...);
        case 6: return K<6>::run(args...);
        case 7: return K<7>::run(args...);
        case 8: return K<8>::run(args...);
        case 10: return K<10>::run(args...);
        case 11: return K<11>::run(args...);
        case 12: return K<12>::run(args...);
        case 13: return K<13>::run(args...);
        case 14: return K<14>::run(args...);
        case 20: return K<20>::run(args...);
        case 23: return K<23>::run(args...);
        case 42: return K<42>::run(args...);
    }
    return fail(SPA_ERR_TYPE, "QR: type %d is not a non-grid QR type", T);
}

template <int T> struct Hist {
    static int run(const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg,
                   uint32_t* counts, int mv, void* work, hipStream_t st) {
        const int64_t n = (int64_t)nseg * SEG_BLOCKS<T>;
        const QrWork w = qr_work(work, n, MAXSYM<T>);
        if (int e = qr_flags(F, P, sg, nseg, SEG_BLOCKS<T>, Ty<T>::BS, w, counts, false, st)) return e;
        // the differing blocks are a small share of the batch in practice: at most 2048 workgroups
        // stride over the list
        const int64_t wgs = (n + 255) / 256 < 2048 ? (n + 255) / 256 : 2048;
        hipLaunchKernelGGL(k_qr_hist<T>, dim3((unsigned)wgs), dim3(256), 0, st, (const uint8_t*)F, (const uint8_t*)P,
                           (const uint8_t*)seed, (const TM*)tm, (const SG*)sg, (const uint32_t*)w.list,
                           (const uint32_t*)w.nlist, counts, mv);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct Encode {
    static int run(const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, const int* remap,
                   const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap, uint32_t* out_len, int mv, void* work,
                   hipStream_t st) {
        const int64_t n = (int64_t)nseg * SEG_BLOCKS<T>;
        const QrWork w = qr_work(work, n, MAXSYM<T>);
        if (int e = qr_flags(F, P, sg, nseg, SEG_BLOCKS<T>, Ty<T>::BS, w, nullptr, true, st)) return e;
        const int64_t wgs = ((int64_t)w.cap + 255) / 256 < 2048 ? ((int64_t)w.cap + 255) / 256 : 2048;
        hipLaunchKernelGGL(k_qr_syms<T>, dim3((unsigned)wgs), dim3(256), 0, st, (const uint8_t*)F, (const uint8_t*)P,
                           (const uint8_t*)seed, (const TM*)tm, (const SG*)sg, (const uint32_t*)w.list,
                           (const uint32_t*)w.nlist, w.cap, w.nsym, w.syms, mv);
        hipLaunchKernelGGL(k_qr_rcp, dim3(NTAB2), dim3(256), 0, st, remap, freq, w.rcp);
        hipLaunchKernelGGL(k_qr_enc<T>, dim3((unsigned)((nseg + 63) / 64)), dim3(64), 0, st, (const uint8_t*)F,
                           (const uint8_t*)P, (const uint8_t*)seed, (const TM*)tm, (const SG*)sg, nseg, remap, freq, cum,
                           (const uint32_t*)w.rcp, (uint8_t*)out, cap, out_len, (const uint8_t*)w.neq, (const uint32_t*)w.idx_of,
                           (const uint16_t*)w.nsym, (const uint32_t*)w.syms, mv);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct Decode {
    static int run(const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* P, const void* seed, const void* tm, const void* sg,
                   int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum, const uint32_t* lut, void* F, int mv,
                   hipStream_t st) {
        if (int e = qr_prefill(F, P, sg, nseg, Ty<T>::BS, st)) return e;
        hipLaunchKernelGGL(k_qr_dec<T>, dim3((unsigned)((nseg + DEC_WG - 1) / DEC_WG)), dim3(DEC_WG), 0, st,
                           (const uint8_t*)in, in_bytes, in_off, (const uint8_t*)P, (const uint8_t*)seed, (const TM*)tm,
                           (const SG*)sg, nseg, remap, freq, cum, lut, (uint8_t*)F, mv);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};

template <int T> struct MaxSym {
    static int run() { return MAXSYM<T>; }
};

bool grid_type(int T) { return T == 16 || T == 17 || T == 18 || T == 19 || T == 21 || T == 22 || T == 29; }

// ---- per-weight side kernels of the seed-less and sibling coders (qr.py:811-878)

// the interval of original values that rounds to each weight's code (one infinite side at the end of
// the code range; both for a zero scale)
template <int T>
__global__ __launch_bounds__(256) void k_intervals(const uint8_t* __restrict__ F, int64_t nw, float* __restrict__ lo,
                                                   float* __restrict__ hi) {
    using Y = Ty<T>;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nw) return;
    const uint8_t* b = F + (i / Y::QK) * Y::BS;
    const int w = (int)(i % Y::QK), q = get_code<T>(b, w);
    float a, c;
    wscale<T>(b, w, a, c);
    float l, h;
    if constexpr (NONLIN<T>) {
        l = q > 0 ? a * (0.5f * (KV[q - 1] + KV[q])) : -INFINITY;
        h = q < 15 ? a * (0.5f * (KV[q] + KV[q + 1])) : INFINITY;
        if (a < 0.f) { const float t = l; l = q < 15 ? h : -INFINITY; h = q > 0 ? t : INFINITY; }
        if (a == 0.f) { l = -INFINITY; h = INFINITY; }
    } else {
        const float v = a * (float)q + c, e = fabsf(a) * 0.5f;
        l = v - e;
        h = v + e;
        const bool lowend = q == Y::QMIN, highend = q == Y::QMAX;
        if (a > 0.f) { if (lowend) l = -INFINITY; if (highend) h = INFINITY; }
        else if (a < 0.f) { if (highend) l = -INFINITY; if (lowend) h = INFINITY; }
        else { l = -INFINITY; h = INFINITY; }
    }
    lo[i] = l;
    hi[i] = h;
}

// 1 where a weight's code and its sub-block's integer scale (and min) equal the other block's
template <int T>
__global__ __launch_bounds__(256) void k_weq(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P, int64_t nw,
                                             uint8_t* __restrict__ out) {
    using Y = Ty<T>;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nw) return;
    const uint8_t* f = F + (i / Y::QK) * Y::BS;
    const uint8_t* p = P + (i / Y::QK) * Y::BS;
    const int w = (int)(i % Y::QK);
    bool eq = get_code<T>(f, w) == get_code<T>(p, w);
    const int sub = w / Y::SUBLEN;
    if constexpr (T == 10) eq = eq && f[sub] == p[sub];
    if constexpr (T == 11) eq = eq && q3k_scale(f + 96, sub) == q3k_scale(p + 96, sub);
    if constexpr (T == 12 || T == 13) {
        int s1, m1, s2, m2;
        k4_scale_min(sub, f + 4, s1, m1);
        k4_scale_min(sub, p + 4, s2, m2);
        eq = eq && s1 == s2 && m1 == m2;
    }
    if constexpr (T == 14) eq = eq && f[192 + sub] == p[192 + sub];
    if constexpr (T == 23) eq = eq && get_field<T>(f, 1 + sub) == get_field<T>(p, 1 + sub);
    out[i] = (uint8_t)eq;
}

template <int T>
__global__ __launch_bounds__(256) void k_block_fields(const uint8_t* __restrict__ F, int64_t nblk, int* __restrict__ out) {
    using Y = Ty<T>;
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
#pragma unroll
    for (int k = 0; k < Y::NF; ++k) out[b * Y::NF + k] = get_field<T>(F + b * Y::BS, k);
}

// blocks with the given field values and zero codes
template <int T>
__global__ __launch_bounds__(256) void k_blocks_from_fields(const int* __restrict__ v, int n, uint8_t* __restrict__ out) {
    using Y = Ty<T>;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= n) return;
    uint8_t o[Y::BS];
#pragma unroll
    for (int i = 0; i < Y::BS; ++i) o[i] = 0;
    int f[Y::NF];
#pragma unroll
    for (int j = 0; j < Y::NF; ++j) f[j] = v[(int64_t)k * Y::NF + j];
    set_fields<T>(o, f);
#pragma unroll
    for (int i = 0; i < Y::BS; ++i) out[(int64_t)k * Y::BS + i] = o[i];
}

unsigned wgs_for(int64_t n) { return (unsigned)((n + 255) / 256); }

// every QR type, grid types included
template <template <int> class K, class... A>
int dispatch_any(int T, A&&... args) {
    switch (T) {
        case 16: return K<16>::run(args...);
        case 17: return K<17>::run(args...);
        case 18: return K<18>::run(args...);
        case 19: return K<19>::run(args...);
        case 21: return K<21>::run(args...);
        case 22: return K<22>::run(args...);
        case 29: return K<29>::run(args...);
    }
    return dispatch<K>(T, args...);
}

template <int T> struct Intervals {
    static int run(const void* F, int64_t nw, float* lo, float* hi, hipStream_t st) {
        hipLaunchKernelGGL(k_intervals<T>, dim3(wgs_for(nw)), dim3(256), 0, st, (const uint8_t*)F, nw, lo, hi);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct Weq {
    static int run(const void* F, const void* P, int64_t nw, uint8_t* out, hipStream_t st) {
        hipLaunchKernelGGL(k_weq<T>, dim3(wgs_for(nw)), dim3(256), 0, st, (const uint8_t*)F, (const uint8_t*)P, nw, out);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct Fields {
    static int run(const void* F, int64_t nblk, int* out, hipStream_t st) {
        hipLaunchKernelGGL(k_block_fields<T>, dim3(wgs_for(nblk)), dim3(256), 0, st, (const uint8_t*)F, nblk, out);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct FromFields {
    static int run(const int* v, int n, void* out, hipStream_t st) {
        hipLaunchKernelGGL(k_blocks_from_fields<T>, dim3(wgs_for(n)), dim3(256), 0, st, v, n, (uint8_t*)out);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};

int check_common(int T, int nseg, int mv, const void* gk) {
    if (nseg < 0) return fail(SPA_ERR_ARG, "QR: negative segment count");
    if (mv != 1 && mv != 2) return fail(SPA_ERR_ARG, "QR: unknown model %d", mv);
    if (grid_type(T) && !gk) return fail(SPA_ERR_ARG, "QR: grid type %d needs its grid keys", T);
    return 0;
}

}  // namespace

// grid types (qr_grid.hip)
int grid_hist(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, uint32_t* counts,
              const uint16_t* gk, const float* imx, int mv, void* work, hipStream_t st);
int grid_encode(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, const int* remap,
                const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap, uint32_t* out_len, const uint16_t* gk,
                const float* imx, int mv, void* work, hipStream_t st);
int grid_decode(int T, const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* P, const void* seed, const void* tm, const void* sg,
                int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum, const uint32_t* lut, void* F,
                const uint16_t* gk, const float* imx, int mv, hipStream_t st);
int grid_half_steps(int T, const void* F, int64_t nw, float* h, hipStream_t st);

}  // namespace qr
}  // namespace spa

using namespace spa::qr;

// Workspace of spa_qr_encode_noalloc: one copy per device, held until the process ends. Host code
// never uses this name as an address: each device's copy is reached through the pointer
// hipGetSymbolAddress returns on that device (scratch_on_device).
#define SPA_QR_NOALLOC_SCRATCH (64u << 20)
static __device__ __align__(256) uint8_t scratch[SPA_QR_NOALLOC_SCRATCH];

namespace {
constexpr int kMaxDev = 16;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDev];
hipEvent_t g_scratch_done[kMaxDev];   // recorded after the last kernels that used the device's scratch

// the current device's copy of `scratch` and its event (set up once per device, with that device
// current: the symbol's address and one event; nothing is allocated on the device). Called with
// g_scratch_mu held.
int scratch_on_device(int* dev_out, void** out) {
    int dev = 0;
    SPA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDev) return spa::fail(SPA_ERR_ARG, "QR: device %d out of range", dev);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return spa::fail(SPA_ERR_HIP, "QR: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        SPA_HIP_TRY(hipEventCreateWithFlags(&g_scratch_done[dev], hipEventDisableTiming));   // (a wait on it before
        g_scratch_ptr[dev] = p;                                                               // its first record is a no-op)
    }
    *dev_out = dev;
    *out = g_scratch_ptr[dev];
    return 0;
}
}  // namespace

extern "C" {

int spa_qr_grid_h(int T, const void* F, int64_t nw, float* h, void* stream) {
    if (nw < 0) return spa::fail(SPA_ERR_ARG, "spa_qr_grid_h: negative count");
    if (!nw) return 0;
    if (!F || !h) return spa::fail(SPA_ERR_ARG, "spa_qr_grid_h: null pointer");
    return grid_half_steps(T, F, nw, h, (hipStream_t)stream);
}

int spa_qr_intervals(int T, const void* F, int64_t nw, float* lo, float* hi, void* stream) {
    if (nw < 0) return spa::fail(SPA_ERR_ARG, "spa_qr_intervals: negative count");
    if (!nw) return 0;
    if (!F || !lo || !hi) return spa::fail(SPA_ERR_ARG, "spa_qr_intervals: null pointer");
    return dispatch<Intervals>(T, F, nw, lo, hi, (hipStream_t)stream);
}

int spa_qr_weight_equal(int T, const void* F, const void* P, int64_t nw, uint8_t* out, void* stream) {
    if (nw < 0) return spa::fail(SPA_ERR_ARG, "spa_qr_weight_equal: negative count");
    if (!nw) return 0;
    if (!F || !P || !out) return spa::fail(SPA_ERR_ARG, "spa_qr_weight_equal: null pointer");
    return dispatch<Weq>(T, F, P, nw, out, (hipStream_t)stream);
}

int spa_qr_block_fields(int T, const void* F, int64_t nblk, int* out, void* stream) {
    if (nblk < 0) return spa::fail(SPA_ERR_ARG, "spa_qr_block_fields: negative count");
    if (!nblk) return 0;
    if (!F || !out) return spa::fail(SPA_ERR_ARG, "spa_qr_block_fields: null pointer");
    return dispatch_any<Fields>(T, F, nblk, out, (hipStream_t)stream);
}

int spa_qr_blocks_from_fields(int T, const int* v, int n, void* out, void* stream) {
    if (n < 0) return spa::fail(SPA_ERR_ARG, "spa_qr_blocks_from_fields: negative count");
    if (!n) return 0;
    if (!v || !out) return spa::fail(SPA_ERR_ARG, "spa_qr_blocks_from_fields: null pointer");
    return dispatch_any<FromFields>(T, v, n, out, (hipStream_t)stream);
}

int spa_qr_nfields(int T) {
    switch (T) {
        case 2: case 6: case 8: case 20: case 42: return 1;
        case 3: case 7: return 2;
        case 10: return 34;
        case 11: case 14: case 17: case 22: case 29: return 17;
        case 12: case 13: return 18;
        case 23: case 16: case 18: case 19: case 21: return 9;
    }
    return 0;
}

int spa_qr_seg_blocks(int T) {
    switch (T) {
        case 2: case 3: case 6: case 7: case 8: case 20: return 512;
        case 42: return 256;
        case 10: case 11: case 12: case 13: case 14: case 23: case 16: case 17: case 18: case 19: case 21: case 22: case 29:
            return 64;
    }
    return 0;
}

size_t spa_qr_work_bytes(int T, int nseg) {
    const int seg = spa_qr_seg_blocks(T);
    if (!seg || nseg < 0) return 0;
    return qr_work_bytes((int64_t)nseg * seg, grid_type(T) ? 0 : dispatch<MaxSym>(T));
}

int spa_qr_hist(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg,
                uint32_t* counts, const uint16_t* gk, const float* imx, int mv, void* work, void* stream) {
    if (int e = check_common(T, nseg, mv, gk)) return e;
    if (nseg == 0) return 0;
    if (!work) return spa::fail(SPA_ERR_ARG, "QR: no workspace (spa_qr_work_bytes)");
    if (grid_type(T)) return grid_hist(T, F, P, seed, tm, sg, nseg, counts, gk, imx, mv, work, (hipStream_t)stream);
    return dispatch<Hist>(T, F, P, seed, tm, sg, nseg, counts, mv, work, (hipStream_t)stream);
}

int spa_qr_encode(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg,
                  const int* remap, const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap, uint32_t* out_len,
                  const uint16_t* gk, const float* imx, int mv, void* work, void* stream) {
    if (int e = check_common(T, nseg, mv, gk)) return e;
    if (cap < 1024) return spa::fail(SPA_ERR_ARG, "QR: segment capacity %llu too small", (unsigned long long)cap);
    if (nseg == 0) return 0;
    if (!work) return spa::fail(SPA_ERR_ARG, "QR: no workspace (spa_qr_work_bytes)");
    if (grid_type(T))
        return grid_encode(T, F, P, seed, tm, sg, nseg, remap, freq, cum, out, cap, out_len, gk, imx, mv, work,
                           (hipStream_t)stream);
    return dispatch<Encode>(T, F, P, seed, tm, sg, nseg, remap, freq, cum, out, cap, out_len, mv, work, (hipStream_t)stream);
}

int spa_qr_decode(int T, const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* P, const void* seed,
                  const void* tm, const void* sg, int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum,
                  const uint32_t* lut, void* F, const uint16_t* gk, const float* imx, int mv, void* stream) {
    if (int e = check_common(T, nseg, mv, gk)) return e;
    if (nseg == 0) return 0;
    if (grid_type(T))
        return grid_decode(T, in, in_bytes, in_off, P, seed, tm, sg, nseg, remap, freq, cum, lut, F, gk, imx, mv,
                           (hipStream_t)stream);
    return dispatch<Decode>(T, in, in_bytes, in_off, P, seed, tm, sg, nseg, remap, freq, cum, lut, F, mv, (hipStream_t)stream);
}

int spa_qr_gather(const void* src, uint64_t cap, const uint32_t* len, const uint64_t* off, int nseg, void* dst, void* stream) {
    if (nseg <= 0) return 0;
    hipLaunchKernelGGL(k_qr_gather, dim3((unsigned)nseg), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)src, cap, len,
                       off, nseg, (uint8_t*)dst);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

int spa_rans_build_lut32(const uint32_t* cum, int ntab, uint32_t* lut, void* stream) {
    if (ntab <= 0) return 0;
    hipLaunchKernelGGL(k_build_lut32, dim3((unsigned)ntab), dim3(256), 0, (hipStream_t)stream, cum, ntab, lut);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

int spa_rans_build_lut(const uint32_t* cum, int ntab, uint8_t* lut, void* stream) {
    if (ntab <= 0) return 0;
    hipLaunchKernelGGL(k_build_lut, dim3((unsigned)ntab), dim3(256), 0, (hipStream_t)stream, cum, ntab, lut);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

int spa_qr_encode_noalloc(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg,
                          const int* remap, const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap,
                          uint32_t* out_len, const uint16_t* gk, const float* imx, int mv, void* stream) {
    if (!spa_qr_seg_blocks(T)) return spa::fail(SPA_ERR_TYPE, "QR: type %d is not a QR type", T);
    if (int e = check_common(T, nseg, mv, gk)) return e;
    if (cap < 1024) return spa::fail(SPA_ERR_ARG, "QR: segment capacity %llu too small", (unsigned long long)cap);
    const size_t need = spa_qr_work_bytes(T, nseg);
    if (need > SPA_QR_NOALLOC_SCRATCH)
        return spa::fail(SPA_ERR_ARG, "spa_qr_encode_noalloc: %d segments of type %d need %zu bytes of workspace, "
                         "more than the %u of its static scratch (split the batch or use spa_qr_encode)",
                         nseg, T, need, SPA_QR_NOALLOC_SCRATCH);
    if (nseg == 0) return 0;
    // the calls on one device take the scratch in turn: each call's stream waits for the event the
    // previous call recorded after its kernels, and records it again after its own (under a graph
    // capture the graph's own order is the caller's, and neither is added to it)
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    void* work = nullptr;
    int dev = 0;
    if (int e = scratch_on_device(&dev, &work)) return e;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SPA_HIP_TRY(hipStreamIsCapturing((hipStream_t)stream, &cs));
    const bool order = cs == hipStreamCaptureStatusNone;
    if (order) SPA_HIP_TRY(hipStreamWaitEvent((hipStream_t)stream, g_scratch_done[dev], 0));
    const int rc = grid_type(T) ? grid_encode(T, F, P, seed, tm, sg, nseg, remap, freq, cum, out, cap, out_len, gk, imx, mv,
                                              work, (hipStream_t)stream)
                                : dispatch<Encode>(T, F, P, seed, tm, sg, nseg, remap, freq, cum, out, cap, out_len, mv, work,
                                                   (hipStream_t)stream);
    if (order) SPA_HIP_TRY(hipEventRecord(g_scratch_done[dev], (hipStream_t)stream));
    return rc;
}

size_t spa_qr_noalloc_scratch_bytes(void) { return SPA_QR_NOALLOC_SCRATCH; }

}  // extern "C"
