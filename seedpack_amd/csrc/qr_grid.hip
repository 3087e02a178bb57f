// QR residual coder for the grid i-quant types (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M):
// histogram, encode and decode with the grid model of seedpack/qr.py:385-637.
//
// Model. After the block flag and the scale fields (as for the other types), a grid block is coded
// in units of 8 weights. Per unit: the targets u = |x| / s (IQ1: x / s) from the seed and the file's
// own scale, weights sqrt(sigma2 + x^2) (times the imatrix); per lattice group of the unit the rank
// of the file's grid point among all grid points in (weighted distance, index) order, with a context
// from the gap between the two nearest distances (rank >= 16 escapes to the index's two bytes);
// then each sign against the seed's sign (context: level 0 or not, |u|); IQ1_M adds its shift bit.
//
// Mapping on the MI355X: one wavefront per rANS segment (encode, decode) or per differing block
// (histogram; the flag symbols of all blocks and the list of differing ones come from qr_flags.h).
// Every lane runs the same symbol sequence with the same coder state -- the coder is serial by
// nature -- while the lattice scan, the only heavy part (256 to 2048 points per group), is split
// over the 64 lanes: lane l owns points l, l+64, ...; their keys stay in registers for the whole
// launch. Ranks are wave sums of integer counts; the nearest distances and the decoder's ordered
// candidates are wave reductions under the exact (distance, index) order, so the result equals the
// reference's sequential scan bit for bit. Lane 0 alone writes stream bytes and counters; the
// decoder assembles each block in LDS, every lane applying the same writes. Workgroups are one
// wavefront, so a workgroup barrier orders the pair table's writes and reads within the wave.
#include "../../include/seedpack_amd.h"
#include "launch.h"
#include "qr_flags.h"
#include "qr_model.h"

namespace spa {
namespace qr {
namespace {

constexpr int GRID_RANK = NSB_MAX, GRID_SIGN = NSB_MAX + 8, GRID_SHIFT = NSB_MAX + 24;   // model 1
constexpr int GRANK2 = NTAB + 128, GSIGN2 = NTAB + 144;                                  // model 2: by position
constexpr int TOPK = 16;
constexpr float INF = __builtin_huge_valf();
// x / literal in the reference's QR kernels is x * RN(1 / literal) (ptxas; its --cpu build does the same)
constexpr float R_IQ2S = 1.0f / 0.9875f, R_IQ3S = 1.0f / 1.033f, R_IQ1S = 1.0f / 1.125f, R_IQ1M = 1.0f / 1.1125f;

template <int T> struct G {
    static constexpr int N = (T == 18 || T == 21) ? 4 : 8;          // weights per lattice group
    static constexpr int NG = 8 / N;                                  // groups per unit of 8
    static constexpr bool SGN = !(T == 19 || T == 29);                // lattice of |x| plus signs
    static constexpr bool PAR = T == 16 || T == 17 || T == 18;        // 7 stored signs + even parity
    static constexpr int GS = (T == 16 || T == 18) ? 256 : (T == 17 || T == 21) ? 512 : T == 22 ? 1024 : 2048;
    static constexpr int B = N == 8 ? 2 : 3, L = 1 << B;              // bits per level in a key
    static constexpr int PER = GS / 64;                               // grid points per lane
};

__device__ __forceinline__ uint32_t rd32(const uint8_t* b) { return rd16(b) | (rd16(b + 2) << 16); }

// ---- grid indices, signs and IQ1_M shift bits inside a block (qr.py:396-446)
template <int T>
__device__ __forceinline__ int get_gidx(const uint8_t* b, int g) {
    if constexpr (T == 16) return b[2 + 8 * (g >> 2) + (g & 3)];
    if constexpr (T == 17) return (int)(rd16(b + 2 + 2 * g) & 511);
    if constexpr (T == 22) return b[2 + g] | ((b[66 + (g >> 2)] << (8 - 2 * (g & 3))) & 0x300);
    if constexpr (T == 18) return b[2 + g];
    if constexpr (T == 21) return b[2 + g] | ((b[66 + (g >> 3)] << (8 - (g & 7))) & 256);
    if constexpr (T == 19) return b[2 + g] | ((int)((rd16(b + 34 + 2 * (g >> 2)) >> (3 * (g & 3))) & 7) << 8);
    if constexpr (T == 29) return b[g] | ((b[32 + 2 * (g >> 2) + ((g & 3) >> 1)] << ((g & 1) ? 4 : 8)) & 0x700);
    return 0;
}
template <int T>
__device__ __forceinline__ void put_gidx(uint8_t* b, int g, int k) {
    if constexpr (T == 16) b[2 + 8 * (g >> 2) + (g & 3)] |= k & 255;
    if constexpr (T == 18) b[2 + g] |= k & 255;
    if constexpr (T == 17) { b[2 + 2 * g] |= k & 255; b[3 + 2 * g] |= (k >> 8) & 1; }
    if constexpr (T == 22) { b[2 + g] |= k & 255; b[66 + (g >> 2)] |= ((k >> 8) & 3) << (2 * (g & 3)); }
    if constexpr (T == 21) { b[2 + g] |= k & 255; b[66 + (g >> 3)] |= ((k >> 8) & 1) << (g & 7); }
    if constexpr (T == 19) {
        b[2 + g] |= k & 255;
        const int v = ((k >> 8) & 7) << (3 * (g & 3));
        b[34 + 2 * (g >> 2)] |= v & 255;
        b[35 + 2 * (g >> 2)] |= v >> 8;
    }
    if constexpr (T == 29) { b[g] |= k & 255; b[32 + 2 * (g >> 2) + ((g & 3) >> 1)] |= ((k >> 8) & 7) << ((g & 1) ? 4 : 0); }
}
// 1 if weight w is stored negative (parity types: the 8th sign of a group follows from the other 7)
template <int T>
__device__ __forceinline__ int get_neg(const uint8_t* b, int w) {
    const int j = w & 7;
    uint32_t s7;
    if constexpr (T == 16) s7 = (rd32(b + 2 + 8 * (w >> 5) + 4) >> (7 * ((w >> 3) & 3))) & 127;
    else if constexpr (T == 17) s7 = rd16(b + 2 + 2 * (w >> 3)) >> 9;
    else if constexpr (T == 18) s7 = (rd32(b + 66 + 4 * (w >> 5)) >> (7 * ((w >> 3) & 3))) & 127;
    else if constexpr (T == 22) return (b[34 + (w >> 3)] >> j) & 1;
    else if constexpr (T == 21) return (b[74 + (w >> 3)] >> j) & 1;
    else return 0;
    return j < 7 ? (int)((s7 >> j) & 1) : (int)(__popc(s7) & 1);
}
template <int T>
__device__ __forceinline__ void put_neg(uint8_t* b, int w) {       // parity types: w % 8 < 7
    const int j = w & 7;
    int p;
    if constexpr (T == 16) p = 8 * (2 + 8 * (w >> 5) + 4) + 7 * ((w >> 3) & 3) + j;
    else if constexpr (T == 17) p = 8 * (2 + 2 * (w >> 3)) + 9 + j;
    else if constexpr (T == 18) p = 8 * (66 + 4 * (w >> 5)) + 7 * ((w >> 3) & 3) + j;
    else if constexpr (T == 22) p = 8 * (34 + (w >> 3)) + j;
    else if constexpr (T == 21) p = 8 * (74 + (w >> 3)) + j;
    else return;
    b[p >> 3] |= (uint8_t)(1u << (p & 7));
}
__device__ __forceinline__ int get_shift(const uint8_t* b, int u) { return (b[32 + 2 * (u >> 2) + ((u & 3) >> 1)] >> ((u & 1) ? 7 : 3)) & 1; }
__device__ __forceinline__ void put_shift(uint8_t* b, int u) { b[32 + 2 * (u >> 2) + ((u & 3) >> 1)] |= (u & 1) ? 0x80 : 0x08; }

// scale s of unit u (level l has the value s (2 l + 1); IQ1: s (l - 1 + dl)), the quantizers' fudge
// factors on the stored fp16 taken back out (qr.py:449-463)
template <int T>
__device__ __forceinline__ void gscale(const uint8_t* b, int u, float& s, float& dl) {
    float d;
    int ls;
    dl = 0.f;
    if constexpr (T == 16) { d = h2f(rd16(b)); ls = b[2 + 8 * (u >> 2) + 7] >> 4; }
    if constexpr (T == 17) { d = h2f(rd16(b)); ls = (b[66 + (u >> 2)] >> (4 * ((u & 3) >> 1))) & 15; }
    if constexpr (T == 22) { d = h2f(rd16(b)) * R_IQ2S; ls = (b[74 + (u >> 2)] >> (4 * ((u & 3) >> 1))) & 15; }
    if constexpr (T == 18) { d = h2f(rd16(b)); ls = b[66 + 4 * (u >> 2) + 3] >> 4; }
    if constexpr (T == 21) { d = h2f(rd16(b)) * R_IQ3S; const int ib = u >> 2; ls = (b[106 + (ib >> 1)] >> (4 * (ib & 1))) & 15; }
    if constexpr (T == 19) {
        d = h2f(rd16(b)) * R_IQ1S;
        const uint32_t qh = rd16(b + 34 + 2 * (u >> 2));
        ls = (qh >> 12) & 7;
        dl = (qh & 0x8000) ? -0.125f : 0.125f;
    }
    if constexpr (T == 29) {
        d = h2f((uint32_t)iq1m_d(b)) * R_IQ1M;
        const int j = 2 * (u >> 2) + ((u & 3) >> 1);
        ls = (int)(rd16(b + 48 + 2 * (j >> 2)) >> (3 * (j & 3))) & 7;
        dl = get_shift(b, u) ? -0.125f : 0.125f;
    }
    s = d * (float)(2 * ls + 1);
}

struct Unit {
    float u[8], w[8];
    int pn[8];          // seed sign (after the parity flip)
    float s, dl;
};

// A block's 256 seed values and the imatrix entries of their columns, staged in LDS by the wave (four
// of each per lane) so the model reads neither from global memory one value at a time.
struct BlockSeed {
    float* x;
    float* im;
    bool has_im;
};
// stages block gw0's values into bs (all 64 lanes of the single-wave workgroup take part) and returns
// the grid types' sigma2 from the in-order sum of squares of the 256 seed values (qr.py:557-560)
template <int T>
__device__ __forceinline__ float stage_block(const BlockSeed& bs, int lane, int st, const uint8_t* sbase, int64_t gw0,
                                             const float* im, int cols) {
    __syncthreads();                              // the previous block's readers are done
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = lane + 64 * k;
        float x, h;
        seed_val(st, sbase, gw0 + i, cols, x, h);
        bs.x[i] = x;
        if (im) bs.im[i] = im[(gw0 + i) % cols];
    }
    __syncthreads();
    float sx2 = 0.f;
    for (int i = 0; i < 256; i += 4) {
        const float4 q = *reinterpret_cast<const float4*>(bs.x + i);
        sx2 += q.x * q.x;
        sx2 += q.y * q.y;
        sx2 += q.z * q.z;
        sx2 += q.w * q.w;
    }
    return (T == 16 || T == 17) ? sx2 * (1.0f / 256.f) : (2.f * sx2) * (1.0f / 256.f);
}

// targets, weights and seed signs of unit u (qr.py:569-593)
template <int T>
__device__ __forceinline__ void unit_model(const uint8_t* fb, int u, const BlockSeed& bs, float sigma2, Unit& g) {
    using Gt = G<T>;
    gscale<T>(fb, u, g.s, g.dl);
    float x[8], v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x[i] = bs.x[8 * u + i];
        float wi = sqrtf(sigma2 + x[i] * x[i]);
        if (bs.has_im) wi = wi * bs.im[8 * u + i];
        g.w[i] = wi;
        g.pn[i] = x[i] < 0.f;
        v[i] = Gt::SGN ? fabsf(x[i]) : x[i];
    }
    if constexpr (Gt::SGN && Gt::PAR) {            // odd count of negatives: the least weighty one flips
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) cnt += g.pn[i];
        if (cnt & 1) {
            int im_ = 0;
            float mn = g.w[0] * x[0] * x[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
                const float a = g.w[i] * x[i] * x[i];
                if (a < mn) { mn = a; im_ = i; }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (i == im_) { g.pn[i] ^= 1; v[i] = -v[i]; }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) g.u[i] = v[i] / g.s;
}

// the pair table of group gg: for each pair p of its coordinates and levels (la, lb), entry
// p * E + (la | lb << B) = w_a (q_la - u_a)^2 + w_b (q_lb - u_b)^2, as qr.py:505-517 lays it out.
// Lanes fill entries lane & (E - 1) of every pair (lanes beyond E write the same values again); the
// caller then synchronises the (single-wave) workgroup.
template <int T>
__device__ __forceinline__ void pair_table(float* tab, const Unit& g, int gg, int lane) {
    using Gt = G<T>;
    constexpr int E = Gt::L * Gt::L;
    const int e = lane & (E - 1);
    const int la = e & (Gt::L - 1), lb = e >> Gt::B;
    const float qa = Gt::SGN ? (float)(2 * la + 1) : (float)(la - 1) + g.dl;
    const float qb = Gt::SGN ? (float)(2 * lb + 1) : (float)(lb - 1) + g.dl;
#pragma unroll
    for (int p = 0; p < Gt::N / 2; ++p) {
        const int i = gg * Gt::N + 2 * p;
        const float ea = qa - g.u[i], eb = qb - g.u[i + 1];
        tab[p * E + e] = g.w[i] * (ea * ea) + g.w[i + 1] * (eb * eb);
    }
}
template <int T> constexpr int TAB_N = (G<T>::N / 2) * G<T>::L * G<T>::L;   // 64 (IQ3: 128) floats

// weighted distance of the point with levels `key`: N/2 table entries summed in pair order,
// NaN -> inf (qr.py:518-525)
template <int T>
__device__ __forceinline__ float pdist(const float* tab, uint32_t key) {
    using Gt = G<T>;
    constexpr int E = Gt::L * Gt::L;
    float d = 0.f;
#pragma unroll
    for (int p = 0; p < Gt::N / 2; ++p) d = d + tab[p * E + ((key >> (2 * Gt::B * p)) & (E - 1))];
    return isnan(d) ? INF : d;
}

__device__ __forceinline__ int gapctx(float d1, float d2) {
    const float g = (d2 - d1) / (d1 + 1e-30f);
    return (g >= 0.05f) + (g >= 0.2f) + (g >= 0.6f);
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
// the two smallest values of the multiset held across the wave (each lane: its own two smallest)
__device__ __forceinline__ void wave_two_min(float& a1, float& a2) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const float b1 = __shfl_xor(a1, m, 64), b2 = __shfl_xor(a2, m, 64);
        const float lo = a1 < b1 ? a1 : b1, hi = a1 < b1 ? b1 : a1;
        const float s2 = a2 < b2 ? a2 : b2;
        a1 = lo;
        a2 = hi < s2 ? hi : s2;
    }
}
__device__ __forceinline__ bool before(float da, int ka, float db, int kb) { return da < db || (da == db && ka < kb); }
__device__ __forceinline__ void wave_argmin(float& d, int& k) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const float od = __shfl_xor(d, m, 64);
        const int ok = __shfl_xor(k, m, 64);
        if (before(od, ok, d, k)) { d = od; k = ok; }
    }
}

__device__ __forceinline__ int rank_ctx0(int mv, int64_t col, int cols) {
    return mv >= 2 ? GRANK2 + 4 * (cols <= 0 || col < 256 ? 0 : 1 + (int)min((int64_t)2, col * 3 / cols)) : GRID_RANK;
}
__device__ __forceinline__ int sign_ctx0(int mv, int64_t col, int cols) {
    return mv >= 2 ? GSIGN2 + 16 * (cols <= 0 || col < 256 ? 0 : 1 + (int)min((int64_t)2, col * 3 / cols)) : GRID_SIGN;
}

template <int T>
__device__ __forceinline__ int sign_ctx(const Unit& g, const uint16_t* gk, const int (&tg)[2], int j) {
    using Gt = G<T>;
    const int t = min(tg[j / Gt::N], Gt::GS - 1);
    const int lev = (gk[t] >> (Gt::B * (j % Gt::N))) & (Gt::L - 1);
    const float m4 = fabsf(g.u[j]) * 4.f;
    return (lev == 0) * 8 + (m4 < 7.f ? (int)m4 : 7);
}

// symbol sinks of the encoder's model walk: count (histogram) or code (rANS, backwards)
struct Count {
    uint32_t* counts;
    int lane;
    __device__ __forceinline__ void put(int tab, uint32_t sym) {
        if (lane == 0) atomicAdd(&counts[tab * 256 + sym], 1u);
    }
};
struct Code {
    uint32_t x;
    uint8_t* ptr;
    const int* remap;
    const uint16_t* freq;
    const uint32_t* cum;
    int lane;
    __device__ __forceinline__ void put_fc(uint32_t f, uint32_t c) {
        const uint32_t xm = ((RANS_L >> PB) << 8) * f;
        while (x >= xm) {
            --ptr;
            if (lane == 0) *ptr = (uint8_t)(x & 0xff);
            x >>= 8;
        }
        x = ((x / f) << PB) + (x % f) + c;
    }
    __device__ __forceinline__ void put(int tab, uint32_t sym) {
        const int tt = remap[tab];
        put_fc(freq[tt * 256 + sym], cum[tt * 257 + sym]);
    }
};

// grid codes of one block in encode order (units 31..0, per unit signs 7..0, groups last to first,
// IQ1_M's shift bit last); returns false if the sink asks to stop (coder near its buffer start)
template <int T, class S, class Stop>
__device__ __forceinline__ bool grid_walk(S& out, Stop stop, const uint8_t* fb, const uint8_t* pb, const uint16_t* gk,
                                          const uint32_t (&keys)[G<T>::PER], float* tab, int lane, int st,
                                          const uint8_t* sbase, int64_t gw0, int cols, const float* im, int mv,
                                          const BlockSeed& bs) {
    using Gt = G<T>;
    const float sigma2 = stage_block<T>(bs, lane, st, sbase, gw0, im, cols);
    const int64_t col0 = cols > 0 ? gw0 % cols : 0;
    for (int u = 31; u >= 0; --u) {
        const int rank0 = rank_ctx0(mv, col0 + 8 * u, cols), sign0 = sign_ctx0(mv, col0 + 8 * u, cols);
        Unit g;
        unit_model<T>(fb, u, bs, sigma2, g);
        int tg[2] = {0, 0};
#pragma unroll
        for (int gg = 0; gg < Gt::NG; ++gg) tg[gg] = get_gidx<T>(fb, u * Gt::NG + gg);
        if constexpr (Gt::SGN) {
#pragma unroll
            for (int j = 7; j >= 0; --j) {
                if (Gt::PAR && j == 7) continue;
                out.put(sign0 + sign_ctx<T>(g, gk, tg, j), (uint32_t)(get_neg<T>(fb, 8 * u + j) ^ g.pn[j]));
            }
        }
#pragma unroll
        for (int gg = Gt::NG - 1; gg >= 0; --gg) {
            pair_table<T>(tab, g, gg, lane);
            __syncthreads();
            const int t = tg[gg];
            const float dt = pdist<T>(tab, gk[t]);
            int cnt = 0;
            float m1 = INF, m2 = INF;
#pragma unroll
            for (int i = 0; i < Gt::PER; ++i) {
                const int k = lane + 64 * i;
                const float d = pdist<T>(tab, keys[i]);
                cnt += (d < dt || (d == dt && k < t)) ? 1 : 0;
                if (d < m1) { m2 = m1; m1 = d; } else if (d < m2) m2 = d;
            }
            __syncthreads();
            const int rank = wave_sum(cnt);
            wave_two_min(m1, m2);
            const int ctx = gapctx(m1, m2);
            if (rank >= TOPK) {
                out.put(FESC_HI, (uint32_t)(t >> 8));
                out.put(FESC_LO, (uint32_t)(t & 255));
                out.put(rank0 + ctx, TOPK);
            } else {
                out.put(rank0 + ctx, (uint32_t)rank);
            }
        }
        if constexpr (T == 29) out.put(GRID_SHIFT, (uint32_t)(get_shift(fb, u) ^ get_shift(pb, u)));
        if (stop(out)) return false;
    }
    return true;
}

template <int T>
__device__ __forceinline__ void load_keys(const uint16_t* gk, int lane, uint32_t (&keys)[G<T>::PER]) {
#pragma unroll
    for (int i = 0; i < G<T>::PER; ++i) keys[i] = gk[lane + 64 * i];
}

// one wavefront per differing block of the list (slot = segment * SEG_BLOCKS + block), the grid's
// waves striding over it; the flag symbols were counted with the list
template <int T>
__global__ __launch_bounds__(64) void k_qrg_hist(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                                 const uint8_t* __restrict__ seed, const TM* __restrict__ tm,
                                                 const SG* __restrict__ sg, const uint32_t* __restrict__ list,
                                                 const uint32_t* __restrict__ nlist, uint32_t* __restrict__ counts,
                                                 const uint16_t* __restrict__ gk, const float* __restrict__ imx, int mv) {
    using Y = Ty<T>;
    constexpr int SEG = SEG_BLOCKS<T>;
    const int lane = threadIdx.x;
    __shared__ float tab[TAB_N<T>];
    __shared__ __align__(16) float sx[256], sim[256];
    uint32_t keys[G<T>::PER];
    load_keys<T>(gk, lane, keys);
    const uint32_t n = *nlist;
    for (uint32_t i = blockIdx.x; i < n; i += gridDim.x) {
        const uint32_t slot = list[i];
        const SG g = sg[slot / SEG];
        const TM m = tm[g.t];
        const int64_t b = g.b0 + (int)(slot % SEG);
        const uint8_t* fb = F + b * Y::BS;
        const uint8_t* pb = P + b * Y::BS;
        Count out{counts, lane};
        int tv[Y::NF];
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) tv[k] = get_field<T>(fb, k);
        int any = 0;
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) {
            const int kd = fkind<T>(k), dlt = tv[k] - fpred<T>(mv, pb, k, tv[0], tv[1]);
            if (kd < 2 && (dlt < -127 || dlt > 127)) {
                out.put(kd * 2 + any, 128);
                out.put(FESC_LO, (uint32_t)(tv[k] & 255));
                out.put(FESC_HI, (uint32_t)(tv[k] >> 8));
            } else {
                out.put(kd * 2 + any, (uint32_t)(dlt & 255));
            }
            any |= dlt != 0;
        }
        const float* im = (m.imx_off >= 0 && m.cols > 0) ? imx + m.imx_off : nullptr;
        grid_walk<T>(out, [](Count&) { return false; }, fb, pb, gk, keys, tab, lane, m.seed_type, seed + m.seed_off,
                     (b - m.blk0) * Y::QK, m.cols, im, mv, BlockSeed{sx, sim, im != nullptr});
    }
}

// room kept below the coder's write pointer for one more unit, the block's fields and its flag
constexpr int64_t ROOM = 256;

template <int T>
__global__ __launch_bounds__(64) void k_qrg_enc(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                                const uint8_t* __restrict__ seed, const TM* __restrict__ tm,
                                                const SG* __restrict__ sg, int nseg, const int* __restrict__ remap,
                                                const uint16_t* __restrict__ freq, const uint32_t* __restrict__ cum,
                                                uint8_t* __restrict__ out, uint64_t cap, uint32_t* __restrict__ out_len,
                                                const uint16_t* __restrict__ gk, const float* __restrict__ imx,
                                                const uint8_t* __restrict__ neq, int mv) {
    using Y = Ty<T>;
    const int lane = threadIdx.x;
    const int s = blockIdx.x;
    if (s >= nseg) return;
    const SG g = sg[s];
    const TM m = tm[g.t];
    const uint8_t* sbase = seed + m.seed_off;
    const float* im = (m.imx_off >= 0 && m.cols > 0) ? imx + m.imx_off : nullptr;
    uint8_t* const base = out + (uint64_t)s * cap;
    uint8_t* const end = base + cap;
    __shared__ float tab[TAB_N<T>];
    __shared__ __align__(16) float sx[256], sim[256];
    uint32_t keys[G<T>::PER];
    load_keys<T>(gk, lane, keys);
    Code e{RANS_L, end, remap, freq, cum, lane};
    auto stop = [base](Code& c) { return c.ptr - base < ROOM; };
    // the segment's block flags as one mask (a segment has at most 64 blocks), the flag tables in registers
    static_assert(SEG_BLOCKS<T> <= 64, "one mask bit per block of the segment");
    const uint64_t nm = __ballot(lane < g.nb && neq[g.b0 + lane] != 0);
    FlagTab ft;
    ft.load(remap, freq, cum);
    for (int64_t b = g.b0 + g.nb - 1; b >= g.b0; --b) {
        const uint8_t* fb = F + b * Y::BS;
        const uint8_t* pb = P + b * Y::BS;
        const int i = (int)(b - g.b0);
        const bool eq = !((nm >> i) & 1u);
        const int prev = i > 0 ? (((nm >> (i - 1)) & 1u) ? 0 : 1) : 1;
        if (eq) {
            e.put_fc(ft.freq_of(prev, 1), ft.cum_of(prev, 1));
            if (stop(e)) { if (lane == 0) out_len[s] = 0xffffffffu; return; }
            continue;
        }
        if (!grid_walk<T>(e, stop, fb, pb, gk, keys, tab, lane, m.seed_type, sbase, (b - m.blk0) * Y::QK, m.cols, im, mv,
                          BlockSeed{sx, sim, im != nullptr})) {
            if (lane == 0) out_len[s] = 0xffffffffu;
            return;
        }
        int tv[Y::NF], dl[Y::NF], anyk[Y::NF];
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) tv[k] = get_field<T>(fb, k);
        int any = 0;
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) {
            dl[k] = tv[k] - fpred<T>(mv, pb, k, tv[0], tv[1]);
            anyk[k] = any;
            any |= dl[k] != 0;
        }
#pragma unroll
        for (int k = Y::NF - 1; k >= 0; --k) {
            const int kd = fkind<T>(k);
            if (kd < 2 && (dl[k] < -127 || dl[k] > 127)) {
                e.put(FESC_HI, (uint32_t)(tv[k] >> 8));
                e.put(FESC_LO, (uint32_t)(tv[k] & 255));
                e.put(kd * 2 + anyk[k], 128);
            } else {
                e.put(kd * 2 + anyk[k], (uint32_t)(dl[k] & 255));
            }
        }
        e.put_fc(ft.freq_of(prev, 0), ft.cum_of(prev, 0));
    }
    for (int i = 0; i < 4; ++i) {
        --e.ptr;
        if (lane == 0) *e.ptr = (uint8_t)(e.x & 0xff);
        e.x >>= 8;
    }
    if (lane == 0) out_len[s] = (uint32_t)(end - e.ptr);
}

struct Decoder {
    uint32_t x;
    ByteQ bq;
    const int* remap;
    const uint16_t* freq;
    const uint32_t* cum;
    const uint32_t* lut;
    __device__ __forceinline__ int get(int tab) {
        // one load per symbol: its LUT32 entry holds the symbol, freq - 1 and slot - cum
        const int tt = remap[tab];
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

template <int T>
__global__ __launch_bounds__(64) void k_qrg_dec(const uint8_t* __restrict__ in, uint64_t in_bytes,
                                                const uint64_t* __restrict__ in_off,
                                                const uint8_t* __restrict__ P, const uint8_t* __restrict__ seed,
                                                const TM* __restrict__ tm, const SG* __restrict__ sg, int nseg,
                                                const int* __restrict__ remap, const uint16_t* __restrict__ freq,
                                                const uint32_t* __restrict__ cum, const uint32_t* __restrict__ lut,
                                                uint8_t* __restrict__ F, const uint16_t* __restrict__ gk,
                                                const float* __restrict__ imx, int mv) {
    using Y = Ty<T>;
    using Gt = G<T>;
    constexpr int BSW = (Y::BS + 3) / 4;
    __shared__ uint32_t blk32[BSW];
    __shared__ float tab[TAB_N<T>];
    __shared__ __align__(16) float sx[256], sim[256];
    uint8_t* blk = reinterpret_cast<uint8_t*>(blk32);
    const int lane = threadIdx.x;
    const int s = blockIdx.x;
    if (s >= nseg) return;
    const SG g = sg[s];
    const TM m = tm[g.t];
    const uint8_t* sbase = seed + m.seed_off;
    const float* im = (m.imx_off >= 0 && m.cols > 0) ? imx + m.imx_off : nullptr;
    const BlockSeed bs{sx, sim, im != nullptr};
    uint32_t keys[Gt::PER];
    load_keys<T>(gk, lane, keys);
    const uint8_t* const in_end = in + in_bytes;
    Decoder d{0, {}, remap, freq, cum, lut};
    d.bq.start(in + (in_off[s] < in_bytes ? in_off[s] : in_bytes), in_end);
    for (int i = 0; i < 4; ++i) d.x = (d.x << 8) | d.bq.next();
    FlagTab ft;
    ft.load(remap, freq, cum);
    int prev = 1;
    for (int64_t b = g.b0; b < g.b0 + g.nb; ++b) {
        const uint8_t* pb = P + b * Y::BS;
        uint8_t* dst = F + b * Y::BS;
        const int eq = ft.get(d.x, d.bq, prev);
        prev = eq;
        if (eq) continue;                         // F holds P's bytes already (qr_prefill)
        // every lane applies the same writes to the block in LDS, so each lane's reads see them
#pragma unroll
        for (int i = 0; i < BSW; ++i) blk32[i] = 0;
        int vals[Y::NF];
        int any = 0;
#pragma unroll
        for (int k = 0; k < Y::NF; ++k) {
            const int kd = fkind<T>(k);
            const int pr = fpred<T>(mv, pb, k, k > 0 ? vals[0] : 0, 0);
            const int sym = d.get(kd * 2 + any);
            int t;
            if (kd < 2 && sym == 128) {
                const int lo = d.get(FESC_LO), hi = d.get(FESC_HI);
                t = lo | (hi << 8);
            } else {
                t = pr + s8((uint32_t)sym);
                if (kd < 2) t &= 0xffff;
            }
            vals[k] = t;
            any |= t != pr;
        }
        set_fields<T>(blk, vals);
        const int64_t gw0 = (b - m.blk0) * Y::QK;
        const int64_t col0 = m.cols > 0 ? gw0 % m.cols : 0;
        const float sigma2 = stage_block<T>(bs, lane, m.seed_type, sbase, gw0, im, m.cols);
        for (int u = 0; u < 32; ++u) {
            const int rank0 = rank_ctx0(mv, col0 + 8 * u, m.cols), sign0 = sign_ctx0(mv, col0 + 8 * u, m.cols);
            if constexpr (T == 29) {
                const int sh = d.get(GRID_SHIFT);
                if (sh ^ get_shift(pb, u)) put_shift(blk, u);
            }
            Unit gu;
            unit_model<T>(blk, u, bs, sigma2, gu);
            int tg[2] = {0, 0};
#pragma unroll
            for (int gg = 0; gg < Gt::NG; ++gg) {
                pair_table<T>(tab, gu, gg, lane);
                __syncthreads();
                float dist[Gt::PER];
#pragma unroll
                for (int i = 0; i < Gt::PER; ++i) dist[i] = pdist<T>(tab, keys[i]);
                __syncthreads();
                // points in (distance, index) order over the finite distances, one per round
                float ld = 0.f;
                int lk = -1, found = 0;
                auto next = [&](float& bd, int& bk) {
                    bd = INF;
                    bk = 0x7fffffff;
#pragma unroll
                    for (int i = 0; i < Gt::PER; ++i) {
                        const int k = lane + 64 * i;
                        const float dd = dist[i];
                        if (dd < INF && (lk < 0 || before(ld, lk, dd, k)) && before(dd, k, bd, bk)) { bd = dd; bk = k; }
                    }
                    wave_argmin(bd, bk);
                    if (bk == 0x7fffffff) return false;
                    ld = bd;
                    lk = bk;
                    ++found;
                    return true;
                };
                float d1 = INF, d2 = INF;
                int k1 = 0, k2 = 0;
                if (next(d1, k1)) next(d2, k2);
                if (found < 2) d2 = INF;
                if (found < 1) d1 = INF;
                const int r = d.get(rank0 + gapctx(d1, d2));
                int t;
                if (r >= TOPK) {
                    const int lo = d.get(FESC_LO), hi = d.get(FESC_HI);
                    t = lo | (hi << 8);
                } else if (r == 0 && found >= 1) {
                    t = k1;
                } else if (r == 1 && found >= 2) {
                    t = k2;
                } else {
                    float dn;
                    int kn = 0;
                    while (found <= r && found >= 2 && next(dn, kn)) {}
                    t = found > r ? kn : r - found;
                }
                put_gidx<T>(blk, u * Gt::NG + gg, t);
                tg[gg] = t;
            }
            if constexpr (Gt::SGN) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (Gt::PAR && j == 7) continue;
                    const int sym = d.get(sign0 + sign_ctx<T>(gu, gk, tg, j));
                    if (sym ^ gu.pn[j]) put_neg<T>(blk, 8 * u + j);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (Y::BS + 63) / 64; ++i)
            if (lane + 64 * i < Y::BS) dst[lane + 64 * i] = blk[lane + 64 * i];
    }
}

template <template <int> class K, class... A>
int dispatch_grid(int T, A&&... args) {
    switch (T) {
        case 16: return K<16>::run(args...);
        case 17: return K<17>::run(args...);
        case 18: return K<18>::run(args...);
        case 19: return K<19>::run(args...);
        case 21: return K<21>::run(args...);
        case 22: return K<22>::run(args...);
        case 29: return K<29>::run(args...);
    }
    return fail(SPA_ERR_TYPE, "QR: type %d is not a grid type", T);
}

template <int T> struct GHist {
    static int run(const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, uint32_t* counts,
                   const uint16_t* gk, const float* imx, int mv, void* work, hipStream_t st) {
        const int64_t n = (int64_t)nseg * SEG_BLOCKS<T>;
        const QrWork w = qr_work(work, n, 0);
        if (int e = qr_flags(F, P, sg, nseg, SEG_BLOCKS<T>, Ty<T>::BS, w, counts, false, st)) return e;
        // one wave per differing block; at most 16384 waves stride over the list
        const int64_t waves = n < 16384 ? n : 16384;
        hipLaunchKernelGGL(k_qrg_hist<T>, dim3((unsigned)waves), dim3(64), 0, st, (const uint8_t*)F, (const uint8_t*)P,
                           (const uint8_t*)seed, (const TM*)tm, (const SG*)sg, (const uint32_t*)w.list,
                           (const uint32_t*)w.nlist, counts, gk, imx, mv);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct GEnc {
    static int run(const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, const int* remap,
                   const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap, uint32_t* out_len, const uint16_t* gk,
                   const float* imx, int mv, void* work, hipStream_t st) {
        const QrWork w = qr_work(work, (int64_t)nseg * SEG_BLOCKS<T>, 0);
        if (int e = qr_flags(F, P, sg, nseg, SEG_BLOCKS<T>, Ty<T>::BS, w, nullptr, false, st)) return e;
        hipLaunchKernelGGL(k_qrg_enc<T>, dim3((unsigned)nseg), dim3(64), 0, st, (const uint8_t*)F, (const uint8_t*)P,
                           (const uint8_t*)seed, (const TM*)tm, (const SG*)sg, nseg, remap, freq, cum, (uint8_t*)out, cap,
                           out_len, gk, imx, (const uint8_t*)w.neq, mv);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
template <int T> struct GDec {
    static int run(const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* P, const void* seed, const void* tm, const void* sg,
                   int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum, const uint32_t* lut, void* F,
                   const uint16_t* gk, const float* imx, int mv, hipStream_t st) {
        if (int e = qr_prefill(F, P, sg, nseg, Ty<T>::BS, st)) return e;
        hipLaunchKernelGGL(k_qrg_dec<T>, dim3((unsigned)nseg), dim3(64), 0, st, (const uint8_t*)in, in_bytes, in_off, (const uint8_t*)P,
                           (const uint8_t*)seed, (const TM*)tm, (const SG*)sg, nseg, remap, freq, cum, lut, (uint8_t*)F, gk,
                           imx, mv);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};

}  // namespace

namespace {
// per weight of grid-type blocks: half the step between the grid's levels around it (qr.py:811-817)
template <int T>
__global__ __launch_bounds__(256) void k_grid_h(const uint8_t* __restrict__ F, int64_t nw, float* __restrict__ h) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nw) return;
    float s, dl;
    gscale<T>(F + (i / 256) * Ty<T>::BS, (int)(i % 256) / 8, s, dl);
    h[i] = (T == 19 || T == 29) ? 0.5f * fabsf(s) : fabsf(s);
}
template <int T> struct GridH {
    static int run(const void* F, int64_t nw, float* h, hipStream_t st) {
        hipLaunchKernelGGL(k_grid_h<T>, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, st, (const uint8_t*)F, nw, h);
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
};
}  // namespace

int grid_half_steps(int T, const void* F, int64_t nw, float* h, hipStream_t st) {
    return dispatch_grid<GridH>(T, F, nw, h, st);
}

int grid_hist(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, uint32_t* counts,
              const uint16_t* gk, const float* imx, int mv, void* work, hipStream_t st) {
    return dispatch_grid<GHist>(T, F, P, seed, tm, sg, nseg, counts, gk, imx, mv, work, st);
}
int grid_encode(int T, const void* F, const void* P, const void* seed, const void* tm, const void* sg, int nseg, const int* remap,
                const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap, uint32_t* out_len, const uint16_t* gk,
                const float* imx, int mv, void* work, hipStream_t st) {
    return dispatch_grid<GEnc>(T, F, P, seed, tm, sg, nseg, remap, freq, cum, out, cap, out_len, gk, imx, mv, work, st);
}
int grid_decode(int T, const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* P, const void* seed,
                const void* tm, const void* sg, int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum,
                const uint32_t* lut, void* F, const uint16_t* gk, const float* imx, int mv, hipStream_t st) {
    return dispatch_grid<GDec>(T, in, in_bytes, in_off, P, seed, tm, sg, nseg, remap, freq, cum, lut, F, gk, imx, mv, st);
}

}  // namespace qr
}  // namespace spa
