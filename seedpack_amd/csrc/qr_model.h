// QR residual model for the non-grid quant types (device side).
//
// A block of the file (F) is coded against the predicted block (P) and the seed weights:
//   flag      1 if F == P (context: the previous block's flag within the segment);
//   fields    the integer scale fields of F, each as a difference to P's field rescaled to F's
//             fp16 super-scale (fp16 fields escape to raw bytes beyond +-127);
//   codes     each code as (s * (code - r)) & 255, r = round((x - c) / a) from F's own scales and
//             the seed value x, s the side of the rounding; context = the weight's place in its row
//             and the distance of (x - c) / a to the rounding boundary.
// The symbol alphabet, the contexts and every float operation follow seedpack/qr.py:78-377 exactly:
// the archive stream depends on them. Types are template parameters, so every per-type switch
// folds at compile time.
#pragma once

#include "common.h"

namespace spa {
namespace qr {

constexpr int PB = 12;
constexpr uint32_t PSCALE = 1u << PB;
constexpr uint32_t RANS_L = 1u << 23;
constexpr int NSB_MAX = 20;
constexpr int NTAB = NSB_MAX + 64 + 2;
constexpr int FLAG = NSB_MAX + 64;     // + previous block's flag
constexpr int CODE2 = NTAB;            // exact seeds: position (8) x margin (16)
constexpr int NTAB2 = NTAB + 208;
constexpr int FESC_LO = 8, FESC_HI = 9;
constexpr int MAXF = 34;

// Next stream byte for the decoders' renormalisation: reads stop at `end` (zeros past it), so a
// damaged or truncated stream decodes to garbage without leaving its buffer.
__device__ __forceinline__ uint32_t next_byte(const uint8_t*& ptr, const uint8_t* end) {
    const uint32_t b = ptr < end ? *ptr : 0u;
    ++ptr;
    return b;
}

// The decoders' byte source: the next four stream bytes held in registers, each refilled by a load
// issued as a byte leaves, so a renormalisation waits only on loads issued four bytes earlier (the
// same bytes as next_byte, in order; zeros past `end`, nothing read past it).
struct ByteQ {
    const uint8_t* ptr;                          // the next byte to load
    const uint8_t* end;
    uint32_t b0, b1, b2, b3;
    __device__ __forceinline__ void start(const uint8_t* p, const uint8_t* e) {
        ptr = p;
        end = e;
        b0 = next_byte(ptr, end);
        b1 = next_byte(ptr, end);
        b2 = next_byte(ptr, end);
        b3 = next_byte(ptr, end);
    }
    __device__ __forceinline__ uint32_t next() {
        const uint32_t v = b0;
        b0 = b1;
        b1 = b2;
        b2 = b3;
        b3 = next_byte(ptr, end);
        return v;
    }
};

// Frequencies of the flag symbols 0 and 1 in the two flag contexts p (previous block differing /
// equal): every block codes a flag, most blocks nothing else. A context's symbol 0 starts at 0 and
// symbol 1 at freq(p, 0) (the tables' cumulative counts), so four 16-bit frequencies say everything;
// they sit in one 64-bit register, context p in bits 32p.., symbol v in bits 16v.. of it, and are
// picked by shifts: a pick between separate fields may be turned into an indexed load from a copy of
// the structure in scratch memory. A context without symbols in the batch reads as 0 (a valid batch
// never codes it).
struct FlagTab {
    uint64_t q;
    __device__ __forceinline__ void load(const int* remap, const uint16_t* freq, const uint32_t* cum) {
        (void)cum;
        q = 0;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int tt = remap[FLAG + p];
            if (tt >= 0) q |= (uint64_t)(freq[tt * 256] | ((uint32_t)freq[tt * 256 + 1] << 16)) << (32 * p);
        }
    }
    __device__ __forceinline__ uint32_t freq_of(int p, int v) const {
        return (uint32_t)(q >> (32 * p + 16 * v)) & 0xffffu;
    }
    __device__ __forceinline__ uint32_t cum_of(int p, int v) const { return v ? freq_of(p, 0) : 0u; }
    // the encoder's reciprocals of the four flag frequencies (enc_rcp), held as (v = 0, v = 1) pairs
    uint64_t r0, r1;
    __device__ __forceinline__ void load_rcp(const int* remap, const uint32_t* rcp) {
        r0 = r1 = 0;
        const int t0 = remap[FLAG], t1 = remap[FLAG + 1];
        if (t0 >= 0) r0 = rcp[t0 * 256] | ((uint64_t)rcp[t0 * 256 + 1] << 32);
        if (t1 >= 0) r1 = rcp[t1 * 256] | ((uint64_t)rcp[t1 * 256 + 1] << 32);
    }
    __device__ __forceinline__ uint32_t rcp_of(int p, int v) const { return (uint32_t)((p ? r1 : r0) >> (32 * v)); }
    // one flag decoded from state x in context p: symbol 1's slots start at freq(p, 0), symbol 0's at 0
    // (a valid stream's slot is in one of the two ranges); renormalised from ptr as the general step
    __device__ __forceinline__ int get(uint32_t& x, ByteQ& bq, int p) const {
        const uint32_t slot = x & (PSCALE - 1);
        const uint32_t w = (uint32_t)(q >> (32 * p));
        const uint32_t f0 = w & 0xffffu;
        const int v = slot >= f0 ? 1 : 0;
        x = (w >> (16 * v) & 0xffffu) * (x >> PB) + slot - (v ? f0 : 0u);
#pragma unroll
        for (int i = 0; i < 4 && x < RANS_L; ++i) x = (x << 8) | bq.next();
        return v;
    }
};

// kvalues_iq4nl (ggml-common.h:1120) as floats: the non-linear code values of IQ4_NL / IQ4_XS
__constant__ const float KV[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// descriptors shared with the host (byte layout of seedpack/qr.py:898-900 TM_DT / SG_DT)
struct TM { int64_t blk0, seed_off; int32_t seed_type, cols; int64_t imx_off; };
struct SG { int32_t t, nb; int64_t b0; };
static_assert(sizeof(TM) == 32 && sizeof(SG) == 16, "descriptor layout");

template <int T> struct Ty;
#define SPA_QR_TYPE(t, qk, bs, nf, qmin, qmax, sublen) \
    template <> struct Ty<t> { static constexpr int QK = qk, BS = bs, NF = nf, QMIN = qmin, QMAX = qmax, SUBLEN = sublen; };
SPA_QR_TYPE(2, 32, 18, 1, 0, 15, 32)     // Q4_0
SPA_QR_TYPE(3, 32, 20, 2, 0, 15, 32)     // Q4_1
SPA_QR_TYPE(6, 32, 22, 1, 0, 31, 32)     // Q5_0
SPA_QR_TYPE(7, 32, 24, 2, 0, 31, 32)     // Q5_1
SPA_QR_TYPE(8, 32, 34, 1, -128, 127, 32) // Q8_0
SPA_QR_TYPE(10, 256, 84, 34, 0, 3, 16)   // Q2_K
SPA_QR_TYPE(11, 256, 110, 17, 0, 7, 16)  // Q3_K
SPA_QR_TYPE(12, 256, 144, 18, 0, 15, 32) // Q4_K
SPA_QR_TYPE(13, 256, 176, 18, 0, 31, 32) // Q5_K
SPA_QR_TYPE(14, 256, 210, 17, 0, 63, 16) // Q6_K
SPA_QR_TYPE(20, 32, 18, 1, 0, 15, 32)    // IQ4_NL
SPA_QR_TYPE(23, 256, 136, 9, 0, 15, 32)  // IQ4_XS
SPA_QR_TYPE(42, 64, 18, 1, 0, 3, 32)     // Q2_0
// grid types: codes are lattice points, not integers (QMIN / QMAX / SUBLEN unused)
SPA_QR_TYPE(16, 256, 66, 9, 0, 0, 32)    // IQ2_XXS
SPA_QR_TYPE(17, 256, 74, 17, 0, 0, 32)   // IQ2_XS
SPA_QR_TYPE(18, 256, 98, 9, 0, 0, 32)    // IQ3_XXS
SPA_QR_TYPE(19, 256, 50, 9, 0, 0, 32)    // IQ1_S
SPA_QR_TYPE(21, 256, 110, 9, 0, 0, 32)   // IQ3_S
SPA_QR_TYPE(22, 256, 82, 17, 0, 0, 32)   // IQ2_S
SPA_QR_TYPE(29, 256, 56, 17, 0, 0, 32)   // IQ1_M
#undef SPA_QR_TYPE

template <int T> constexpr bool NONLIN = T == 20 || T == 23;
template <int T> constexpr bool GRIDT = T == 16 || T == 17 || T == 18 || T == 19 || T == 21 || T == 22 || T == 29;
template <int T> constexpr int SEG_BLOCKS = Ty<T>::QK >= 1024 ? 16 : (16384 / Ty<T>::QK > 16 ? 16384 / Ty<T>::QK : 16);

__device__ __forceinline__ uint32_t rd16(const uint8_t* b) { return (uint32_t)b[0] | ((uint32_t)b[1] << 8); }
__device__ __forceinline__ float h2f(uint32_t h) { return f16_to_f32(h & 0xffffu); }
__device__ __forceinline__ int s8(uint32_t v) { return (int)(int8_t)(uint8_t)v; }

__device__ __forceinline__ void k4_scale_min(int j, const uint8_t* q, int& sc, int& m) {
    if (j < 4) { sc = q[j] & 63; m = q[j + 4] & 63; }
    else { sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}
// 6-bit scale i of a Q3_K block (0..63): low nibble from bytes 0..7, two high bits from bytes 8..11
__device__ __forceinline__ int q3k_scale(const uint8_t* s, int i) {
    const int lo = i < 8 ? (s[i] & 15) : (s[i - 8] >> 4);
    const int hi = (s[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return lo | (hi << 4);
}

// ---- codes
template <int T>
__device__ __forceinline__ int get_code(const uint8_t* b, int w) {
    if constexpr (T == 2 || T == 20) return w < 16 ? (b[2 + w] & 15) : (b[2 + w - 16] >> 4);
    if constexpr (T == 3) return w < 16 ? (b[4 + w] & 15) : (b[4 + w - 16] >> 4);
    if constexpr (T == 6 || T == 7) {
        constexpr int QS = T == 6 ? 6 : 8, QH = T == 6 ? 2 : 4;
        const int lo = w < 16 ? (b[QS + w] & 15) : (b[QS + w - 16] >> 4);
        return lo | (((b[QH + (w >> 3)] >> (w & 7)) & 1) << 4);
    }
    if constexpr (T == 8) return s8(b[2 + w]);
    if constexpr (T == 10) { const int n = w >> 7, r = w & 127; return (b[16 + 32 * n + (r & 31)] >> (2 * (r >> 5))) & 3; }
    if constexpr (T == 11) {
        const int n = w >> 7, r = w & 127, j = r >> 5, l = r & 31;
        return ((b[32 + 32 * n + l] >> (2 * j)) & 3) | (((b[l] >> (4 * n + j)) & 1) << 2);
    }
    if constexpr (T == 12 || T == 13) {
        const int c = w >> 6, hf = (w >> 5) & 1, l = w & 31;
        const int v = b[(T == 12 ? 16 : 48) + 32 * c + l];
        const int q = hf ? v >> 4 : v & 15;
        if constexpr (T == 12) return q;
        else return q | (((b[16 + l] >> (2 * c + hf)) & 1) << 4);
    }
    if constexpr (T == 14) {
        const int n = w >> 7, r = w & 127, g = r >> 5, l = r & 31;
        const int v = b[64 * n + l + ((g & 1) ? 32 : 0)];
        return ((g < 2) ? (v & 15) : (v >> 4)) | (((b[128 + 32 * n + l] >> (2 * g)) & 3) << 4);
    }
    if constexpr (T == 23) { const int ib = w >> 5, l = w & 31; const int v = b[8 + 16 * ib + (l & 15)]; return l < 16 ? (v & 15) : (v >> 4); }
    if constexpr (T == 42) return (b[2 + (w >> 2)] >> (2 * (w & 3))) & 3;
    return 0;
}

// ORs code q of weight w into a block whose code bytes start at zero
template <int T>
__device__ __forceinline__ void put_code(uint8_t* b, int w, int q) {
    if constexpr (T == 2 || T == 20) { if (w < 16) b[2 + w] |= q; else b[2 + w - 16] |= q << 4; }
    if constexpr (T == 3) { if (w < 16) b[4 + w] |= q; else b[4 + w - 16] |= q << 4; }
    if constexpr (T == 6 || T == 7) {
        constexpr int QS = T == 6 ? 6 : 8, QH = T == 6 ? 2 : 4;
        if (w < 16) b[QS + w] |= q & 15; else b[QS + w - 16] |= (q & 15) << 4;
        b[QH + (w >> 3)] |= ((q >> 4) & 1) << (w & 7);
    }
    if constexpr (T == 8) b[2 + w] = (uint8_t)q;
    if constexpr (T == 10) { const int n = w >> 7, r = w & 127; b[16 + 32 * n + (r & 31)] |= (q & 3) << (2 * (r >> 5)); }
    if constexpr (T == 11) {
        const int n = w >> 7, r = w & 127, j = r >> 5, l = r & 31;
        b[32 + 32 * n + l] |= (q & 3) << (2 * j);
        b[l] |= ((q >> 2) & 1) << (4 * n + j);
    }
    if constexpr (T == 12) { const int c = w >> 6, hf = (w >> 5) & 1, l = w & 31; b[16 + 32 * c + l] |= hf ? q << 4 : q; }
    if constexpr (T == 13) {
        const int c = w >> 6, hf = (w >> 5) & 1, l = w & 31;
        b[48 + 32 * c + l] |= hf ? (q & 15) << 4 : (q & 15);
        b[16 + l] |= ((q >> 4) & 1) << (2 * c + hf);
    }
    if constexpr (T == 14) {
        const int n = w >> 7, r = w & 127, g = r >> 5, l = r & 31;
        b[64 * n + l + ((g & 1) ? 32 : 0)] |= (g < 2) ? (q & 15) : ((q & 15) << 4);
        b[128 + 32 * n + l] |= ((q >> 4) & 3) << (2 * g);
    }
    if constexpr (T == 23) { const int ib = w >> 5, l = w & 31; b[8 + 16 * ib + (l & 15)] |= l < 16 ? q : q << 4; }
    if constexpr (T == 42) b[2 + (w >> 2)] |= (q & 3) << (2 * (w & 3));
}

// ---- scale fields (integers: fp16 bits of d / dmin / m, the 4-, 6-, 8-bit sub-scales and sub-mins)
// 0 = fp16 scale, 1 = fp16 min, 2 = sub-scale, 3 = sub-min
template <int T>
__device__ __forceinline__ int fkind(int k) {
    if constexpr (T == 3 || T == 7) return k == 0 ? 0 : 1;
    if constexpr (T == 10) return k == 0 ? 0 : (k == 1 ? 1 : (k < 18 ? 2 : 3));
    if constexpr (T == 12 || T == 13) return k == 0 ? 0 : (k == 1 ? 1 : (k < 10 ? 2 : 3));
    if constexpr (T == 11 || T == 14 || T == 23 || GRIDT<T>) return k == 0 ? 0 : 2;
    return 0;
}

// IQ1_M: the fp16 super-scale bits kept in the top nibbles of the four scale words
__device__ __forceinline__ int iq1m_d(const uint8_t* b) {
    return (int)((rd16(b + 48) >> 12) | ((rd16(b + 50) >> 8) & 0xf0) | ((rd16(b + 52) >> 4) & 0xf00) | (rd16(b + 54) & 0xf000));
}

template <int T>
__device__ __forceinline__ int get_field(const uint8_t* b, int k) {
    if constexpr (T == 2 || T == 6 || T == 8 || T == 20 || T == 42) return (int)rd16(b);
    if constexpr (T == 3 || T == 7) return (int)rd16(b + 2 * k);
    if constexpr (T == 10) {
        if (k == 0) return (int)rd16(b + 80);
        if (k == 1) return (int)rd16(b + 82);
        return k < 18 ? (b[k - 2] & 15) : (b[k - 18] >> 4);
    }
    if constexpr (T == 11) return k == 0 ? (int)rd16(b + 108) : q3k_scale(b + 96, k - 1);
    if constexpr (T == 12 || T == 13) {
        if (k < 2) return (int)rd16(b + 2 * k);
        int sc, m;
        k4_scale_min(k < 10 ? k - 2 : k - 10, b + 4, sc, m);
        return k < 10 ? sc : m;
    }
    if constexpr (T == 14) return k == 0 ? (int)rd16(b + 208) : s8(b[192 + k - 1]);
    if constexpr (T == 23) {
        if (k == 0) return (int)rd16(b);
        const int ib = k - 1, sh = (int)rd16(b + 2);
        return ((b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
    }
    // grid types: fp16 d, then the 4-bit (IQ1: 3-bit; IQ1_S with its shift bit) sub-block scales
    if constexpr (T == 29) {
        if (k == 0) return iq1m_d(b);
        const int j = k - 1;
        return (int)(rd16(b + 48 + 2 * (j >> 2)) >> (3 * (j & 3))) & 7;
    }
    if constexpr (T == 16) return k == 0 ? (int)rd16(b) : b[2 + 8 * (k - 1) + 7] >> 4;
    if constexpr (T == 18) return k == 0 ? (int)rd16(b) : b[66 + 4 * (k - 1) + 3] >> 4;
    if constexpr (T == 17 || T == 22 || T == 21) {
        constexpr int O = T == 17 ? 66 : T == 22 ? 74 : 106;
        return k == 0 ? (int)rd16(b) : (b[O + (k - 1) / 2] >> (4 * ((k - 1) % 2))) & 15;
    }
    if constexpr (T == 19) return k == 0 ? (int)rd16(b) : b[34 + 2 * (k - 1) + 1] >> 4;
    return 0;
}

__device__ __forceinline__ void wr16(uint8_t* b, int v) { b[0] = (uint8_t)(v & 255); b[1] = (uint8_t)((v >> 8) & 255); }

// writes every scale field of a block whose scale bytes start at zero
template <int T>
__device__ __forceinline__ void set_fields(uint8_t* b, const int (&v)[Ty<T>::NF]) {
    if constexpr (T == 2 || T == 6 || T == 8 || T == 20 || T == 42) wr16(b, v[0]);
    if constexpr (T == 3 || T == 7) { wr16(b, v[0]); wr16(b + 2, v[1]); }
    if constexpr (T == 10) {
        wr16(b + 80, v[0]); wr16(b + 82, v[1]);
#pragma unroll
        for (int j = 0; j < 16; ++j) b[j] = (uint8_t)((v[2 + j] & 15) | ((v[18 + j] & 15) << 4));
    }
    if constexpr (T == 11) {
        wr16(b + 108, v[0]);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int l = v[1 + j];
            if (j < 8) b[96 + j] |= l & 15; else b[96 + j - 8] |= (l & 15) << 4;
            b[104 + (j & 3)] |= ((l >> 4) & 3) << (2 * (j >> 2));
        }
    }
    if constexpr (T == 12 || T == 13) {
        wr16(b, v[0]); wr16(b + 2, v[1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            b[4 + j] = (uint8_t)(v[2 + j] | ((v[6 + j] >> 4) << 6));
            b[8 + j] = (uint8_t)(v[10 + j] | ((v[14 + j] >> 4) << 6));
            b[12 + j] = (uint8_t)((v[6 + j] & 15) | ((v[14 + j] & 15) << 4));
        }
    }
    if constexpr (T == 14) {
        wr16(b + 208, v[0]);
#pragma unroll
        for (int j = 0; j < 16; ++j) b[192 + j] = (uint8_t)v[1 + j];
    }
    if constexpr (T == 23) {
        wr16(b, v[0]);
        int sh = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            const int ls = v[1 + ib];
            b[4 + ib / 2] |= (ls & 15) << (4 * (ib % 2));
            sh |= ((ls >> 4) & 3) << (2 * ib);
        }
        wr16(b + 2, sh);
    }
    // grid types: the scale bits share bytes with grid indices and signs, so they are OR-ed in
    if constexpr (T == 16 || T == 18) {
        wr16(b, v[0]);
#pragma unroll
        for (int j = 0; j < 8; ++j) b[(T == 16 ? 2 + 8 * j + 7 : 66 + 4 * j + 3)] |= (v[1 + j] & 15) << 4;
    }
    if constexpr (T == 17 || T == 22 || T == 21) {
        constexpr int O = T == 17 ? 66 : T == 22 ? 74 : 106, NS = T == 21 ? 8 : 16;
        wr16(b, v[0]);
#pragma unroll
        for (int j = 0; j < NS; ++j) b[O + j / 2] |= (v[1 + j] & 15) << (4 * (j % 2));
    }
    if constexpr (T == 19) {
        wr16(b, v[0]);
#pragma unroll
        for (int j = 0; j < 8; ++j) b[34 + 2 * j + 1] |= (v[1 + j] & 15) << 4;
    }
    if constexpr (T == 29) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int sv = (v[1 + j] & 7) << (3 * (j & 3));
            b[48 + 2 * (j >> 2)] |= sv & 255;
            b[49 + 2 * (j >> 2)] |= sv >> 8;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) b[49 + 2 * i] |= ((v[0] >> (4 * i)) & 15) << 4;
    }
}

// prediction of field k, given F's fp16 fields t0 (and t1): model 2 rescales the sub-scales
// (K-quants: and sub-mins) so that sub-scale x super-scale stays the predicted block's
template <int T>
__device__ __forceinline__ int fpred(int mv, const uint8_t* pb, int k, int t0, int t1) {
    const int pr = get_field<T>(pb, k);
    if constexpr (GRIDT<T>) {
        // the sub-scale rescaled so that d (2 ls + 1) stays the prediction's; IQ1_S keeps its shift bit
        if (mv < 2 || k < 1) return pr;
        const float tv = h2f((uint32_t)t0), pv = h2f((uint32_t)get_field<T>(pb, 0));
        if (tv == 0.f || !isfinite(tv) || !isfinite(pv)) return pr;
        constexpr float hi = (T == 19 || T == 29) ? 7.f : 15.f;
        const int ls = T == 19 ? (pr & 7) : pr;
        const float v = rintf(((((float)(2 * ls + 1) * pv) / tv) - 1.f) * 0.5f);
        const int q = (int)fminf(fmaxf(v, 0.f), hi);
        return T == 19 ? ((pr & 8) | q) : q;
    }
    constexpr bool two = T == 10 || T == 12 || T == 13;
    constexpr bool rescaled = two || T == 11 || T == 14 || T == 23;
    if (mv < 2 || !rescaled || k < (two ? 2 : 1)) return pr;
    const int ref = (two && k >= (T == 10 ? 18 : 10)) ? 1 : 0;
    const float tv = h2f((uint32_t)(ref ? t1 : t0)), pv = h2f((uint32_t)get_field<T>(pb, ref));
    if (tv == 0.f || !isfinite(tv) || !isfinite(pv)) return pr;
    if constexpr (T == 11 || T == 23) {
        const float v = rintf(((float)(pr - 32) * pv) / tv);
        return (int)fminf(fmaxf(v, -32.f), 31.f) + 32;
    } else {
        const float v = rintf(((float)pr * pv) / tv);
        if constexpr (T == 14) return (int)fminf(fmaxf(v, -128.f), 127.f);
        else return (int)fminf(fmaxf(v, 0.f), T == 10 ? 15.f : 63.f);
    }
}

// value = a * code + c of weight w (IQ4: a * KV[code])
template <int T>
__device__ __forceinline__ void wscale(const uint8_t* b, int w, float& a, float& c) {
    c = 0.f;
    if constexpr (T == 2) { a = h2f(rd16(b)); c = -8.f * a; }
    if constexpr (T == 3 || T == 7) { a = h2f(rd16(b)); c = h2f(rd16(b + 2)); }
    if constexpr (T == 6) { a = h2f(rd16(b)); c = -16.f * a; }
    if constexpr (T == 8 || T == 20) a = h2f(rd16(b));
    if constexpr (T == 42) { a = h2f(rd16(b)); c = -a; }
    if constexpr (T == 10) {
        const int n = w >> 7, r = w & 127, j = r >> 5;
        const int sc = b[8 * n + 2 * j + ((r & 31) >= 16)];
        a = h2f(rd16(b + 80)) * (float)(sc & 15);
        c = -(h2f(rd16(b + 82)) * (float)(sc >> 4));
    }
    if constexpr (T == 11) {
        const int n = w >> 7, r = w & 127, j = r >> 5;
        const int s = q3k_scale(b + 96, 8 * n + 2 * j + ((r & 31) >= 16));
        a = h2f(rd16(b + 108)) * (float)(s - 32);
        c = -4.f * a;
    }
    if constexpr (T == 12 || T == 13) {
        int sc, m;
        k4_scale_min(w >> 5, b + 4, sc, m);
        a = h2f(rd16(b)) * (float)sc;
        c = -(h2f(rd16(b + 2)) * (float)m);
    }
    if constexpr (T == 14) {
        const int n = w >> 7, r = w & 127, g = r >> 5, l = r & 31;
        a = h2f(rd16(b + 208)) * (float)s8(b[192 + 8 * n + (l >> 4) + 2 * g]);
        c = -32.f * a;
    }
    if constexpr (T == 23) {
        const int ib = w >> 5, sh = (int)rd16(b + 2);
        const int ls = ((b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        a = h2f(rd16(b)) * (float)(ls - 32);
    }
}

// seed types besides the float ones: no seed (the tensor's per-column RMS is the uncertainty, the
// value 0), and an explicit (value, uncertainty) pair of float32 per weight
constexpr int SEED_COLRMS = 98, SEED_EXPLICIT = 99;
// the uncertainty context's offset: 8, or 3 when the seed is only the column RMS
constexpr int HBOFF = 8, HBOFF_COL = 3;

// a quantized seed's value of weight w of its block and half its code's step
template <int S>
__device__ __forceinline__ void quant_seed(const uint8_t* blk, int w, float& x, float& h) {
    float a, c;
    wscale<S>(blk, w, a, c);
    const int q = get_code<S>(blk, w);
    if constexpr (NONLIN<S>) {
        x = a * KV[q];
        const float g = q < 15 ? KV[q + 1] - KV[q] : KV[15] - KV[14];
        h = fabsf(a) * (0.5f * g);
    } else {
        x = a * (float)q + c;
        h = fabsf(a) * 0.5f;
    }
}
template <int S>
__device__ __forceinline__ void quant_seed_at(const uint8_t* sb, int64_t gw, float& x, float& h) {
    quant_seed<S>(sb + (gw / Ty<S>::QK) * Ty<S>::BS, (int)(gw % Ty<S>::QK), x, h);
}

// seed value of global weight gw and its half uncertainty (qr.py seed_val): F32 (0), F16 (1), BF16 (30),
// a quantized tensor of a QR type without a grid, the column RMS (98), an explicit pair (99)
__device__ __forceinline__ void seed_val_any(int st, const uint8_t* sb, int64_t gw, int cols, float& x, float& h) {
    h = 0.f;
    switch (st) {
        case SEED_COLRMS: x = 0.f; h = reinterpret_cast<const float*>(sb)[gw % cols]; return;
        case SEED_EXPLICIT: x = reinterpret_cast<const float*>(sb)[2 * gw]; h = reinterpret_cast<const float*>(sb)[2 * gw + 1]; return;
        case 2: quant_seed_at<2>(sb, gw, x, h); return;
        case 3: quant_seed_at<3>(sb, gw, x, h); return;
        case 6: quant_seed_at<6>(sb, gw, x, h); return;
        case 7: quant_seed_at<7>(sb, gw, x, h); return;
        case 8: quant_seed_at<8>(sb, gw, x, h); return;
        case 10: quant_seed_at<10>(sb, gw, x, h); return;
        case 11: quant_seed_at<11>(sb, gw, x, h); return;
        case 12: quant_seed_at<12>(sb, gw, x, h); return;
        case 13: quant_seed_at<13>(sb, gw, x, h); return;
        case 14: quant_seed_at<14>(sb, gw, x, h); return;
        case 20: quant_seed_at<20>(sb, gw, x, h); return;
        case 23: quant_seed_at<23>(sb, gw, x, h); return;
        case 42: quant_seed_at<42>(sb, gw, x, h); return;
    }
    x = 0.f;
}
__device__ __forceinline__ void seed_val(int st, const uint8_t* sb, int64_t gw, int cols, float& x, float& h) {
    h = 0.f;
    if (st == 30) x = __uint_as_float((uint32_t)(sb[2 * gw] | (sb[2 * gw + 1] << 8)) << 16);
    else if (st == 0) x = reinterpret_cast<const float*>(sb)[gw];
    else if (st == 1) x = h2f((uint32_t)(sb[2 * gw] | (sb[2 * gw + 1] << 8)));
    else seed_val_any(st, sb, gw, cols, x, h);
}

// position of a weight's column in its row: the first 256 columns, then 7 parts
__device__ __forceinline__ int pos8(int64_t col, int cols) {
    return cols <= 0 || col < 256 ? 0 : 1 + (int)min((int64_t)6, col * 7 / cols);
}

__device__ __forceinline__ int hboff_of(const TM& m) { return m.seed_type == SEED_COLRMS ? HBOFF_COL : HBOFF; }

// predicted code r, mirror sign s and context of weight w from F's own scales (a, c)
template <int T>
__device__ __forceinline__ void predict(float a, float c, const uint8_t* pb, int w, float x, float h, int mv, int p8,
                                        int hboff, int& r, int& s, int& ctx) {
    float u, hu;
    if constexpr (NONLIN<T>) {
        const float t = x / a;
        int i = 0;
        while (i < 14 && t >= KV[i + 1]) i++;
        const float g = KV[i + 1] - KV[i];
        u = (float)i + (t - KV[i]) / g;
        hu = h / (fabsf(a) * g);
    } else {
        u = (x - c) / a;
        hu = h / fabsf(a);
    }
    if (!isfinite(u) || !isfinite(hu)) {          // zero scale: the predicted block's code
        r = get_code<T>(pb, w); s = 1; ctx = NSB_MAX + 63;
        return;
    }
    const float ru = rintf(u), fr = u - ru;
    r = (int)fmaxf(fminf(ru, (float)Ty<T>::QMAX), (float)Ty<T>::QMIN);
    s = fr >= 0.f ? 1 : -1;
    int mb = min(7, (int)(fabsf(fr) * 16.f));
    if (hboff == HBOFF_COL) {                     // no seed: r is the zero point; its place in the range
        s = 1;
        mb = min(7, max(0, (r - Ty<T>::QMIN) * 8 / (Ty<T>::QMAX - Ty<T>::QMIN + 1)));
    }
    int hb = 0;
    if (hu > 0.f) hb = max(1, min(7, ilogbf(hu) + hboff));
    ctx = NSB_MAX + hb * 8 + mb;
    if (mv >= 2 && hu == 0.f && hboff != HBOFF_COL) ctx = CODE2 + p8 * 16 + min(15, (int)(fabsf(fr) * 32.f));
}

}  // namespace qr
}  // namespace spa
