// K-quant super-block quantizers (256 weights): Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, imatrix (`_impl`)
// and NULL-imatrix (`_ref`) paths.
//
// Mapping: a group of G lanes per super-block, one lane per sub-block (G = 8 sub-blocks of 32 for
// Q4_K/Q5_K, G = 16 sub-blocks of 16 for Q2_K/Q3_K/Q6_K); a 256-lane workgroup handles 256/G
// consecutive super-blocks. The per-sub-block searches (the bulk of the work) run in parallel; with
// an imatrix the super-block's own searches over its G sub-block results run once, one lane per
// task (the scales, the mins) in the workgroup's first wave, while the other waves wait.
// The super-block sum of squares must be one left-to-right float sum over 256 terms: lane g adds
// its terms to the running sum it receives from lane g-1 (a shuffle per hand-off), so the order is
// the reference's. Sub-block results reach every lane of the group by shuffles; each lane repeats
// the small super-block level searches (identical inputs, identical result), requantizes its own
// sub-block, and parks its level values in LDS. Lane 0 of the group then packs the block bytes
// into an LDS tile that the workgroup stores with coalesced dword writes.
#include "common.h"
#include "launch.h"
#include "search.h"

namespace spa {
namespace {

constexpr int WG = 256;

struct KHeader {
    uint32_t d, dmin;          // fp16 bits
    uint32_t sc[16];           // scale bytes (as many as the type has)
    bool zero;                 // Q6_K all-zero super-block
};

// The super-block's sum of x*x over all 256 weights, left to right, computed across the group.
template <int G, int SUB>
__device__ __forceinline__ float group_sumsq(const float (&x)[SUB], int sub) {
    float sq[SUB];
#pragma unroll
    for (int i = 0; i < SUB; ++i) sq[i] = x[i] * x[i];
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (sub == g) {
#pragma unroll
            for (int i = 0; i < SUB; ++i) s += sq[i];
        }
        s = __shfl(s, g, G);
    }
    return s;
}

template <int G>
__device__ __forceinline__ void group_gather(float v, float (&all)[G]) {
#pragma unroll
    for (int k = 0; k < G; ++k) all[k] = __shfl(v, k, G);
}

template <int SUB>
__device__ __forceinline__ void park_levels(uint8_t* lt, const int (&L)[SUB]) {
    uint32_t* p = reinterpret_cast<uint32_t*>(lt);
#pragma unroll
    for (int i = 0; i < SUB; i += 4)
        p[i / 4] = (uint32_t)(L[i] & 0xff) | ((uint32_t)(L[i + 1] & 0xff) << 8) | ((uint32_t)(L[i + 2] & 0xff) << 16) |
                   ((uint32_t)(L[i + 3] & 0xff) << 24);
}

// get_scale_min_k4 -- ggml-quants.c:880-887 (j is a compile-time index after unrolling)
__device__ __forceinline__ uint32_t scale_min_k4(int j, const uint32_t (&q)[16]) {
    uint32_t d, m;
    if (j < 4) {
        d = q[j] & 63; m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
    return (d & 0xff) | ((m & 0xff) << 8);
}

// 6-bit scale/min packing of Q4_K/Q5_K (ggml-quants.c:1491-1501, :1590-1601).
__device__ __forceinline__ void pack_k4_scales(const int (&Ls)[8], const int (&Lm)[8], uint32_t (&sc)[16]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) sc[j] = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t ls = (uint32_t)Ls[j] & 0xff, lm = (uint32_t)Lm[j] & 0xff;
        if (j < 4) {
            sc[j] = ls;
            sc[j + 4] = lm;
        } else {
            sc[j + 4] = ((ls & 0xF) | ((lm & 0xF) << 4)) & 0xff;
            sc[j - 4] = (sc[j - 4] | ((ls >> 4) << 6)) & 0xff;
            sc[j - 0] = (sc[j - 0] | ((lm >> 4) << 6)) & 0xff;
        }
    }
}

// ---------------------------------------------------------------- Q4_K / Q5_K (G = 8, SUB = 32)

template <int NMAX>
struct Q45K {
    static constexpr int G = 8, SUB = 32;
    // quantize_row_q4_K_impl (ggml-quants.c:1554-1625) / quantize_row_q5_K_impl (:1759-1850), and the
    // NULL-imatrix rows quantize_row_q4_K_ref (:1458-1528) / quantize_row_q5_K_ref (:1645-1731).
    template <bool IMX>
    __device__ __forceinline__ static KHeader search(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB]) {
        KHeader h;
        h.zero = false;
        float scale, min;
        float w[SUB];
        if constexpr (IMX) {
            const float sum_x2 = group_sumsq<G, SUB>(x, sub);
            const float sigma2 = 2 * sum_x2 / 256;
#pragma unroll
            for (int l = 0; l < SUB; ++l) w[l] = qw[l] * sqrtf(sigma2 + x[l] * x[l]);
            float sumw = 0;
#pragma unroll
            for (int l = 0; l < SUB; ++l) sumw += w[l];
            scale = make_qkx3_quants<SUB, NMAX>(x, w, L, min, -0.9f, 0.05f, 36);
            float scales[G], mins[G], sw[G];
            group_gather<G>(scale, scales);
            group_gather<G>(min, mins);
            group_gather<G>(sumw, sw);
            int Ls[G], Lm[G];
            const float d_block = make_qp_quants<G>(63, scales, Ls, sw);
            const float m_block = make_qp_quants<G>(63, mins, Lm, sw);
            if (NMAX == 31) {   // Q5_K clamps the (uint8) levels to 63 (ggml-quants.c:1798-1799)
#pragma unroll
                for (int j = 0; j < G; ++j) { Ls[j] = tmin(63, Ls[j] & 0xff); Lm[j] = tmin(63, Lm[j] & 0xff); }
            }
            pack_k4_scales(Ls, Lm, h.sc);
            h.d = f32_to_f16(d_block);
            h.dmin = f32_to_f16(m_block);
        } else {
            float sum_x2 = 0;
#pragma unroll
            for (int l = 0; l < SUB; ++l) sum_x2 += x[l] * x[l];
            const float av_x = sqrtf(sum_x2 / 32);
#pragma unroll
            for (int l = 0; l < SUB; ++l) w[l] = av_x + fabsf(x[l]);
            if (NMAX == 15)
                scale = make_qkx2_quants<SUB, NMAX, false>(x, w, L, min, -1.f, 0.1f, 20);
            else
                scale = make_qkx2_quants<SUB, NMAX, false>(x, w, L, min, -0.5f, 0.1f, 15);
            float scales[G], mins[G];
            group_gather<G>(scale, scales);
            group_gather<G>(min, mins);
            float max_scale = 0, max_min = 0;
#pragma unroll
            for (int j = 0; j < G; ++j) {
                if (scales[j] > max_scale) max_scale = scales[j];
                if (mins[j] > max_min) max_min = mins[j];
            }
            const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
            const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
            int Ls[G], Lm[G];
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const uint32_t ls = (uint32_t)nearest_int(inv_scale * scales[j]) & 0xff;
                const uint32_t lm = (uint32_t)nearest_int(inv_min * mins[j]) & 0xff;
                Ls[j] = (int)tmin(63u, ls);
                Lm[j] = (int)tmin(63u, lm);
            }
            pack_k4_scales(Ls, Lm, h.sc);
            h.d = f32_to_f16(max_scale / 63.f);
            h.dmin = f32_to_f16(max_min / 63.f);
        }
        return h;
    }
    // imatrix path split for the kernel's block-level phase: the sub-block search (every lane) ...
    static constexpr int NT = 2;
    __device__ __forceinline__ static void sub_imx(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB], float& a, float& b,
                                                   float& wsum) {
        const float sum_x2 = group_sumsq<G, SUB>(x, sub);
        const float sigma2 = 2 * sum_x2 / 256;
        float w[SUB];
#pragma unroll
        for (int l = 0; l < SUB; ++l) w[l] = qw[l] * sqrtf(sigma2 + x[l] * x[l]);
        float sumw = 0;
#pragma unroll
        for (int l = 0; l < SUB; ++l) sumw += w[l];
        float min;
        a = make_qkx3_quants<SUB, NMAX>(x, w, L, min, -0.9f, 0.05f, 36);
        b = min;
        wsum = sumw;
    }
    // ... the super-block's scales (task 0) or mins (task 1) quantized (one lane each) ...
    __device__ __forceinline__ static void task(int, const float (&v)[G], const float (&sw)[G], uint32_t& f16, uint8_t (&lv)[G]) {
        int Lq[G];
        f16 = f32_to_f16(make_qp_quants<G>(63, v, Lq, sw));
#pragma unroll
        for (int j = 0; j < G; ++j) lv[j] = (uint8_t)(NMAX == 31 ? tmin(63, Lq[j] & 0xff) : (Lq[j] & 0xff));
    }
    // ... and the header from the two
    __device__ __forceinline__ static KHeader assemble(const uint32_t* f16, const uint8_t (*lv)[G]) {
        KHeader h;
        h.zero = false;
        int Ls[G], Lm[G];
#pragma unroll
        for (int j = 0; j < G; ++j) { Ls[j] = lv[0][j]; Lm[j] = lv[1][j]; }
        pack_k4_scales(Ls, Lm, h.sc);
        h.d = f16[0];
        h.dmin = f16[1];
        return h;
    }
    // decoded (scale, min) levels of sub-block j, as get_scale_min_k4 reads them back
    __device__ __forceinline__ static uint32_t info(const KHeader& h, int j) { return scale_min_k4(j, h.sc); }
    // requantize this sub-block with the stored scales (ggml-quants.c:1607-1616)
    __device__ __forceinline__ static void requant(const float (&x)[SUB], const KHeader& h, uint32_t inf, int (&L)[SUB]) {
        const float d = f16_to_f32(h.d) * (float)(inf & 0xff);
        if (d != 0.f) {
            const float dm = f16_to_f32(h.dmin) * (float)(inf >> 8);
#pragma unroll
            for (int ii = 0; ii < SUB; ++ii) {
                const int l = nearest_int((x[ii] + dm) / d);
                L[ii] = tmax(0, tmin(NMAX, l));
            }
        }
    }
    __device__ __forceinline__ static void pack(const KHeader& h, const uint8_t* L, TileOut o) {
        o.put16(0, h.d);
        o.put16(2, h.dmin);
#pragma unroll
        for (int j = 0; j < 12; j += 2) o.put2(4 + j, h.sc[j], h.sc[j + 1]);
        if (NMAX == 15) {   // Q4_K: qs[128] at 16
            for (int j = 0; j < 256; j += 64)
                for (int l = 0; l < 32; l += 2)
                    o.put2(16 + j / 2 + l, L[j + l] | (L[j + l + 32] << 4), L[j + l + 1] | (L[j + l + 33] << 4));
        } else {            // Q5_K: qh[32] at 16, qs[128] at 48 (ggml-quants.c:1711-1729)
            for (int j = 0; j < 32; j += 2) {
                uint32_t qh[2];
                for (int k = 0; k < 2; ++k) {
                    uint32_t v = 0;
                    for (int n = 0; n < 4; ++n)
                        v |= ((L[64 * n + j + k] > 15 ? 1u : 0u) << (2 * n)) | ((L[64 * n + j + k + 32] > 15 ? 2u : 0u) << (2 * n));
                    qh[k] = v;
                }
                o.put2(16 + j, qh[0], qh[1]);
            }
            for (int n = 0; n < 256; n += 64)
                for (int j = 0; j < 32; j += 2) {
                    uint32_t q[2];
                    for (int k = 0; k < 2; ++k) {
                        const uint32_t l1 = L[n + j + k], l2 = L[n + j + k + 32];
                        q[k] = ((l1 > 15 ? l1 - 16 : l1) | ((l2 > 15 ? l2 - 16 : l2) << 4)) & 0xff;
                    }
                    o.put2(48 + n / 2 + j, q[0], q[1]);
                }
        }
    }
};

// ---------------------------------------------------------------- Q2_K (G = 16, SUB = 16)

struct Q2K {
    static constexpr int G = 16, SUB = 16, BS = 84;
    // quantize_row_q2_K_impl (ggml-quants.c:1150-1210) and quantize_row_q2_K_ref (:891-960).
    template <bool IMX>
    __device__ __forceinline__ static KHeader search(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB]) {
        KHeader h;
        h.zero = false;
        float dmf, mmf;
        if constexpr (IMX) {
            const float sumx2 = group_sumsq<G, SUB>(x, sub);
            const float sigma2 = sumx2 / 256;
            float w[SUB];
#pragma unroll
            for (int l = 0; l < SUB; ++l) w[l] = qw[l] * sqrtf(sigma2 + x[l] * x[l]);
            float sumw = 0;
#pragma unroll
            for (int l = 0; l < SUB; ++l) sumw += w[l];
            float min;
            const float scale = make_qkx3_quants<SUB, 3>(x, w, L, min, -0.9f, 0.05f, 36);
            float scales[G], mins[G], sw[G];
            group_gather<G>(scale, scales);
            group_gather<G>(min, mins);
            group_gather<G>(sumw, sw);
            int Ls[G], Lm[G];
            const float dm = make_qp_quants<G>(15, scales, Ls, sw);
            const float mm = make_qp_quants<G>(15, mins, Lm, sw);
            h.d = f32_to_f16(dm);
            h.dmin = f32_to_f16(mm);
            dmf = f16_to_f32(h.d);
            mmf = f16_to_f32(h.dmin);
#pragma unroll
            for (int j = 0; j < G; ++j) h.sc[j] = ((uint32_t)Ls[j] | ((uint32_t)Lm[j] << 4)) & 0xff;
        } else {
            float w[SUB];
#pragma unroll
            for (int l = 0; l < SUB; ++l) w[l] = fabsf(x[l]);
            float min;
            const float scale = make_qkx2_quants<SUB, 3, true>(x, w, L, min, -0.5f, 0.1f, 15);
            float scales[G], mins[G];
            group_gather<G>(scale, scales);
            group_gather<G>(min, mins);
            float max_scale = 0, max_min = 0;
#pragma unroll
            for (int j = 0; j < G; ++j) {
                if (scales[j] > max_scale) max_scale = scales[j];
                if (mins[j] > max_min) max_min = mins[j];
            }
            if (max_scale > 0) {
                const float iscale = 15.f / max_scale;
#pragma unroll
                for (int j = 0; j < G; ++j) h.sc[j] = (uint32_t)nearest_int(iscale * scales[j]) & 0xff;
                h.d = f32_to_f16(max_scale / 15.f);
            } else {
#pragma unroll
                for (int j = 0; j < G; ++j) h.sc[j] = 0;
                h.d = f32_to_f16(0.f);
            }
            if (max_min > 0) {
                const float iscale = 15.f / max_min;
#pragma unroll
                for (int j = 0; j < G; ++j) h.sc[j] = (h.sc[j] | ((uint32_t)nearest_int(iscale * mins[j]) << 4)) & 0xff;
                h.dmin = f32_to_f16(max_min / 15.f);
            } else {
                h.dmin = f32_to_f16(0.f);
            }
            dmf = f16_to_f32(h.d);
            mmf = f16_to_f32(h.dmin);
        }
        (void)dmf; (void)mmf;
        return h;
    }
    // imatrix path split for the kernel's block-level phase (see Q45K)
    static constexpr int NT = 2;
    __device__ __forceinline__ static void sub_imx(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB], float& a, float& b,
                                                   float& wsum) {
        const float sumx2 = group_sumsq<G, SUB>(x, sub);
        const float sigma2 = sumx2 / 256;
        float w[SUB];
#pragma unroll
        for (int l = 0; l < SUB; ++l) w[l] = qw[l] * sqrtf(sigma2 + x[l] * x[l]);
        float sumw = 0;
#pragma unroll
        for (int l = 0; l < SUB; ++l) sumw += w[l];
        float min;
        a = make_qkx3_quants<SUB, 3>(x, w, L, min, -0.9f, 0.05f, 36);
        b = min;
        wsum = sumw;
    }
    __device__ __forceinline__ static void task(int, const float (&v)[G], const float (&sw)[G], uint32_t& f16, uint8_t (&lv)[G]) {
        int Lq[G];
        f16 = f32_to_f16(make_qp_quants<G>(15, v, Lq, sw));
#pragma unroll
        for (int j = 0; j < G; ++j) lv[j] = (uint8_t)(Lq[j] & 0xff);
    }
    __device__ __forceinline__ static KHeader assemble(const uint32_t* f16, const uint8_t (*lv)[G]) {
        KHeader h;
        h.zero = false;
        h.d = f16[0];
        h.dmin = f16[1];
#pragma unroll
        for (int j = 0; j < G; ++j) h.sc[j] = ((uint32_t)lv[0][j] | ((uint32_t)lv[1][j] << 4)) & 0xff;
        return h;
    }
    __device__ __forceinline__ static uint32_t info(const KHeader& h, int j) { return h.sc[j]; }
    __device__ __forceinline__ static void requant(const float (&x)[SUB], const KHeader& h, uint32_t scj, int (&L)[SUB]) {
        const float d = f16_to_f32(h.d) * (float)(scj & 0xF);
        if (d != 0.f) {
            const float m = f16_to_f32(h.dmin) * (float)(scj >> 4);
#pragma unroll
            for (int ii = 0; ii < SUB; ++ii) {
                const int l = nearest_int((x[ii] + m) / d);
                L[ii] = tmax(0, tmin(3, l));
            }
        }
    }
    __device__ __forceinline__ static void pack(const KHeader& h, const uint8_t* L, TileOut o) {
#pragma unroll
        for (int j = 0; j < 16; j += 2) o.put2(j, h.sc[j], h.sc[j + 1]);
        for (int j = 0; j < 256; j += 128)
            for (int l = 0; l < 32; l += 2) {
                uint32_t q[2];
                for (int k = 0; k < 2; ++k)
                    q[k] = (L[j + l + k] | (L[j + l + k + 32] << 2) | (L[j + l + k + 64] << 4) | (L[j + l + k + 96] << 6)) & 0xff;
                o.put2(16 + j / 4 + l, q[0], q[1]);
            }
        o.put16(80, h.d);
        o.put16(82, h.dmin);
    }
};

// ---------------------------------------------------------------- Q3_K (G = 16, SUB = 16)

// make_q3_quants(n = 16, nmax = 4, do_rmse = true) -- ggml-quants.c:697-754 (Q3_K reference path).
__device__ __forceinline__ float make_q3_quants16(const float (&x)[16], int (&L)[16]) {
    constexpr int nmax = 4;
    float max = 0, amax = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
#pragma unroll
        for (int i = 0; i < 16; ++i) L[i] = 0;
        return 0.f;
    }
    const float iscale = (float)(-nmax) / max;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = tmax(-nmax, tmin(nmax - 1, l));
        L[i] = l;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    for (int itry = 0; itry < 5; ++itry) {
        int n_changed = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float w = x[i] * x[i];
            float slx = sumlx - w * x[i] * (float)L[i];
            if (slx > 0) {
                float sl2 = suml2 - w * (float)L[i] * (float)L[i];
                int new_l = nearest_int(x[i] * sl2 / slx);
                new_l = tmax(-nmax, tmin(nmax - 1, new_l));
                if (new_l != L[i]) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = new_l; sumlx = slx; suml2 = sl2;
                        ++n_changed;
                    }
                }
            }
        }
        if (!n_changed) break;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) L[i] += nmax;
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

struct Q3K {
    static constexpr int G = 16, SUB = 16, BS = 110;
    // quantize_row_q3_K_impl (ggml-quants.c:1356-1438) and quantize_row_q3_K_ref (:1230-1305).
    template <bool IMX>
    __device__ __forceinline__ static KHeader search(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB]) {
        KHeader h;
        h.zero = false;
#pragma unroll
        for (int j = 0; j < 16; ++j) h.sc[j] = 0;
        if constexpr (IMX) {
            const float sumx2 = group_sumsq<G, SUB>(x, sub);
            const float sigma2 = 2 * sumx2 / 256;
            float w[SUB];
#pragma unroll
            for (int l = 0; l < SUB; ++l) w[l] = qw[l] * sqrtf(sigma2 + x[l] * x[l]);
            float sumw = 0;
#pragma unroll
            for (int l = 0; l < SUB; ++l) sumw += w[l];
            const float scale = make_qx_quants<SUB, true>(4, x, w, L);
            float scales[G], sw[G];
            group_gather<G>(scale, scales);
            group_gather<G>(sumw, sw);
            int Ls[G];
            const float d_block = make_qx_quants<G, true>(32, scales, sw, Ls);
#pragma unroll
            for (int j = 0; j < G; ++j) {
                int l = Ls[j];
                if (j < 8) h.sc[j] = (uint32_t)(l & 0xF);
                else h.sc[j - 8] = (h.sc[j - 8] | ((uint32_t)(l & 0xF) << 4)) & 0xff;
                l >>= 4;
                h.sc[j % 4 + 8] = (h.sc[j % 4 + 8] | ((uint32_t)l << (2 * (j / 4)))) & 0xff;
            }
            h.d = f32_to_f16(d_block);
        } else {
            const float scale = make_q3_quants16(x, L);
            float scales[G];
            group_gather<G>(scale, scales);
            float max_scale = 0, amax = 0;
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float s = fabsf(scales[j]);
                if (s > amax) { amax = s; max_scale = scales[j]; }
            }
            if (max_scale != 0.f) {
                const float iscale = -32.f / max_scale;
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    int l = (int)(int8_t)nearest_int(iscale * scales[j]);
                    l = tmax(-32, tmin(31, l)) + 32;
                    if (j < 8) h.sc[j] = (uint32_t)(l & 0xF);
                    else h.sc[j - 8] = (h.sc[j - 8] | ((uint32_t)(l & 0xF) << 4)) & 0xff;
                    l = (int)(int8_t)l >> 4;
                    h.sc[j % 4 + 8] = (h.sc[j % 4 + 8] | ((uint32_t)l << (2 * (j / 4)))) & 0xff;
                }
                h.d = f32_to_f16(1 / iscale);
            } else {
                h.d = f32_to_f16(0.f);
            }
        }
        return h;
    }
    // imatrix path split for the kernel's block-level phase (see Q45K): one task, the scales' quantization
    static constexpr int NT = 1;
    __device__ __forceinline__ static void sub_imx(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB], float& a, float& b,
                                                   float& wsum) {
        const float sumx2 = group_sumsq<G, SUB>(x, sub);
        const float sigma2 = 2 * sumx2 / 256;
        float w[SUB];
#pragma unroll
        for (int l = 0; l < SUB; ++l) w[l] = qw[l] * sqrtf(sigma2 + x[l] * x[l]);
        float sumw = 0;
#pragma unroll
        for (int l = 0; l < SUB; ++l) sumw += w[l];
        a = make_qx_quants<SUB, true>(4, x, w, L);
        b = 0.f;
        wsum = sumw;
    }
    __device__ __forceinline__ static void task(int, const float (&a)[G], const float (&sw)[G], uint32_t& f16, uint8_t (&lv)[G]) {
        int Ls[G];
        f16 = f32_to_f16(make_qx_quants<G, true>(32, a, sw, Ls));
#pragma unroll
        for (int j = 0; j < G; ++j) lv[j] = (uint8_t)Ls[j];
    }
    __device__ __forceinline__ static KHeader assemble(const uint32_t* f16, const uint8_t (*lv)[G]) {
        KHeader h;
        h.zero = false;
#pragma unroll
        for (int j = 0; j < 16; ++j) h.sc[j] = 0;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            int l = lv[0][j];
            if (j < 8) h.sc[j] = (uint32_t)(l & 0xF);
            else h.sc[j - 8] = (h.sc[j - 8] | ((uint32_t)(l & 0xF) << 4)) & 0xff;
            l >>= 4;
            h.sc[j % 4 + 8] = (h.sc[j % 4 + 8] | ((uint32_t)l << (2 * (j / 4)))) & 0xff;
        }
        h.d = f16[0];
        return h;
    }
    // the signed 6-bit scale of sub-block j as read back from the packed bytes (ggml-quants.c:1411-1413)
    __device__ __forceinline__ static uint32_t info(const KHeader& h, int j) {
        int sc = j < 8 ? (int)(h.sc[j] & 0xF) : (int)(h.sc[j - 8] >> 4);
        sc = (int)(int8_t)((sc | (int)(((h.sc[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32);
        return (uint32_t)sc;
    }
    __device__ __forceinline__ static void requant(const float (&x)[SUB], const KHeader& h, uint32_t inf, int (&L)[SUB]) {
        const float d = f16_to_f32(h.d) * (float)(int)inf;
        if (d != 0.f) {
#pragma unroll
            for (int ii = 0; ii < SUB; ++ii) {
                int l = nearest_int(x[ii] / d);
                l = tmax(-4, tmin(3, l));
                L[ii] = l + 4;
            }
        }
    }
    __device__ __forceinline__ static void pack(const KHeader& h, const uint8_t* L, TileOut o) {
        // hmask[32] at 0, qs[64] at 32, scales[12] at 96, d at 108 (ggml-quants.c:1410-1435). Levels are
        // 0..7: bit 2 goes to hmask (bit k of byte m for level 32k+m) and the low two bits to qs.
        for (int m = 0; m < 32; m += 2) {
            uint32_t hb[2];
            for (int k2 = 0; k2 < 2; ++k2) {
                uint32_t v = 0;
                for (int k = 0; k < 8; ++k) v |= (L[32 * k + m + k2] > 3 ? 1u : 0u) << k;
                hb[k2] = v;
            }
            o.put2(m, hb[0], hb[1]);
        }
        for (int j = 0; j < 256; j += 128)
            for (int l = 0; l < 32; l += 2) {
                uint32_t q[2];
                for (int k = 0; k < 2; ++k)
                    q[k] = ((L[j + l + k] & 3) | ((L[j + l + k + 32] & 3) << 2) | ((L[j + l + k + 64] & 3) << 4) |
                            ((L[j + l + k + 96] & 3) << 6)) & 0xff;
                o.put2(32 + j / 4 + l, q[0], q[1]);
            }
#pragma unroll
        for (int j = 0; j < 12; j += 2) o.put2(96 + j, h.sc[j], h.sc[j + 1]);
        o.put16(108, h.d);
    }
};

// ---------------------------------------------------------------- Q6_K (G = 16, SUB = 16)

struct Q6K {
    static constexpr int G = 16, SUB = 16, BS = 210;
    static constexpr int NT = 0;       // the block level is a max and a rounding: no split
    // quantize_row_q6_K_impl (ggml-quants.c:1971-2053) and quantize_row_q6_K_ref (:1870-1938): the
    // imatrix path weights by the raw imatrix, the NULL path by x*x.
    template <bool IMX>
    __device__ __forceinline__ static KHeader search(float (&x)[SUB], const float* qw, int sub, int (&L)[SUB]) {
        KHeader h;
        h.zero = false;
        float scale;
        if constexpr (IMX) {
            float w[SUB];
#pragma unroll
            for (int l = 0; l < SUB; ++l) w[l] = qw[l];
            scale = make_qx_quants<SUB, true>(32, x, w, L);
        } else {
            float w[SUB];
            scale = make_qx_quants<SUB, false>(32, x, w, L);
        }
        float scales[G];
        group_gather<G>(scale, scales);
        float max_scale = 0, max_abs_scale = 0;
#pragma unroll
        for (int ib = 0; ib < G; ++ib) {
            const float a = fabsf(scales[ib]);
            if (a > max_abs_scale) { max_abs_scale = a; max_scale = scales[ib]; }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            h.zero = true;
            h.d = 0;
            return h;
        }
        const float iscale = -128.f / max_scale;
        h.d = f32_to_f16(1 / iscale);
#pragma unroll
        for (int ib = 0; ib < G; ++ib) h.sc[ib] = (uint32_t)tmin(127, nearest_int(iscale * scales[ib])) & 0xff;
        return h;
    }
    __device__ __forceinline__ static uint32_t info(const KHeader& h, int j) { return h.zero ? 0u : h.sc[j]; }
    __device__ __forceinline__ static void requant(const float (&x)[SUB], const KHeader& h, uint32_t scj, int (&L)[SUB]) {
        if (h.zero) return;
        const float d = f16_to_f32(h.d) * (float)(int)(int8_t)scj;
        if (d != 0.f) {
#pragma unroll
            for (int ii = 0; ii < SUB; ++ii) {
                int l = nearest_int(x[ii] / d);
                l = tmax(-32, tmin(31, l));
                L[ii] = l + 32;
            }
        }
    }
    __device__ __forceinline__ static void pack(const KHeader& h, const uint8_t* L, TileOut o) {
        // ql[128] at 0, qh[64] at 128, scales[16] at 192, d at 208 (ggml-quants.c:1922-1935)
        if (h.zero) {
            for (int j = 0; j < 210; j += 2) o.put16(j, 0);
            return;
        }
        for (int j = 0; j < 256; j += 128) {
            for (int l = 0; l < 32; l += 2) {
                uint32_t a[2], b[2], c[2];
                for (int k = 0; k < 2; ++k) {
                    const uint32_t q1 = L[j + l + k + 0] & 0xF, q2 = L[j + l + k + 32] & 0xF;
                    const uint32_t q3 = L[j + l + k + 64] & 0xF, q4 = L[j + l + k + 96] & 0xF;
                    a[k] = (q1 | (q3 << 4)) & 0xff;
                    b[k] = (q2 | (q4 << 4)) & 0xff;
                    c[k] = ((L[j + l + k] >> 4) | ((L[j + l + k + 32] >> 4) << 2) | ((L[j + l + k + 64] >> 4) << 4) |
                            ((L[j + l + k + 96] >> 4) << 6)) & 0xff;
                }
                o.put2(j / 2 + l, a[0], a[1]);
                o.put2(j / 2 + l + 32, b[0], b[1]);
                o.put2(128 + j / 4 + l, c[0], c[1]);
            }
        }
#pragma unroll
        for (int j = 0; j < 16; j += 2) o.put2(192 + j, h.sc[j], h.sc[j + 1]);
        o.put16(208, h.d);
    }
};

struct Q4K : Q45K<15> { static constexpr int BS = 144; };
struct Q5K : Q45K<31> { static constexpr int BS = 176; };

template <class Op, bool IMX>
__global__ __launch_bounds__(WG) void k_kquant(const void* __restrict__ src, int kind, uint8_t* __restrict__ dst,
                                               int64_t nsb, int64_t sb_per_row, const float* __restrict__ imx) {
    constexpr int G = Op::G, SUB = Op::SUB, SBW = WG / G;
    __shared__ __align__(16) uint8_t ltile[SBW * 256];
    __shared__ __align__(16) uint16_t otile[SBW * Op::BS / 2];
    __shared__ uint32_t ginfo[SBW][G];
    const int lsb = threadIdx.x / G, sub = threadIdx.x % G;
    const int64_t sb0 = (int64_t)blockIdx.x * SBW;
    const int64_t sb = sb0 + lsb;
    const bool active = sb < nsb;
    const int64_t sbc = active ? sb : nsb - 1;      // lanes past the end recompute the last block
    float x[SUB];
    load_weights<SUB>(src, kind, sbc * 256 + sub * SUB, x);
    const float* qw = nullptr;
    if (IMX) {
        const int64_t row = sbc / sb_per_row;
        qw = imx + (sbc - row * sb_per_row) * 256 + sub * SUB;
    }
    int L[SUB];
    KHeader h;
    if constexpr (IMX && Op::NT > 0) {
        // The block-level searches (make_qp_quants / make_qx_quants over the G sub-block results) run
        // once per super-block, one lane per task, instead of in every lane of the group: lanes
        // publish their sub-block results, the first NT x SBW lanes of the workgroup run the tasks,
        // every lane assembles its header from the tasks' outputs.
        __shared__ float pa[SBW][G], pb[SBW][G], pw[SBW][G];
        __shared__ uint32_t tf[SBW][Op::NT];
        __shared__ uint8_t tl[SBW][Op::NT][G];
        Op::sub_imx(x, qw, sub, L, pa[lsb][sub], pb[lsb][sub], pw[lsb][sub]);
        __syncthreads();
        if (threadIdx.x < SBW * Op::NT) {
            const int tsb = threadIdx.x / Op::NT, which = threadIdx.x % Op::NT;
            const float* src = which ? pb[tsb] : pa[tsb];     // the task's values: scales or mins
            float v[G], w[G];
#pragma unroll
            for (int j = 0; j < G; ++j) { v[j] = src[j]; w[j] = pw[tsb][j]; }
            uint8_t lv[G];
            Op::task(which, v, w, tf[tsb][which], lv);
#pragma unroll
            for (int j = 0; j < G; ++j) tl[tsb][which][j] = lv[j];
        }
        __syncthreads();
        h = Op::assemble(tf[lsb], tl[lsb]);
    } else {
        h = Op::template search<IMX>(x, qw, sub, L);
    }
    // every lane of the group holds the same header; lane 0 publishes the per-sub-block decode
    if (sub == 0) {
#pragma unroll
        for (int k = 0; k < G; ++k) ginfo[lsb][k] = Op::info(h, k);
    }
    __syncthreads();
    Op::requant(x, h, ginfo[lsb][sub], L);
    park_levels<SUB>(ltile + lsb * 256 + sub * SUB, L);
    __syncthreads();
    if (active && sub == 0) Op::pack(h, ltile + lsb * 256, TileOut{otile + lsb * (Op::BS / 2)});
    __syncthreads();
    const int nb = (int)(nsb - sb0 < SBW ? nsb - sb0 : SBW);
    store_tile(otile, dst + sb0 * Op::BS, nb * Op::BS);
}

template <class Op>
int run(const QuantArgs& a) {
    const int64_t nsb = a.nrows * a.n_per_row / 256;
    if (nsb == 0) return 0;
    constexpr int SBW = WG / Op::G;
    const int64_t grid = (nsb + SBW - 1) / SBW;
    if (a.imatrix)
        hipLaunchKernelGGL((k_kquant<Op, true>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nsb, a.n_per_row / 256, a.imatrix);
    else
        hipLaunchKernelGGL((k_kquant<Op, false>), dim3((unsigned)grid), dim3(WG), 0, a.stream, a.src, a.src_kind,
                           (uint8_t*)a.dst, nsb, a.n_per_row / 256, a.imatrix);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

int launch_kquant(const QuantArgs& a) {
    switch (a.type) {
        case 10: return run<Q2K>(a);
        case 11: return run<Q3K>(a);
        case 12: return run<Q4K>(a);
        case 13: return run<Q5K>(a);
        case 14: return run<Q6K>(a);
        default: return fail(-2, "launch_kquant: type %d is not a K-quant", a.type);
    }
}

}  // namespace spa
