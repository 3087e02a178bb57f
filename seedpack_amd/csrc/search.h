// Lane-local scale/min searches of the K-quant and legacy quantizers.
//
// Each function keeps one (sub-)block in registers (N is a compile-time size, loops are fully
// unrolled) and follows the reference's operation order exactly: every sum is accumulated left to
// right, every product is parenthesised as the C expression parses, and ties follow the same strict
// comparisons. Arrays that the C code keeps as uint8_t/int8_t are truncated the same way.
#pragma once

#include "common.h"

namespace spa {

constexpr float GROUP_MAX_EPS = 1e-15f;   // ggml-quants.c:20

// make_qx_quants(n, nmax, x, L, rmse_type = 1, qw) -- ggml-quants.c:628-695.
// QW = true: w = qw[i]; QW = false (qw == NULL): w = x[i]*x[i].
// L[i] receives nmax + clamp(l, -nmax, nmax-1).
template <int N, bool QW>
__device__ __forceinline__ float make_qx_quants(int nmax, const float (&x)[N], const float (&qw)[N], int (&L)[N]) {
    float max = 0, amax = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
#pragma unroll
        for (int i = 0; i < N; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = (float)(-nmax) / max;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = tmax(-nmax, tmin(nmax - 1, l));
        const float w = QW ? qw[i] : x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    float best_iscale = iscale;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        const float isc = -((float)nmax + 0.1f * (float)is) / max;
        float slx = 0, sl2 = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int l = nearest_int(isc * x[i]);
            l = tmax(-nmax, tmin(nmax - 1, l));
            const float w = QW ? qw[i] : x[i] * x[i];
            slx += w * x[i] * (float)l;
            sl2 += w * (float)l * (float)l;
        }
        if (sl2 > 0 && slx * slx > best * sl2) {
            best_iscale = isc;
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    // L is a pure function of the winning iscale, so it is produced once here.
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = nearest_int(best_iscale * x[i]);
        L[i] = nmax + tmax(-nmax, tmin(nmax - 1, l));
    }
    return scale;
}

// make_qkx2_quants -- ggml-quants.c:799-878 (the NULL-imatrix K-quant paths).
template <int N, int NMAX, bool USE_MAD>
__device__ __forceinline__ float make_qkx2_quants(const float (&x)[N], const float (&w)[N], int (&L)[N], float& the_min,
                                                  float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
#pragma unroll
        for (int i = 0; i < N; ++i) L[i] = 0;
        the_min = -min;
        return 0.f;
    }
    float iscale = (float)NMAX / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = tmax(0, tmin(NMAX, l));
        float diff = scale * (float)L[i] + min - x[i];
        diff = USE_MAD ? fabsf(diff) : diff * diff;
        best_error += w[i] * diff;
    }
    if (nstep < 1) { the_min = -min; return scale; }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)NMAX) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        int La[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = tmax(0, tmin(NMAX, l));
            La[i] = l;
            sum_l += w[i] * (float)l;
            sum_l2 += w[i] * (float)l * (float)l;
            sum_xl += w[i] * (float)l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                float diff = this_scale * (float)La[i] + this_min - x[i];
                diff = USE_MAD ? fabsf(diff) : diff * diff;
                cur_error += w[i] * diff;
            }
            if (cur_error < best_error) {
#pragma unroll
                for (int i = 0; i < N; ++i) L[i] = La[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    the_min = -min;
    return scale;
}

// make_qkx3_quants with non-NULL weights and use_mad = false -- ggml-quants.c:993-1075 (every
// imatrix K-quant and Q4_1/Q5_1 call site passes weights and use_mad = false).
// Note the running `min`: a step that wins changes the offset used by every later step.
// The levels of a step are a pure function of (iscale, min), so only the winning pair is kept and
// L is produced once at the end. Inside the step loop, nearest_int(MIN(v, nmax)) for 0 < v <= nmax
// is computed as rintf(fminf(fmaxf(v, 0), nmax)): both round half to even and return the same integer
// (the magic-number form is exact for |v| < 2^22); v <= 0 and NaN give a zero level as in the C code
// (possibly -0.0, which changes nothing: every sum starts at +0.0 and adds non-negative terms or
// w*l*x products, and an IEEE sum from +0.0 is never -0.0, so each sum and each squared difference
// is the same number).
template <int N, int NMAX>
__device__ __forceinline__ float make_qkx3_quants(const float (&x)[N], const float (&w)[N], int (&L)[N], float& the_min,
                                                  float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (min > 0) min = 0;
    if (max <= min) {
#pragma unroll
        for (int i = 0; i < N; ++i) L[i] = 0;
        the_min = -min;
        return 0.f;
    }
    const float iscale0 = (float)NMAX / (max - min);
    float scale = 1 / iscale0;
    float best_mad = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int l = tmax(0, tmin(NMAX, nearest_int(iscale0 * (x[i] - min))));
        float diff = scale * (float)l + min - x[i];
        diff = diff * diff;
        best_mad += w[i] * diff;
    }
    const float min0 = min;
    float best_iscale = iscale0, best_min = min0;   // (iscale, min) that produced the kept levels
    bool from_step = false;
    // x - min for the running min, kept for 16-weight sub-blocks (recomputed only when a step wins and
    // moves the min); the 32-weight ones have no registers to spare for it (occupancy 3 -> 2)
    constexpr bool KEEP = N <= 16;
    float xm[KEEP ? N : 1];
    if constexpr (KEEP) {
#pragma unroll
        for (int i = 0; i < N; ++i) xm[i] = x[i] - min;
    }
    for (int is = 0; is <= nstep; ++is) {
        const float iscale = (rmin + rdelta * (float)is + (float)NMAX) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        float Lf[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float v = iscale * (KEEP ? xm[i] : x[i] - min);
            const float fl = rintf(fminf(fmaxf(v, 0.f), (float)NMAX));
            Lf[i] = fl;
            const float wl = w[i] * fl;
            sum_l += wl;
            sum_l2 += wl * fl;
            sum_xl += wl * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                float diff = this_scale * Lf[i] + this_min - x[i];
                diff = diff * diff;
                mad += w[i] * diff;
            }
            if (mad < best_mad) {
                best_iscale = iscale;
                best_min = min;
                from_step = true;
                best_mad = mad;
                scale = this_scale;
                min = this_min;
                if constexpr (KEEP) {
#pragma unroll
                    for (int i = 0; i < N; ++i) xm[i] = x[i] - min;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (from_step) {
            const float v = best_iscale * (x[i] - best_min);
            L[i] = v > 0.f ? (int)rintf(fminf(v, (float)NMAX)) : 0;
        } else {
            L[i] = tmax(0, tmin(NMAX, nearest_int(best_iscale * (x[i] - best_min))));
        }
    }
    the_min = -min;
    return scale;
}

// make_qp_quants -- ggml-quants.c:1077-1148. L is uint8_t in the reference; stores wrap mod 256.
template <int N>
__device__ __forceinline__ float make_qp_quants(int nmax, const float (&x)[N], int (&L)[N], const float (&qw)[N]) {
    float max = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) max = tmax(max, x[i]);
    if (max < GROUP_MAX_EPS) {
#pragma unroll
        for (int i = 0; i < N; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = (float)nmax / max;
#pragma unroll
    for (int i = 0; i < N; ++i) L[i] = nearest_int(iscale * x[i]) & 0xff;
    const float scale = 1 / iscale;
    float best_mse = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float diff = x[i] - scale * (float)L[i];
        best_mse += qw[i] * diff * diff;
    }
    for (int is = -4; is <= 4; ++is) {
        if (is == 0) continue;
        const float iscale_is = (0.1f * (float)is + (float)nmax) / max;
        const float scale_is = 1 / iscale_is;
        float mse = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int l = nearest_int(iscale_is * x[i]);
            l = tmin(nmax, l);
            const float diff = x[i] - scale_is * (float)l;
            mse += qw[i] * diff * diff;
        }
        if (mse < best_mse) {
            best_mse = mse;
            iscale = iscale_is;
        }
    }
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = tmin(nmax, l);
        L[i] = l & 0xff;
        const float fl = (float)l;   // the sums take the int level; only L wraps (x < 0 in IQ2_XXS)
        sumlx += qw[i] * x[i] * fl;
        suml2 += qw[i] * fl * fl;
    }
    for (int itry = 0; itry < 5; ++itry) {
        int n_changed = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float w = qw[i];
            const float fL = (float)L[i];
            float slx = sumlx - w * x[i] * fL;
            float sl2 = suml2 - w * fL * fL;
            if (slx > 0 && sl2 > 0) {
                int new_l = nearest_int(x[i] * sl2 / slx);
                new_l = tmin(nmax, new_l);
                if (new_l != L[i]) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (slx * slx * suml2 > sumlx * sumlx * sl2) {
                        L[i] = new_l & 0xff;
                        sumlx = slx;
                        suml2 = sl2;
                        ++n_changed;
                    }
                }
            }
        }
        if (!n_changed) break;
    }
    return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

}  // namespace spa
