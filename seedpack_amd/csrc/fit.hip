// Estimating what a quant was made from, when the repository does not hold it:
//
// * the importance-matrix fit (imxfit.py:30-63): a legacy quantizer's block scale is the weighted
//   least-squares fit of the block to its codes, so the block's residual x - v is weighted-orthogonal
//   to its codes l (and, with a kept minimum, to 1). k_conditions forms those conditions per weight,
//   normalised per block, laid out (block of columns, position, row) for the Gram sums;
// * the sibling estimate (siblings.py:51-77): the precision-weighted mean of the versions of a tensor
//   seen so far, x = sum(x_i / h_i^2) / sum(1 / h_i^2), h = sum(1 / h_i^2)^-1/2, with h_i half the
//   interval a version's code stands for.
//
// Every float operation is the reference's, one rounding per operation (no contraction).
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "launch.h"

namespace spa {
namespace {

__device__ __forceinline__ float h2f_at(const uint8_t* p) { return f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

// (cp.maximum semantics: NaN propagates)
__device__ __forceinline__ float max_nan(float a, float b) { return (a != a || a > b) ? a : b; }

// a lane per row (coalesced condition stores), blockIdx.y the block of columns
template <int QK, int BS, bool TWO>
__global__ __launch_bounds__(256) void k_conditions(const float* __restrict__ X, const uint8_t* __restrict__ F,
                                                    const float* __restrict__ V, const double* __restrict__ rowsq,
                                                    int64_t R, int64_t cols, float* __restrict__ e1, float* __restrict__ e2) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= R) return;
    const int64_t b = blockIdx.y, nb = cols / QK;
    const uint8_t* blk = F + (r * nb + b) * BS;
    const float d = h2f_at(blk), m = TWO ? h2f_at(blk + 2) : 0.f;
    const float dd = d == 0.f ? 1.f : d;
    const float a = (float)(rowsq[r] / (double)cols);
    const float* x = X + r * cols + b * QK;
    const float* v = V + r * cols + b * QK;
    float c1[QK], c2[QK];
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int i = 0; i < QK; ++i) {
        const float xi = x[i], vi = v[i];
        const float l = rintf((vi - m) / dd);
        const float c = sqrtf(a + xi * xi);
        const float cr = c * (xi - vi);
        c1[i] = cr * l;
        const double q1 = (double)c1[i];
        s1 = s1 + q1 * q1;
        if (TWO) {
            c2[i] = cr * (m != 0.f ? 1.f : 0.f);
            const double q2 = (double)c2[i];
            s2 = s2 + q2 * q2;
        }
    }
    const float n1 = max_nan((float)sqrt(s1), 1e-30f);
    const float n2 = TWO ? max_nan((float)sqrt(s2), 1e-30f) : 1.f;
#pragma unroll
    for (int i = 0; i < QK; ++i) {
        e1[(b * QK + i) * R + r] = c1[i] / n1;
        if (TWO) e2[(b * QK + i) * R + r] = c2[i] / n2;
    }
}

__global__ __launch_bounds__(256) void k_half_step(const float* __restrict__ x, const float* __restrict__ lo,
                                                   const float* __restrict__ hi, int64_t n, float* __restrict__ h) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float l = lo[i], u = hi[i], v = x[i];
    const bool fl = isfinite(l), fu = isfinite(u);
    h[i] = fl && fu ? 0.5f * (u - l) : fu ? u - v : fl ? v - l : -1.f;
}

__global__ __launch_bounds__(256) void k_est_add(const float* __restrict__ x, const float* __restrict__ h, int64_t n,
                                                 float* __restrict__ ws, float* __restrict__ wx) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float hv = h[i];
    if (hv < 0.f) return;
    const float w = 1.f / fmaxf(hv * hv, 1e-30f);
    ws[i] = ws[i] + w;
    wx[i] = wx[i] + x[i] * w;
}

__global__ __launch_bounds__(256) void k_est_seed(const float* __restrict__ ws, const float* __restrict__ wx,
                                                  const float* __restrict__ x0, int64_t n, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float s = ws[i];
    if (s > 0.f) {
        out[2 * i] = wx[i] / s;
        out[2 * i + 1] = 1.f / sqrtf(s);
    } else {
        out[2 * i] = x0[i];
        out[2 * i + 1] = 0.f;
    }
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace
}  // namespace spa

using spa::fail;

extern "C" {

int spa_imx_conditions(int T, const float* X, const void* F, const float* V, const double* rowsq, int64_t R, int64_t cols,
                       float* e1, float* e2, void* stream) {
    if (T != 2 && T != 3 && T != 6 && T != 7)
        return fail(SPA_ERR_TYPE, "spa_imx_conditions: type %d is not Q4_0, Q4_1, Q5_0 or Q5_1", T);
    if (R < 0 || cols <= 0 || cols % 32) return fail(SPA_ERR_ARG, "spa_imx_conditions: %lld columns (a multiple of 32)", (long long)cols);
    if (!R) return SPA_OK;
    const bool two = T == 3 || T == 7;
    if (!X || !F || !V || !rowsq || !e1 || (two && !e2)) return fail(SPA_ERR_ARG, "spa_imx_conditions: null pointer");
    if (cols / 32 > 65535) return fail(SPA_ERR_ARG, "spa_imx_conditions: %lld blocks per row (at most 65535)", (long long)(cols / 32));
    const dim3 grid(spa::blocks_for(R), (unsigned)(cols / 32));
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* f = (const uint8_t*)F;
    switch (T) {
        case 2: hipLaunchKernelGGL((spa::k_conditions<32, 18, false>), grid, dim3(256), 0, st, X, f, V, rowsq, R, cols, e1, e2); break;
        case 3: hipLaunchKernelGGL((spa::k_conditions<32, 20, true>), grid, dim3(256), 0, st, X, f, V, rowsq, R, cols, e1, e2); break;
        case 6: hipLaunchKernelGGL((spa::k_conditions<32, 22, false>), grid, dim3(256), 0, st, X, f, V, rowsq, R, cols, e1, e2); break;
        default: hipLaunchKernelGGL((spa::k_conditions<32, 24, true>), grid, dim3(256), 0, st, X, f, V, rowsq, R, cols, e1, e2); break;
    }
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_est_half_step(const float* x, const float* lo, const float* hi, int64_t n, float* h, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_est_half_step: negative count");
    if (!n) return SPA_OK;
    if (!x || !lo || !hi || !h) return fail(SPA_ERR_ARG, "spa_est_half_step: null pointer");
    hipLaunchKernelGGL(spa::k_half_step, dim3(spa::blocks_for(n)), dim3(256), 0, (hipStream_t)stream, x, lo, hi, n, h);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_est_add(const float* x, const float* h, int64_t n, float* ws, float* wx, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_est_add: negative count");
    if (!n) return SPA_OK;
    if (!x || !h || !ws || !wx) return fail(SPA_ERR_ARG, "spa_est_add: null pointer");
    hipLaunchKernelGGL(spa::k_est_add, dim3(spa::blocks_for(n)), dim3(256), 0, (hipStream_t)stream, x, h, n, ws, wx);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_est_seed(const float* ws, const float* wx, const float* x0, int64_t n, float* out, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_est_seed: negative count");
    if (!n) return SPA_OK;
    if (!ws || !wx || !x0 || !out) return fail(SPA_ERR_ARG, "spa_est_seed: null pointer");
    hipLaunchKernelGGL(spa::k_est_seed, dim3(spa::blocks_for(n)), dim3(256), 0, (hipStream_t)stream, ws, wx, x0, n, out);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
