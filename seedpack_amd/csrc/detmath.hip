// Deterministic arithmetic for the coders' decisions (detmath.py): float64 sums in index order, one
// output per lane (row and column sums, batched Gram matrices and matrix-vector products), small
// systems by Gaussian elimination with partial pivoting, and log2 / exp2 from basic operations. The
// results are fixed functions of the inputs: every sum is formed term by term in index order, the
// products of two floats are exact in float64, and nothing is contracted.
//
// MI355X mapping: the order of each sum is serial, so the lanes share the loads instead: row sums
// stage 64x64 tiles through LDS with coalesced loads and each lane then walks its row of the tile;
// Gram / bdot stage 64 columns of a batch element's k rows and each lane walks its (a, b) pairs over
// them (the Gram matrix is symmetric term by term, so a <= b is formed once and mirrored); a system
// is solved by one wave, a lane per equation.
#include "../../include/seedpack_amd.h"
#include "common.h"
#include "detmath.h"
#include "launch.h"

namespace spa {
namespace {

constexpr int TILE = 64;

// an element as float64: float32 / float64 as they are, uint16 as BF16 bits
__device__ __forceinline__ double as_f64(float v) { return (double)v; }
__device__ __forceinline__ double as_f64(double v) { return v; }
__device__ __forceinline__ double as_f64(uint16_t u) { return (double)__uint_as_float((uint32_t)u << 16); }

template <typename T>
__global__ __launch_bounds__(TILE) void k_rows(const T* __restrict__ x, int64_t nr, int64_t nc, int sq,
                                               double* __restrict__ out) {
    __shared__ T tile[TILE][TILE + 1];
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * TILE;
    const int64_t row = r0 + lane;
    double s = 0.0;
    for (int64_t c0 = 0; c0 < nc; c0 += TILE) {
        const int64_t c = c0 + lane;
#pragma unroll 8
        for (int r = 0; r < TILE; ++r)
            tile[r][lane] = (r0 + r < nr && c < nc) ? x[(r0 + r) * nc + c] : T(0);
        __syncthreads();
        const int n = nc - c0 < TILE ? (int)(nc - c0) : TILE;
        if (row < nr) {
            if (sq)
                for (int j = 0; j < n; ++j) { const double v = as_f64(tile[lane][j]); s = s + v * v; }
            else
                for (int j = 0; j < n; ++j) s = s + as_f64(tile[lane][j]);
        }
        __syncthreads();
    }
    if (row < nr) out[row] = s;
}

// Column sums in row order, 64 columns per workgroup: the 256 lanes load a tile of CT_ROWS rows x 64
// columns (coalesced 256-byte row pieces, the next tile's values held in registers while the current
// one is summed), lanes 0..63 add their column's values from LDS in row order (one float64 chain per
// column, as the reference's lane per column).
constexpr int CT_ROWS = 128;
__global__ __launch_bounds__(256) void k_cols(const float* __restrict__ x, int64_t nr, int64_t nc, int sq,
                                              const uint8_t* __restrict__ mask, double* __restrict__ out) {
    __shared__ float tile[CT_ROWS][64 + 1];
    __shared__ uint8_t on[CT_ROWS];
    const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;          // grp: rows grp, grp + 4, ...
    const int64_t c0 = (int64_t)blockIdx.x * 64, c = c0 + lane;
    constexpr int PER = CT_ROWS / 4;
    float v[PER];
    auto fetch = [&](int64_t r0) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int64_t r = r0 + grp + 4 * k;
            v[k] = (r < nr && c < nc) ? x[r * nc + c] : 0.f;
        }
    };
    double s = 0.0;
    fetch(0);
    for (int64_t r0 = 0; r0 < nr; r0 += CT_ROWS) {
#pragma unroll
        for (int k = 0; k < PER; ++k) tile[grp + 4 * k][lane] = v[k];
        if (threadIdx.x < CT_ROWS) {
            const int64_t r = r0 + threadIdx.x;
            on[threadIdx.x] = r < nr && (!mask || mask[r]);
        }
        __syncthreads();
        if (r0 + CT_ROWS < nr) fetch(r0 + CT_ROWS);          // in flight while this tile is summed
        if (threadIdx.x < 64 && c < nc) {
            const int n = nr - r0 < CT_ROWS ? (int)(nr - r0) : CT_ROWS;
            for (int r = 0; r < n; ++r)
                if (on[r]) { const double d = (double)tile[r][lane]; s = s + (sq ? d * d : d); }
        }
        __syncthreads();
    }
    if (threadIdx.x < 64 && c < nc) out[c] = s;
}

// X: n x k x d; out[c][a][b] = sum_t X[c][a][t] X[c][b][t] (a workgroup per batch element c)
__global__ __launch_bounds__(256) void k_gram(const float* __restrict__ X, int k, int64_t d, float* __restrict__ out) {
    extern __shared__ float xs[];                 // [k][TILE + 1]
    const int64_t c = blockIdx.x;
    const float* xc = X + c * (int64_t)k * d;
    const int npair = k * (k + 1) / 2;
    // a lane's pairs: p = threadIdx.x + 256 q, at most 2 for k <= 16, 3 for k <= 32 (528 pairs)
    constexpr int PMAX = 3;
    int pa[PMAX], pb[PMAX];
    double s[PMAX];
#pragma unroll
    for (int q = 0; q < PMAX; ++q) {
        int p = threadIdx.x + 256 * q, a = 0;
        pa[q] = -1;
        pb[q] = 0;
        s[q] = 0.0;
        if (p < npair) {
            while (p >= k - a) { p -= k - a; ++a; }
            pa[q] = a;
            pb[q] = a + p;
        }
    }
    for (int64_t t0 = 0; t0 < d; t0 += TILE) {
        const int n = d - t0 < TILE ? (int)(d - t0) : TILE;
        for (int i = threadIdx.x; i < k * TILE; i += 256) {
            const int a = i / TILE, j = i % TILE;
            xs[a * (TILE + 1) + j] = j < n ? xc[(int64_t)a * d + t0 + j] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PMAX; ++q) {
            if (pa[q] < 0) continue;
            const float* xa = xs + pa[q] * (TILE + 1);
            const float* xb = xs + pb[q] * (TILE + 1);
            for (int j = 0; j < n; ++j) s[q] = s[q] + (double)xa[j] * (double)xb[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < PMAX; ++q) {
        if (pa[q] < 0) continue;
        const float v = (float)s[q];
        out[(c * k + pa[q]) * k + pb[q]] = v;
        out[(c * k + pb[q]) * k + pa[q]] = v;
    }
}

// out[c][a] = sum_t X[c][a][t] y[c][t]
__global__ __launch_bounds__(64) void k_bdot(const float* __restrict__ X, const float* __restrict__ y, int k, int64_t d,
                                             float* __restrict__ out) {
    __shared__ float xs[32][TILE + 1];
    __shared__ float ys[TILE];
    const int64_t c = blockIdx.x;
    const int a = threadIdx.x;
    double s = 0.0;
    for (int64_t t0 = 0; t0 < d; t0 += TILE) {
        const int n = d - t0 < TILE ? (int)(d - t0) : TILE;
        for (int r = 0; r < k; ++r) xs[r][threadIdx.x] = threadIdx.x < n ? X[(c * k + r) * d + t0 + threadIdx.x] : 0.f;
        ys[threadIdx.x] = threadIdx.x < n ? y[c * d + t0 + threadIdx.x] : 0.f;
        __syncthreads();
        if (a < k)
            for (int j = 0; j < n; ++j) s = s + (double)xs[a][j] * (double)ys[j];
        __syncthreads();
    }
    if (a < k) out[c * k + a] = (float)s;
}

// A[c] x = b[c], k <= 16: a wave per system, lane i holds equation i (k coefficients + right side)
__global__ __launch_bounds__(64) void k_solve(const float* __restrict__ A, const float* __restrict__ b, int k,
                                              float* __restrict__ x) {
    const int64_t c = blockIdx.x;
    const int i = threadIdx.x;
    double m[17];
#pragma unroll
    for (int j = 0; j < 17; ++j) {
        const bool in = i < k && j <= k;
        m[j] = !in ? 0.0 : (j < k ? (double)A[(c * k + i) * k + j] : (double)b[c * k + i]);
    }
#pragma unroll
    for (int col = 0; col < 16; ++col) {
        if (col >= k) continue;             // (uniform; the loop stays unrolled, col a constant)
        // pivot: the first equation from col on with the largest |m[col]| (strict compares in index
        // order); lanes below col and past k do not take part
        double best = __shfl(fabs(m[col]), col, 64);
        int piv = col;
        for (int r = col + 1; r < k; ++r) {
            const double v = __shfl(fabs(m[col]), r, 64);
            if (v > best) { best = v; piv = r; }
        }
        if (piv != col) {                         // swap equations col and piv
#pragma unroll
            for (int j = 0; j < 17; ++j) {
                const double vc = __shfl(m[j], col, 64), vp = __shfl(m[j], piv, 64);
                if (i == col) m[j] = vp;
                if (i == piv) m[j] = vc;
            }
        }
        const double p = __shfl(m[col], col, 64);
        const double f = m[col] / p;
#pragma unroll
        for (int j = 0; j < 17; ++j) {
            const double mc = __shfl(m[j], col, 64);
            if (i > col && i < k && j >= col && j <= k) m[j] = m[j] - f * mc;
        }
    }
    // back substitution from the last equation up: x_r = (m_r[k] - sum_{j>r} m_r[j] x_j) / m_r[r], the
    // terms in j order (coefficients picked by unrolled selects: no register array is indexed at run
    // time)
    double xi = 0.0;
    for (int r = k - 1; r >= 0; --r) {
        double s = 0.0, dg = 1.0;
#pragma unroll
        for (int j = 0; j < 17; ++j) {
            if (j == k) s = m[j];
            if (j == r) dg = m[j];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const double xj = __shfl(xi, j, 64);
            if (j > r && j < k) s = s - m[j] * xj;
        }
        const double v = s / dg;
        if (i == r) xi = v;
    }
    if (i < k) x[c * k + i] = (float)xi;
}

__global__ __launch_bounds__(256) void k_log2(const double* __restrict__ x, int64_t n, double* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = dm::dm_log2(x[i]);
}
__global__ __launch_bounds__(256) void k_exp2(const double* __restrict__ x, int64_t n, double* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = dm::dm_exp2(x[i]);
}

unsigned blocks_for(int64_t n, int wg) { return (unsigned)((n + wg - 1) / wg); }

}  // namespace
}  // namespace spa

using spa::fail;

extern "C" {

int spa_dm_rows(const void* x, int f64, int64_t nr, int64_t nc, int sq, double* out, void* stream) {
    if (nr < 0 || nc < 0) return fail(SPA_ERR_ARG, "spa_dm_rows: negative shape");
    if (!nr) return SPA_OK;
    if (!out || (nc && !x)) return fail(SPA_ERR_ARG, "spa_dm_rows: null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (f64 == 2)
        hipLaunchKernelGGL(spa::k_rows<uint16_t>, dim3(spa::blocks_for(nr, spa::TILE)), dim3(spa::TILE), 0, st,
                           (const uint16_t*)x, nr, nc, sq, out);
    else if (f64)
        hipLaunchKernelGGL(spa::k_rows<double>, dim3(spa::blocks_for(nr, spa::TILE)), dim3(spa::TILE), 0, st,
                           (const double*)x, nr, nc, sq, out);
    else
        hipLaunchKernelGGL(spa::k_rows<float>, dim3(spa::blocks_for(nr, spa::TILE)), dim3(spa::TILE), 0, st,
                           (const float*)x, nr, nc, sq, out);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_dm_cols(const float* x, int64_t nr, int64_t nc, int sq, const uint8_t* mask, double* out, void* stream) {
    if (nr < 0 || nc < 0) return fail(SPA_ERR_ARG, "spa_dm_cols: negative shape");
    if (!nc) return SPA_OK;
    if (!out || (nr && !x)) return fail(SPA_ERR_ARG, "spa_dm_cols: null pointer");
    hipLaunchKernelGGL(spa::k_cols, dim3(spa::blocks_for(nc, 64)), dim3(256), 0, (hipStream_t)stream, x, nr, nc, sq,
                       mask, out);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_dm_gram(const float* X, int64_t n, int k, int64_t d, float* out, void* stream) {
    if (n < 0 || d < 0 || k < 1 || k > 32) return fail(SPA_ERR_ARG, "spa_dm_gram: n %lld, k %d (1..32), d %lld", (long long)n, k, (long long)d);
    if (!n) return SPA_OK;
    if (!X || !out) return fail(SPA_ERR_ARG, "spa_dm_gram: null pointer");
    hipLaunchKernelGGL(spa::k_gram, dim3((unsigned)n), dim3(256), (size_t)k * (spa::TILE + 1) * sizeof(float),
                       (hipStream_t)stream, X, k, d, out);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_dm_bdot(const float* X, const float* y, int64_t n, int k, int64_t d, float* out, void* stream) {
    if (n < 0 || d < 0 || k < 1 || k > 32) return fail(SPA_ERR_ARG, "spa_dm_bdot: n %lld, k %d (1..32), d %lld", (long long)n, k, (long long)d);
    if (!n) return SPA_OK;
    if (!X || !y || !out) return fail(SPA_ERR_ARG, "spa_dm_bdot: null pointer");
    hipLaunchKernelGGL(spa::k_bdot, dim3((unsigned)n), dim3(64), 0, (hipStream_t)stream, X, y, k, d, out);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_dm_solve(const float* A, const float* b, int64_t n, int k, float* x, void* stream) {
    if (n < 0 || k < 1 || k > 16) return fail(SPA_ERR_ARG, "spa_dm_solve: n %lld, k %d (1..16)", (long long)n, k);
    if (!n) return SPA_OK;
    if (!A || !b || !x) return fail(SPA_ERR_ARG, "spa_dm_solve: null pointer");
    hipLaunchKernelGGL(spa::k_solve, dim3((unsigned)n), dim3(64), 0, (hipStream_t)stream, A, b, k, x);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_dm_log2(const double* x, int64_t n, double* y, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_dm_log2: negative count");
    if (!n) return SPA_OK;
    if (!x || !y) return fail(SPA_ERR_ARG, "spa_dm_log2: null pointer");
    hipLaunchKernelGGL(spa::k_log2, dim3(spa::blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, x, n, y);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

int spa_dm_exp2(const double* x, int64_t n, double* y, void* stream) {
    if (n < 0) return fail(SPA_ERR_ARG, "spa_dm_exp2: negative count");
    if (!n) return SPA_OK;
    if (!x || !y) return fail(SPA_ERR_ARG, "spa_dm_exp2: null pointer");
    hipLaunchKernelGGL(spa::k_exp2, dim3(spa::blocks_for(n, 256)), dim3(256), 0, (hipStream_t)stream, x, n, y);
    SPA_HIP_TRY(hipGetLastError());
    return SPA_OK;
}

}  // extern "C"
