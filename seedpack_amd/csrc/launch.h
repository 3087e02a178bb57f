// Host-side launchers of the quantizer kernels, one per ggml type family. Each returns 0 or a
// negative SPA_ERR_* code and enqueues work on `stream` only (no synchronisation).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spa {

struct QuantArgs {
    int type;               // ggml type id
    int variant;            // quantizer variant (IQ1_M: 0 current, 1 pre-f95b0d9539)
    const void* src;        // device weights, nrows * n_per_row elements
    int src_kind;           // SrcKind
    int64_t nrows;
    int64_t n_per_row;
    const float* imatrix;   // device, n_per_row floats, or nullptr
    void* dst;              // device, nrows * row_size bytes
    hipStream_t stream;
    float* work;            // device scratch of quantize_work_bytes bytes, or nullptr
};

// Device scratch that a quantize launch can use (0: none): the legacy imatrix types keep one row
// statistic per row there.
int64_t quantize_work_bytes(int type, int64_t nrows, bool imatrix);

// Type table (requant.py:21-27): block elements and block bytes; 0 if the type is unknown.
int type_qk(int type);
int type_bs(int type);

int launch_legacy(const QuantArgs& a);   // Q4_0 Q4_1 Q5_0 Q5_1 Q8_0 Q2_0
int launch_kquant(const QuantArgs& a);   // Q2_K Q3_K Q4_K Q5_K Q6_K
int launch_iq4(const QuantArgs& a);      // IQ4_NL IQ4_XS
int launch_iqgrid(const QuantArgs& a);   // IQ2_XXS IQ2_XS IQ2_S IQ3_XXS IQ3_S IQ1_S IQ1_M

// Sets the thread's last error message (printf-style) and returns `code`.
int fail(int code, const char* fmt, ...);

}  // namespace spa

#define SPA_HIP_TRY(expr)                                                                  \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) return ::spa::fail(-5, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)
