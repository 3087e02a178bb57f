/* seedpack_amd -- C ABI of the MI355X (gfx950) seed-and-regrow hot path.
 *
 * Plain pointers and sizes only. Device pointers are HIP device allocations (spa_malloc or any
 * hipMalloc'd memory of the same process); `stream` is a hipStream_t or NULL for the null stream.
 * Every function returns SPA_OK (0) or a negative SPA_ERR_* code; spa_last_error() returns the
 * calling thread's last message. Quantize/encode calls only enqueue work on `stream`.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   - seedpack/gpuquant.py:202-211   k_quantize_<fn> kernels (one thread per row) and
 *     seedpack/gpuquant.py:360-456   GPUQuant.quantize_tensors / _launch;
 *   - seedpack/requant.py:21-42      quantize_<t>(src, dst, nrow, n_per_row, imatrix) of libggmlq;
 *   - seedpack/gpuquant.py:248-260   the BF16 -> f32 widening pass (fused into the load here);
 *   - seedpack/gpuquant.py:311-326   IQ table upload (built by the library itself here).
 */
#ifndef SEEDPACK_AMD_H
#define SEEDPACK_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPA_OK 0
#define SPA_ERR_OVERFLOW (-1)   /* an output slot was too small (caller retries with more room) */
#define SPA_ERR_TYPE (-2)       /* unknown or unsupported ggml type / variant */
#define SPA_ERR_ASSERT (-3)     /* a precondition of the reference quantizer failed (GGML_ASSERT) */
#define SPA_ERR_ARG (-4)        /* bad size, alignment or pointer */
#define SPA_ERR_HIP (-5)        /* a HIP runtime call failed */

#define SPA_SRC_BF16 0
#define SPA_SRC_F16 1
#define SPA_SRC_F32 2

/* ---- runtime plumbing (device memory, streams, events) ---- */
const char* spa_last_error(void);
int spa_device_count(int* n);
int spa_set_device(int device);
int spa_malloc(void** ptr, size_t nbytes);
int spa_free(void* ptr);
int spa_memcpy_h2d(void* dst, const void* src, size_t nbytes, void* stream);
int spa_memcpy_d2h(void* dst, const void* src, size_t nbytes, void* stream);
int spa_memcpy_d2d(void* dst, const void* src, size_t nbytes, void* stream);
int spa_memset(void* ptr, int value, size_t nbytes, void* stream);
int spa_stream_create(void** stream);
int spa_stream_destroy(void* stream);
int spa_stream_synchronize(void* stream);
int spa_device_synchronize(void);
int spa_event_create(void** event);
int spa_event_destroy(void* event);
int spa_event_record(void* event, void* stream);
int spa_event_elapsed_ms(float* ms, void* start, void* stop);
int spa_mem_info(size_t* free_bytes, size_t* total_bytes);
/* Device-to-device copy by a plain streaming kernel (16-byte multiples); the HBM yardstick the
 * traffic counters of the other kernels are scaled against. No reference counterpart. */
int spa_copy(void* dst, const void* src, size_t nbytes, void* stream);

/* ---- quantizers ---- */

/* Bytes of one quantized row: n_per_row / qk * block_bytes (requant.py:21-27); 0 for an unknown
 * type or a row length that is not a whole number of blocks. */
size_t spa_row_size(int ggml_type, int64_t n_per_row);

/* Number of quantizer variants of a type (IQ1_M has 2: the current search and the pre-f95b0d9539
 * one, gpuquant.py:182-185); 0 if the type is not supported. */
int spa_type_variants(int ggml_type);

/* Quantizes nrows x n_per_row weights (row-major, src_kind SPA_SRC_*) into dst
 * (nrows * spa_row_size bytes), byte-identical to llama.cpp's quantize_<type>(src, dst, nrows,
 * n_per_row, imatrix) built with -ffp-contract=off. imatrix: device pointer to n_per_row floats,
 * or NULL for the reference (no-imatrix) path. Replaces gpuquant.py:205-211 + :432-456. */
int spa_quantize(int ggml_type, int variant, const void* src, int src_kind, int64_t nrows, int64_t n_per_row,
                 const float* imatrix, void* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SEEDPACK_AMD_H */
