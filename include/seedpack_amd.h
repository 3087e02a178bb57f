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
/* How the library's waits (spa_stream_synchronize, spa_event_synchronize, spa_memcpy_h2d / d2h) wait
 * for the device: 0 the
 * runtime's stream synchronisation (it spins a core until the work is done), 1 an event recorded and
 * polled with sleeps of 20 to 500 us between polls (the core free for host work). Process-wide. No
 * reference counterpart: the packer and the unpacker, whose host side is CPU-bound, use 1. */
int spa_set_sync_mode(int blocking);
int spa_get_device(int* device);
int spa_malloc(void** ptr, size_t nbytes);
int spa_free(void* ptr);
/* Page-locked host memory (hipHostMalloc): copies to and from it run at the link's full rate, as the
 * reference's pinned staging does (gpuquant.py:266-282). */
int spa_host_alloc(void** ptr, size_t nbytes);
int spa_host_free(void* ptr);
int spa_memcpy_h2d(void* dst, const void* src, size_t nbytes, void* stream);
int spa_memcpy_d2h(void* dst, const void* src, size_t nbytes, void* stream);
/* The copy queued on `stream` without waiting for it (dst page-locked; wait with an event). */
int spa_memcpy_d2h_async(void* dst, const void* src, size_t nbytes, void* stream);
int spa_memcpy_d2d(void* dst, const void* src, size_t nbytes, void* stream);
int spa_memset(void* ptr, int value, size_t nbytes, void* stream);
int spa_stream_create(void** stream);
int spa_stream_destroy(void* stream);
int spa_stream_synchronize(void* stream);
int spa_device_synchronize(void);
int spa_event_create(void** event);
int spa_event_destroy(void* event);
int spa_event_record(void* event, void* stream);
/* Work queued on `stream` after this call waits for `event`'s last record. */
int spa_stream_wait_event(void* stream, void* event);
int spa_event_elapsed_ms(float* ms, void* start, void* stop);
/* Waits for the work before `event`'s last record (as spa_set_sync_mode says). */
int spa_event_synchronize(void* event);
int spa_mem_info(size_t* free_bytes, size_t* total_bytes);
/* Device-to-device copy by a plain streaming kernel (16-byte multiples); the HBM yardstick the
 * traffic counters of the other kernels are scaled against. No reference counterpart. */
int spa_copy(void* dst, const void* src, size_t nbytes, void* stream);
/* VALU issue-rate probe: nblocks workgroups of 256 lanes, each lane `iters` loop trips of independent
 * plain 32-bit VALU instructions (op 0: 128 v_fma_f32, op 1: 128 v_add_f32, op 2: 128 v_xor_b32 +
 * 128 v_add_u32, op 3: 64 v_fma_f32 + 64 v_xor_b32 + 64 v_add_u32, op 4: 64 v_mul_f32 + 64 v_add_f32,
 * op 5: 128 v_mul_f32 per trip), nothing stored (`out`,
 * nblocks x 256 floats, is written only in a case the inputs never reach). The VALU yardstick of the
 * searches' roof, as spa_copy is HBM's. spa_valu_probe_insts: the loop's wave64 VALU instructions per
 * launch. No reference counterpart. */
int spa_valu_probe(int op, int64_t nblocks, int iters, float* out, void* stream);
int64_t spa_valu_probe_insts(int op, int64_t nblocks, int iters);
/* n synthetic BF16 weights N(0, std) written in place from a counter-based hash of (seed, index), for
 * benchmark inputs generated on the device. No reference counterpart. */
int spa_synth_normal_bf16(void* dst, int64_t n, uint64_t seed, float std, void* stream);
/* No counterpart in the reference: a synthetic "published" quant file for benchmarks. In about
 * per_million / 10^6 of the nblocks blocks of block_bytes (a counter hash of (seed, block) picks
 * them), one byte is XORed with a non-zero value, as the reference's configuration 1 perturbs 1% of
 * its target's blocks. */
int spa_perturb_blocks(void* dst, int64_t nblocks, int block_bytes, uint32_t per_million, uint64_t seed,
                       void* stream);

/* ---- host helpers ---- */

/* Bytes that `count` consecutive GGUF strings (uint64 length, then the bytes) take from p, or
 * UINT64_MAX when they would run past `avail`: the GGUF header reader steps over a tokenizer's string
 * arrays with it (gguf_reader.py:47-121 reads them item by item). Host memory; no device call. */
uint64_t spa_gguf_strings_bytes(const void* p, uint64_t avail, uint64_t count);

/* CRC-32 of n bytes as zlib.crc32(data, crc) computes it (crc: the previous result, 0 to start): the
 * container's chunk checksums (container.py:59, :85, :162 compute them with zlib.crc32). Host memory,
 * carry-less multiplication folding where the CPU has it. */
uint32_t spa_crc32(uint32_t crc, const void* data, size_t n);

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
 * or NULL for the reference (no-imatrix) path. work: optional device scratch (4-byte aligned) of
 * spa_quantize_work_bytes bytes, used by this call only; NULL is accepted for every type (the
 * imatrix Q4_0/Q4_1/Q5_0/Q5_1 then compute their row statistics inside the quantizer launch,
 * 2.4-4.3x slower). The library allocates nothing. Replaces gpuquant.py:205-211 + :432-456. */
int spa_quantize(int ggml_type, int variant, const void* src, int src_kind, int64_t nrows, int64_t n_per_row,
                 const float* imatrix, void* dst, void* work, void* stream);

/* Bytes of the optional `work` scratch of spa_quantize (0: the call uses none): one float per row
 * for the imatrix Q4_0, Q4_1, Q5_0 and Q5_1 (their row mean squares, ggml-quants.c:2082-2084). */
uint64_t spa_quantize_work_bytes(int ggml_type, int64_t nrows, int64_t n_per_row, int has_imatrix);

/* Dequantizes nrows x n_per_row weights of a quantized row-major run of blocks (src) into dst
 * (nrows * n_per_row floats, 16-byte aligned), bit-identical to llama.cpp's
 * dequantize_row_<type> (ggml-quants.c:439-568, :961-1968, :2489-2764) for the 20 types
 * spa_quantize supports. Replaces the k_dq_<type> launches of GPUQuant.dequantize
 * (gpuquant.py:214-219, :413-421). */
int spa_dequantize(int ggml_type, const void* src, int64_t nrows, int64_t n_per_row, float* dst, void* stream);

/* Host view of IQ lattice table `index` (0 IQ2_XXS, 1 IQ2_XS, 2 IQ1_S/IQ1_M, 3 IQ2_S, 4 IQ3_XXS,
 * 5 IQ3_S), built by the library on first use: the codebook as coordinate bytes (8 or 4 per point),
 * the level-index map and the neighbour lists, equal to what llama.cpp's iq2xs_init_impl /
 * iq3xs_init_impl build (ggml-quants.c:2854-3259, :3704-3903; the reference ships them as
 * seedpack/ggml/iqtables.npz and uploads them, gpuquant.py:311-326). Pointers stay valid for the
 * process. */
int spa_iq_table_host(int index, const void** grid, int* grid_bytes, const int32_t** map, int* map_n,
                      const uint16_t** neighbours, int* nb_n);

/* ---- QR residual coder (all 20 quant types; seedpack/qr.py) ----
 * Batch descriptors are device arrays with the reference's byte layout (qr.py:898-900):
 *   tm: one 32-byte record per tensor {i64 blk0, i64 seed_off, i32 seed_type, i32 cols, i64 imx_off}
 *   sg: one 16-byte record per segment {i32 t, i32 nb, i64 b0}
 * F, P: the batch's file and predicted blocks back to back; seed: the seed tensors (BF16 = type 30,
 * F32 = 0, F16 = 1) addressed by seed_off. gk (the grid keys, qr.py:935-948) and imx (the tensors'
 * importance, addressed by imx_off) are read for the grid types (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS,
 * IQ3_S, IQ1_S, IQ1_M) and may be NULL otherwise.
 * mv: the model version recorded with the batch (2 for new batches, 1 for archives before 0.3.0). */

/* Blocks per rANS segment of a type: max(16, 16384 / QK) (qr.py:952-954); 0 if not a QR type. */
int spa_qr_seg_blocks(int ggml_type);

/* Device workspace bytes spa_qr_hist and spa_qr_encode need for nseg segments of the type: per
 * block slot its equality flag and a list entry (about 5 bytes per block). */
size_t spa_qr_work_bytes(int ggml_type, int nseg);

/* Symbol histogram of the batch into counts[294][256] (u32, accumulated: zero it first). work:
 * spa_qr_work_bytes of device scratch, used by this call only. Replaces the qr_hist kernel
 * (qr.py:674-710). */
int spa_qr_hist(int ggml_type, const void* F, const void* P, const void* seed, const void* tm, const void* sg,
                int nseg, uint32_t* counts, const uint16_t* gk, const float* imx, int mv, void* work, void* stream);

/* rANS-encodes each segment backwards into its own `cap`-byte slot of out (nseg * cap bytes), the
 * stream ending at the slot's end; out_len[s] = bytes used, or 0xFFFFFFFF if the slot overflowed
 * (the caller retries with a larger cap). remap[294] maps a context to its table row (-1 unused),
 * freq[n][256] (u16, rows sum to 4096), cum[n][257]; work as for spa_qr_hist. Replaces qr_enc
 * (qr.py:712-758). */
int spa_qr_encode(int ggml_type, const void* F, const void* P, const void* seed, const void* tm, const void* sg,
                  int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap,
                  uint32_t* out_len, const uint16_t* gk, const float* imx, int mv, void* work, void* stream);

/* Decodes every segment (stream bytes of segment s start at in + in_off[s]) into F (the batch's
 * blocks). `in` holds in_bytes of stream: reads past them see zeros (a damaged stream decodes to
 * garbage, never outside its buffer). lut[n][4096] from spa_rans_build_lut32. Replaces qr_dec
 * (qr.py:760-807). */
int spa_qr_decode(int ggml_type, const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* P,
                  const void* seed, const void* tm, const void* sg, int nseg, const int* remap, const uint16_t* freq,
                  const uint32_t* cum, const uint32_t* lut, void* F, const uint16_t* gk, const float* imx, int mv,
                  void* stream);

/* No counterpart in the reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc). spa_qr_encode with its workspace
 * taken from a static per-device scratch of spa_qr_noalloc_scratch_bytes() (64 MiB) instead of a
 * `work` argument: no allocation, no hipMemset. Calls whose spa_qr_work_bytes(ggml_type, nseg) exceed
 * it fail with SPA_ERR_ARG. All calls on one device share that scratch, and the library orders them:
 * each call's stream waits for the event the previous call on the device recorded after its kernels,
 * so calls on other streams or threads run one after another on the GPU and never race (the first
 * call on a device sets up the scratch's address and that event). Under
 * a HIP graph capture no wait or record is added: the captured graph's own order must keep calls
 * apart. */
int spa_qr_encode_noalloc(int ggml_type, const void* F, const void* P, const void* seed, const void* tm,
                          const void* sg, int nseg, const int* remap, const uint16_t* freq, const uint32_t* cum,
                          void* out, uint64_t cap, uint32_t* out_len, const uint16_t* gk, const float* imx, int mv,
                          void* stream);
size_t spa_qr_noalloc_scratch_bytes(void);

/* ---- per-weight side information of the seed-less and sibling coders (qr.py:811-878) ----
 * seed types of the TM records besides 0 / 1 / 30 (float seeds) and the non-grid QR types (a
 * quantized seed, dequantized per weight with half its code step as the uncertainty): 98 = no seed,
 * the seed buffer holds the tensor's per-column RMS (float32) and the codes are coded against zero;
 * 99 = explicit, the seed buffer holds float32 (value, uncertainty) pairs per weight. */

/* lo/hi[i] = the interval of values that rounds to weight i's code in blocks F of non-grid type T
 * (qr.intervals, qr.py:819-844). */
int spa_qr_intervals(int T, const void* F, int64_t nw, float* lo, float* hi, void* stream);
/* h[i] = half the step between the grid levels around weight i of grid-type blocks F (qr.explicit_seed's
 * grid_h, qr.py:811-817). */
int spa_qr_grid_h(int T, const void* F, int64_t nw, float* h, void* stream);
/* out[i] = 1 where weight i's code and its sub-block's integer scale (and min) are the same in F and P
 * (qr.weight_equal, qr.py:846-863). */
int spa_qr_weight_equal(int T, const void* F, const void* P, int64_t nw, uint8_t* out, void* stream);
/* the scale fields of every block (spa_qr_nfields(T) ints per block) and blocks made of given fields with
 * zero codes (qr.self_side's block_fields / blocks_from_fields, qr.py:865-878). */
int spa_qr_block_fields(int T, const void* F, int64_t nblk, int* out, void* stream);
int spa_qr_blocks_from_fields(int T, const int* v, int n, void* out, void* stream);
int spa_qr_nfields(int T);

/* Compacts the segment slots into one stream: dst[off[s] ..] = the last len[s] bytes of slot s.
 * Replaces gather (qr.py:880-887, gpu2.py:264-271). */
int spa_qr_gather(const void* src, uint64_t cap, const uint32_t* len, const uint64_t* off, int nseg, void* dst,
                  void* stream);

/* lut[t][slot] = the symbol whose cumulative range holds slot, for ntab tables of 4096 slots.
 * Replaces build_lut (qr.py:889-895, gpu2.py:273-279). */
int spa_rans_build_lut(const uint32_t* cum, int ntab, uint8_t* lut, void* stream);

/* lut[t][slot] = s | (freq[s] - 1) << 8 | (slot - cum[s]) << 20 for the symbol s whose cumulative
 * range holds slot, ntab tables of 4096 slots: the QR decoders' table (one load per symbol). Replaces
 * build_lut with the frequency and cumulative lookups of qr_dec folded in (qr.py:760-807, :889-895). */
int spa_rans_build_lut32(const uint32_t* cum, int ntab, uint32_t* lut, void* stream);

/* ---- difference residual (replaces the host-side chunked numpy stage of repo3.py:456-510) ---- */

/* dst = a ^ b over n bytes (dst may be a). nonzero: optional device u64 set to the number of
 * non-zero bytes of dst. Replaces _xor_async / _xor_chunk (repo3.py:456-467). */
int spa_xor(void* dst, const void* a, const void* b, size_t n, unsigned long long* nonzero, void* stream);

/* dst = a ^ b ^ c and its non-zero byte count: the residual a file region holding file ^ p0 would
 * have with prediction c instead. Replaces _xor3 (repo3.py:494-504). */
int spa_xor3(void* dst, const void* a, const void* b, const void* c, size_t n, unsigned long long* nonzero,
             void* stream);

/* *count (device u64) = number of bytes where a and b differ (b NULL: non-zero bytes of a).
 * Replaces _count_diff / _diff_async (repo3.py:476-491). */
int spa_diff_count(const void* a, const void* b, size_t n, unsigned long long* count, void* stream);

/* *count (device u64) = number of non-zero bytes among a[0], a[stride], a[2 stride], ... below n: the
 * sample the residual frame's zstd level is judged from, np.count_nonzero(v[::61]) (repo3.py:1537,
 * :1940), taken on the device-resident residual. */
int spa_count_every(const void* a, size_t n, size_t stride, unsigned long long* count, void* stream);

/* BLAKE3 (default hash mode, 32-byte digests) of nregions byte regions of the device buffer `base`:
 * the reference's file checksum (cli.py:34-39, its catalog's "hash": "blake3") and tensor keys
 * (repo3.py:529, :1029, :2018-2022; siblings.py:216-240), which it computes with the blake3 package on
 * the host. regions (host, u64): offset and length of each region; work (device) of
 * spa_blake3_work_bytes(regions, nregions) bytes; digests (host): 32 bytes per region. Synchronous:
 * returns when the digests are in `digests` (the stream's earlier work is waited for). */
size_t spa_blake3_work_bytes(const uint64_t* regions, int nregions);
int spa_blake3(const void* base, const uint64_t* regions, int nregions, void* work, size_t work_bytes, uint8_t* digests,
               void* stream);

/* BLAKE3 of host data fed in pieces (the reference's blake3.blake3(...).update / hexdigest, used
 * where a file is checked as it is written): spa_b3h_new, then spa_b3h_update with each piece in
 * order (the whole chunks of a large piece hashed on up to `threads` threads), spa_b3h_final for the
 * 32-byte digest (the state is left as it was), spa_b3h_free. A hasher is not shared between threads. */
int spa_b3h_new(void** h);
int spa_b3h_update(void* h, const void* data, size_t n, int threads);
int spa_b3h_final(void* h, uint8_t* out32);
int spa_b3h_free(void* h);

/* Float-tensor prediction from the base weights (src_kind SPA_SRC_*): n values written as the file's
 * type dst_type = 0 (F32), 1 (F16, round to nearest even) or 30 (BF16, (u + 0x7FFF + ((u >> 16) & 1))
 * >> 16). Replaces _float_dev (repo3.py:673-689). */
int spa_float_pred(const void* src, int src_kind, int64_t n, int dst_type, void* dst, void* stream);

/* ---- deterministic arithmetic (replaces detmath.py's kernels dm_rows / dm_rows_d / dm_cols / dm_gram /
 * dm_bdot / dm_solve / dm_log2 / dm_exp2, detmath.py:60-259): float64 sums term by term in index order,
 * products of floats exact in float64, nothing contracted. All launch on `stream` and return. */

/* out[r] = sum_j x[r][j] (sq: x[r][j]^2) over the nr x nc row-major array x (f64 = 0: float32, 1:
 * float64, 2: BF16 bits widened to float32). detmath.rows (detmath.py:185-192). */
int spa_dm_rows(const void* x, int f64, int64_t nr, int64_t nc, int sq, double* out, void* stream);
/* out[c] = sum_r x[r][c] (sq: squares) over the rows r with mask[r] != 0 (mask NULL: all).
 * detmath.cols (detmath.py:195-202). */
int spa_dm_cols(const float* x, int64_t nr, int64_t nc, int sq, const uint8_t* mask, double* out, void* stream);
/* X: n x k x d float32 (k <= 32) -> out[c] = X[c] X[c]^T (n x k x k float32 of float64 sums).
 * detmath.gram (detmath.py:210-216). */
int spa_dm_gram(const float* X, int64_t n, int k, int64_t d, float* out, void* stream);
/* X: n x k x d, y: n x d (k <= 32) -> out[c] = X[c] y[c] (n x k). detmath.bdot (detmath.py:219-225). */
int spa_dm_bdot(const float* X, const float* y, int64_t n, int k, int64_t d, float* out, void* stream);
/* n systems A[c] x = b[c] (k <= 16), Gaussian elimination with partial pivoting in float64.
 * detmath.solve (detmath.py:228-235). */
int spa_dm_solve(const float* A, const float* b, int64_t n, int k, float* x, void* stream);
/* float64 log2 / exp2 elementwise (detmath.py:20-58, :171-182). */
int spa_dm_log2(const double* x, int64_t n, double* y, void* stream);
int spa_dm_exp2(const double* x, int64_t n, double* y, void* stream);

/* ---- M6 Q8_0 codec (codecs_gguf's single-file method M6: gpu_codec.py's hist / encode / decode kernels
 * and the array steps of M6GPU.compress / decompress, gpu_codec.py:33-169, :218-334). blocks: the file's
 * Q8_0 blocks back to back (34 bytes each); meta: 24-byte records {first, nblocks, nb_row, grp, colbase,
 * med} per tensor (gpu_codec.py:190 META_DT); tfirst: each tensor's first block; colmap: per input
 * column its class 0..15, tensors back to back; segments of 512 blocks, 770 tables per tensor group,
 * PB 12. */

/* counts[lo | hi << 8] += 1 for blocks [first, first + nb) (the median of the scale bits, gpu_codec.py:231). */
int spa_m6_scale_hist(const void* blocks, int64_t first, int64_t nb, uint32_t* counts, void* stream);
/* rms[c] = sqrt(sum over rows of q^2 / nrows) per column of nrows x (nb_row * 32) weights, float32 sums
 * in row order (gpu_codec.py:232-233 as the reference's --cpu path computes it). */
int spa_m6_col_rms(const void* blocks, int64_t first, int64_t nrows, int nb_row, float* rms, void* stream);
/* pos[b]: the first position of the largest |weight| of block b (gpu_codec.py:238). */
int spa_m6_pos(const void* blocks, int64_t n, uint8_t* pos, void* stream);
/* the number of 512-block segments of nblocks blocks */
int spa_m6_segments(int nblocks);
/* counts[table * 256 + symbol] += every block's symbols (gpu_codec.py:80-93). */
int spa_m6_hist(const void* blocks, const uint8_t* pos, const void* meta, const int32_t* tfirst, int ntens,
                const uint8_t* colmap, int nblocks, uint32_t* counts, void* stream);
/* each segment coded into its slot of cap (>= 512 * 34 * 2 + 16) bytes, written downwards from the slot's
 * end; out_len[s] its length (gpu_codec.py:95-124); gather with spa_qr_gather. */
int spa_m6_encode(const void* blocks, const uint8_t* pos, const void* meta, const int32_t* tfirst, int ntens,
                  const uint8_t* colmap, int nblocks, const uint16_t* freq, const uint32_t* cum, void* out, uint64_t cap,
                  uint32_t* out_len, void* stream);
/* segment s decoded from in + in_off[s] into blocks (gpu_codec.py:126-157); bytes past in_bytes read as
 * zeros; lut from spa_rans_build_lut. */
int spa_m6_decode(const void* in, uint64_t in_bytes, const uint64_t* in_off, const void* meta, const int32_t* tfirst,
                  int ntens, const uint8_t* colmap, int nblocks, const uint16_t* freq, const uint32_t* cum,
                  const uint8_t* lut, void* blocks, void* stream);

/* ---- static context-mixed rANS (rans.py:55-138: _encode, _decode, _decode_o1; the coder of the CPU
 * single-file methods M3-M5). One stream per lane; streams: 48-byte records {i64 sym_off, n, ctx_off,
 * tab_row, out_off; i32 period, pad}: symbols sym[sym_off..+n), contexts ctx[ctx_off..+n) (decode with
 * period > 0: the previous symbol, reset to 0 every period symbols, ctx unused), tables freq / cum rows
 * tab_row + context (n_sym and n_sym + 1 entries, rows summing to 2^14). */

/* each stream coded into out[out_off, out_off + 2n + 16), written downwards from its end; out_len its length. */
int spa_crans_encode(const uint8_t* sym, const int32_t* ctx, int n_sym, const uint16_t* freq, const uint32_t* cum,
                     const void* streams, int nst, void* out, uint32_t* out_len, void* stream);
/* each stream decoded from in + out_off (bytes past in_bytes read as zeros) into sym; lut from
 * spa_rans_build_lut_pb with pb 14. */
int spa_crans_decode(const void* in, uint64_t in_bytes, const int32_t* ctx, int n_sym, const uint16_t* freq,
                     const uint32_t* cum, const uint8_t* lut, const void* streams, int nst, uint8_t* sym, void* stream);

/* ---- M24 BF16 codec (method m28's base codec; replaces gpu_bf16.py's bf_hist / bf_enc / bf_dec and the
 * column statistics of M24BF16GPU.compress_dev, gpu_bf16.py:36-132, :340-371). TB descriptors are 24
 * bytes {i64 off, i32 rowlen, rowbase, colbase, tab}, SG 16 bytes {i32 t, n, i64 i0} (gpu_bf16.py:271-272);
 * segments of 16384 weights, 160 tables per tensor, PB 12. */

/* s1[c] / s2[c] = float64 sums in row order of w[r][c] / rfa[r] (and its square), w BF16 bits nr x rowlen,
 * the quotient in float32. */
int spa_m24_cols(const void* w, const float* rfa, int64_t nr, int rowlen, double* s1, double* s2, void* stream);
/* counts[(tab + ctx) * 256 + symbol] += the segments' exponent, mantissa and sign symbols. */
int spa_m24_hist(const void* file, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                 const int8_t* scl, uint32_t* counts, void* stream);
/* encode: each segment into its slot of cap bytes (>= 2 * 16384 + 1024), written downwards, out_len[s] its
 * length (0xffffffff on overflow); rcp: a workspace of spa_m24_rcp_bytes(ntab) bytes. */
size_t spa_m24_rcp_bytes(int ntab);
int spa_m24_encode(const void* file, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                   const int8_t* scl, const int* remap, int ntab, const uint16_t* freq, const uint32_t* cum, uint32_t* rcp,
                   void* out, uint64_t cap, uint32_t* out_len, void* stream);
/* decode segment s from in + in_off[s] (reads past in_bytes see zeros) into the tensors of file;
 * lut from spa_rans_build_lut. */
int spa_m24_decode(const void* in, uint64_t in_bytes, const uint64_t* in_off, void* file, const void* tb, const void* sg,
                   int nseg, const int16_t* rfi, const int16_t* cfi, const int8_t* scl, const int* remap,
                   const uint16_t* freq, const uint32_t* cum, const uint8_t* lut, void* stream);

/* ---- M22 Q8_0 codec (gpu3.M22Fast: the codec of Q8Parts and of a seed's Q8_0 tensors). Replaces the
 * kernels of gpu2.py:37-297 (hist_a / enc_a / dec_a, hist_b / enc_b / dec_b) and gpu3.py:26-230 (predict,
 * predict_multi, hist_c / enc_c / dec_c) and the array steps of GPU2.compress / GPU3._plan_tensor
 * (gpu2.py:554-616, gpu3.py:272-353) with detmath.sim8 (detmath.py:250-259). blocks: the coded tensors'
 * Q8_0 blocks back to back (34 bytes each); meta: 32-byte records {first, nblocks, nb_row, grp, colbase,
 * rowbase, off, qset} per tensor (gpu2.py:278 META_DT); skip: per block, bit 0 a duplicate row (not
 * coded), bit 1 coded by phase C, bit 2 position and maximum coded by phase C. Tables: PB 12, phase A
 * 4384 per group, phase B 1088 per group from qbase, phase C 88 per predicted tensor. */

/* pos[b]: the first position of the largest |weight| of block b. */
int spa_q8_pos(const void* blocks, int64_t n, uint8_t* pos, void* stream);
/* row_m[r] = (sum of the row's fp16 scale bits) / blocks per row, rows of all tensors in meta order. */
int spa_q8_row_means(const void* blocks, const void* meta, int ntens, int64_t nrows, int* row_m, void* stream);
/* A tensor's column sums for the context statistics: rel[block] = float(exp2(float(bits - row mean) / 1024))
 * (workspace, nrows * nbr floats), then per slice s of rows_per_slice rows and column c the float64 sums in
 * row order of w and w^2, w = float(q) * rel: part1 / part2 [nslices][nbr * 32] (gpu2.py:588-597). */
int spa_q8_col_stats(const void* blocks, int first, int nbr, int64_t nrows, const int* row_m, float* rel,
                     int64_t rows_per_slice, double* part1, double* part2, void* stream);
/* Duplicate rows: h[r] = sum over the row's 64-bit words of word * mult[word] mod 2^64 (nbr * 34 a multiple
 * of 8), and eq[i] = rows ra[i] and rb[i] are byte-equal (gpu2.py:693-716). */
int spa_q8_row_hash(const void* blocks, int first, int nbr, int64_t nrows, const uint64_t* mult, uint64_t* h, void* stream);
int spa_q8_rows_equal(const void* blocks, int first, int nbr, const int* ra, const int* rb, int n, uint8_t* eq, void* stream);
/* The encoder's reciprocals rcp[t][s] of freq[t][s] for ntab used tables; the decoders' tables lut[t][slot] =
 * symbol | (freq - 1) << 8 | (slot - cum[symbol]) << 20 (4096 words per table). */
int spa_q8_rcp(const uint16_t* freq, int ntab, uint32_t* rcp, void* stream);
int spa_q8_lut32(const uint16_t* freq, const uint32_t* cum, int ntab, uint32_t* lut, void* stream);
/* Phase A (scale bytes, maximum's rank and value; 4096 blocks per segment): histogram, encode (slots of cap
 * bytes written downwards, out_len[s] = length or 0xffffffff on overflow), decode (reads past in_bytes see
 * zeros; lut from spa_q8_lut32). bcf / spread per block-column, perm / rankof [block-column][32], scls per
 * column. */
int spa_q8_hist_a(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                  const uint8_t* bcf, const uint8_t* spread, const uint8_t* rankof, const uint8_t* scls, uint32_t* counts,
                  void* stream);
int spa_q8_enc_a(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                 const uint8_t* bcf, const uint8_t* spread, const uint8_t* rankof, const uint8_t* scls, const int* remap,
                 const uint16_t* freq, const uint32_t* cum, const uint32_t* rcp, void* out, uint64_t cap, uint32_t* out_len,
                 void* stream);
int spa_q8_dec_a(const void* in, uint64_t in_bytes, const uint64_t* in_off, const uint8_t* skip, const void* meta, int ntens,
                 int nblocks, const uint8_t* bcf, const uint8_t* spread, const uint8_t* perm, const uint8_t* scls,
                 const int* remap, const uint32_t* lut, void* blocks, uint8_t* pos, void* stream);
/* Phase B (the other 31 weights, 1024 blocks per segment). The histogram takes work items of 12 bytes
 * {tensor, first block, blocks} (blocks of one tensor, a workgroup each) and counts into the tensor's qset. */
int spa_q8_hist_b(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                  const void* items, int nitems, const int16_t* cfi, const uint8_t* scls, const int* row_m, int qbase,
                  uint32_t* counts, void* stream);
int spa_q8_enc_b(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, int ntens, int nblocks,
                 const int16_t* cfi, const uint8_t* scls, const int* row_m, int qbase, const int* remap, const uint16_t* freq,
                 const uint32_t* cum, const uint32_t* rcp, void* out, uint64_t cap, uint32_t* out_len, void* stream);
int spa_q8_dec_b(const void* in, uint64_t in_bytes, const uint64_t* in_off, const uint8_t* skip, const void* meta, int ntens,
                 int nblocks, const int16_t* cfi, const uint8_t* scls, const int* row_m, int qbase, const int* remap,
                 const uint32_t* lut, void* blocks, const uint8_t* pos, void* stream);
/* Phase C. Row prediction pint[r][j] (int8) from up to 4 parents per row (par / coef [rows][4], mu per
 * column): all rows of one tensor (encoder), or the entries (slot, row) of one wave of every predicted
 * tensor (decoder; slots: 32-byte records {i64 rbase, i64 pbase, i32 first, nbr, mubase, pad}). Segments:
 * 16-byte records {tensor, first row, rows, slot}. fbin per row, cfi with the residual column adjustment. */
int spa_q8_predict(const void* blocks, int first, int nbr, int64_t nrows, const int* par, const float* coef, const float* mu,
                   int8_t* pint, void* stream);
int spa_q8_predict_multi(const void* blocks, const int* ent_slot, const int* ent_row, int nent, int cmax, const void* slots,
                         const int* par, const float* coef, const float* mu, int8_t* pint, void* stream);
/* Per block of 32 predictions (nblk blocks of pint): prk[j] the rank of position j by |prediction|
 * descending (ties by position), pinv[rank] its position, rctx the rank context min(max |p| / 16, 7)
 * (gpu3.py:48-60); the phase C coders read these (prk / pinv laid out as pint, rctx one per block). */
int spa_q8_ranks(const int8_t* pint, int64_t nblk, int8_t* prk, int8_t* pinv, int8_t* rctx, void* stream);
int spa_q8_hist_c(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, const void* segs, int nseg,
                  const void* slots, const int16_t* cfi, const int* row_m, const int8_t* fbin, const int8_t* pint,
                  const int8_t* prk, const int8_t* pinv, const int8_t* rctx, uint32_t* counts, void* stream);
int spa_q8_enc_c(const void* blocks, const uint8_t* pos, const uint8_t* skip, const void* meta, const void* segs, int nseg,
                 const void* slots, const int16_t* cfi, const int* row_m, const int8_t* fbin, const int8_t* pint,
                 const int8_t* prk, const int8_t* pinv, const int8_t* rctx, const int* remap, const uint16_t* freq,
                 const uint32_t* cum, const uint32_t* rcp, void* out, uint64_t cap, uint32_t* out_len, void* stream);
/* decodes segments [seg0, seg1) (one wave) */
int spa_q8_dec_c(const void* in, uint64_t in_bytes, const uint64_t* in_off, int seg0, int seg1, const uint8_t* skip,
                 const void* meta, const void* segs, int nseg, const void* slots, const int16_t* cfi, const int* row_m,
                 const int8_t* fbin, const int8_t* pint, const int8_t* prk, const int8_t* pinv, const int8_t* rctx,
                 const int* remap, const uint32_t* lut, void* blocks, uint8_t* pos, void* stream);
/* The row-prediction planner (gpu3.py:272-353). W[r][c] = q * d (float32, exact); W -= mu per column; Wq =
 * clip(rint(W / nrm[r] * 127), -127, 127) in float64, 0 for rows that are not valid. */
int spa_q8_row_matrix(const void* blocks, int first, int nbr, int64_t nrows, float* W, void* stream);
int spa_q8_center(float* W, const float* mu, int64_t nrows, int C, void* stream);
int spa_q8_norm_i8(const float* W, const double* nrm, const uint8_t* valid, int64_t nrows, int C, int8_t* Wq, void* stream);
/* S[ra][rb] = A B^T exactly in int32 for int8 rows of C columns (C a multiple of 32, 16-byte aligned rows):
 * detmath.sim8. */
int spa_q8_sim8(const int8_t* A, int64_t ra, const int8_t* B, int64_t rb, int C, int32_t* S, void* stream);
/* cand[r][0..3]: the rows c < wstart[r] with valid[c] of largest Wq[r].Wq[c], ties to the lower row, -1 where
 * fewer exist (the reference's sim8 + masked argmax rounds, gpu3.py:296-310). */
int spa_q8_neighbours(const int8_t* Wq, int64_t n, int C, const int* wstart, const uint8_t* valid, int* cand, void* stream);
/* Per row: least squares on its first k = 1..4 candidates (Gram + 1e-3 I, detmath.solve, coefficients in
 * 1/64 steps), the k of lowest estimated bits: frac (residual energy fraction), kuse, coefs [n][4]. */
int spa_q8_fit_rows(const float* W, const int* cand, int64_t n, int C, float* frac, int* kuse, float* coefs, void* stream);
/* part[ch][c]: float64 sums in row order of the chosen residual^2 over the valid rows of each chunk of rows. */
int spa_q8_col_res(const float* W, const int* cand, const float* coefs, const int* kuse, const uint8_t* valid, int64_t n,
                   int C, int64_t chunk, double* part, void* stream);

/* ---- estimating what a quant was made from ---- */

/* The importance fit's conditions of rows X (R x cols float32) quantized as F (type T = Q4_0, Q4_1,
 * Q5_0 or Q5_1; V its dequantized values, rowsq detmath's row sums of squares of X): per weight
 * sqrt(rowsq/cols + x^2) (x - v) l, with l the weight's code (Q4_1 / Q5_1 also times [min != 0]),
 * normalised per block, written as (block of columns, position, row) float32 into e1 (and e2).
 * Replaces the body of imxfit.ls_gram before its Gram sums (imxfit.py:37-58). */
int spa_imx_conditions(int T, const float* X, const void* F, const float* V, const double* rowsq, int64_t R, int64_t cols,
                       float* e1, float* e2, void* stream);
/* The sibling estimate (siblings.py:51-77 half_step / est_add / est_seed): half the interval of a
 * weight's code from its bounds (-1: none); the running precision-weighted sums; the explicit seed
 * (x, h) per weight, or (x0, 0) where no version told anything. */
int spa_est_half_step(const float* x, const float* lo, const float* hi, int64_t n, float* h, void* stream);
int spa_est_add(const float* x, const float* h, int64_t n, float* ws, float* wx, void* stream);
int spa_est_seed(const float* ws, const float* wx, const float* x0, int64_t n, float* out, void* stream);

/* ---- R2 BF16 base codec (replaces the kernels and statistics of bf16v2.py:24-155, :225-271) ----
 * TB descriptors are 32 bytes {i64 doff, i32 rowlen, rowbase, colbase, tab, rmap, pad} and SG 16 bytes
 * {i32 t, n, i64 i0}, the layout of bf16v2.py:157-158 TB_DT / SG_DT; segments of 16384 weights.
 * TB.pad, unused by the reference, is read by spa_r2_hist only: the first of the 64 exponent contexts
 * it counts in LDS (clamped to 0..448); any value gives the same counts. */

/* Side information of one tensor of BF16 bits (nrows x rowlen): rfi[nrows], cfi[rowlen], scl[rowlen]
 * (BF16v2._stats, bf16v2.py:225-244, with detmath.py's sums, log2 and exp2); row_hash[nrows] (optional)
 * the 64-bit row fingerprints (row_hash kernel, bf16v2.py:148-155); work: device workspace of
 * work_bytes >= spa_r2_stats_work_bytes(nrows, rowlen); rf_out (optional): the float64 log2 row RMS.
 * Launches only, on `stream`: tensors given different streams overlap. */
int spa_r2_stats(const void* w, int64_t nrows, int rowlen, int16_t* rfi, int16_t* cfi, int8_t* scl, uint64_t* row_hash,
                 void* work, uint64_t work_bytes, double* rf_out, void* stream);
/* Workspace bytes spa_r2_stats needs for a tensor of nrows x rowlen (0 for an empty one). */
uint64_t spa_r2_stats_work_bytes(int64_t nrows, int rowlen);

/* Context counts of the coded weights of nseg segments (v2_hist, bf16v2.py:54-75); counts has
 * (roles x 656) rows of 256 u32 and is added to. */
int spa_r2_hist(const void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                const int8_t* scl, const int32_t* rowmap, uint32_t* counts, void* stream);

/* Coding words for nctx contexts (roles x 656): fcw[c][sym] = freq[remap[c]][sym] << 16 |
 * cum[remap[c]][sym] (256 u32 per context; zeros where remap[c] < 0). The reference's v2_enc reads
 * freq, cum and remap per symbol (bf16v2.py:84-111). */
int spa_r2_encode_tables(const int32_t* remap, int nctx, const uint16_t* freq, const uint32_t* cum, uint32_t* fcw,
                         void* stream);

/* rANS encode of nseg segments (v2_enc, bf16v2.py:77-111) with spa_r2_encode_tables' words: slot s
 * of `out` (16-byte aligned; cap bytes, a multiple of 16) ends with the segment's bytes, out_len[s]
 * their count (0xFFFFFFFF: under 64 bytes left after some weight, the reference's overflow).
 * fc_work: ceil(nseg / 64) x 64 x 16384 x 3 u32 of workspace. */
int spa_r2_encode(const void* dev, const void* tb, const void* sg, int nseg, const int16_t* rfi, const int16_t* cfi,
                  const int8_t* scl, const int32_t* rowmap, const uint32_t* fcw, uint32_t* fc_work, void* out,
                  uint64_t cap, uint32_t* out_len, void* stream);

/* rANS decode of nseg segments into dev (v2_dec, bf16v2.py:113-137): `in` (16-byte aligned) holds
 * in_bytes of coded stream, segment s starting at in_off[s]; reads stop at in_bytes rounded up to 16
 * (a damaged stream decodes to garbage, never past its buffer, which must span that rounding).
 * dtab from spa_r2_build_dec_tables over all roles x 656 contexts (the reference decodes through
 * build_lut's 2^15-entry tables and a remap, bf16v2.py:113-145; these give the same symbols). */
int spa_r2_decode(const void* in, uint64_t in_bytes, const uint64_t* in_off, void* dev, const void* tb, const void* sg,
                  int nseg, const int16_t* rfi, const int16_t* cfi, const int8_t* scl, const int32_t* rowmap,
                  const uint8_t* dtab, void* stream);

/* Compact decode tables for nctx contexts (roles x 656): context c gets table remap[c] of cum
 * (257 u32 per table), or a one-symbol table when remap[c] < 0; spa_r2_dec_table_bytes() bytes per
 * context: per 128-slot bucket the u64 (symbol | cum << 8 | freq << 24) of its first slot's symbol,
 * then every symbol's u32 (cum | freq << 16). */
int spa_r2_build_dec_tables(const uint32_t* cum, const int32_t* remap, int nctx, uint8_t* dtab, void* stream);
uint64_t spa_r2_dec_table_bytes(void);

/* Duplicate rows restored from their sources: rows pairs[2i] = rows pairs[2i+1] of a tensor of rowlen
 * BF16 weights per row (bf16v2.py:471-476). */
int spa_r2_copy_rows(void* w, int rowlen, const int64_t* pairs, int npairs, void* stream);

/* Decode lookup tables for precision pb (2^pb slots per table); spa_rans_build_lut is pb = 12.
 * Replaces build_lut (bf16v2.py:139-145). */
int spa_rans_build_lut_pb(const uint32_t* cum, int ntab, int pb, uint8_t* lut, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SEEDPACK_AMD_H */
