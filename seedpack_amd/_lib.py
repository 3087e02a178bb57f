"""ctypes binding of libseedpack_amd.so (the C ABI declared in include/seedpack_amd.h).

The library is the product path: there is no CPU fallback. If the shared object is missing or a
HIP call fails, the error is raised, never papered over.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libseedpack_amd.so")

_lib = None
_lock = threading.Lock()

c_void_p, c_int, c_int64, c_size_t, c_float = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
c_uint64 = ctypes.c_uint64

# name -> (restype, argtypes); every symbol of include/seedpack_amd.h
SIGNATURES = {
    "spa_last_error": (ctypes.c_char_p, []),
    "spa_device_count": (c_int, [ctypes.POINTER(c_int)]),
    "spa_set_device": (c_int, [c_int]),
    "spa_set_sync_mode": (c_int, [c_int]),
    "spa_get_device": (c_int, [ctypes.POINTER(c_int)]),
    "spa_malloc": (c_int, [ctypes.POINTER(c_void_p), c_size_t]),
    "spa_free": (c_int, [c_void_p]),
    "spa_host_alloc": (c_int, [ctypes.POINTER(c_void_p), c_size_t]),
    "spa_host_free": (c_int, [c_void_p]),
    "spa_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "spa_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "spa_memcpy_d2h_async": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "spa_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "spa_memset": (c_int, [c_void_p, c_int, c_size_t, c_void_p]),
    "spa_stream_create": (c_int, [ctypes.POINTER(c_void_p)]),
    "spa_stream_destroy": (c_int, [c_void_p]),
    "spa_stream_synchronize": (c_int, [c_void_p]),
    "spa_device_synchronize": (c_int, []),
    "spa_event_create": (c_int, [ctypes.POINTER(c_void_p)]),
    "spa_event_destroy": (c_int, [c_void_p]),
    "spa_event_record": (c_int, [c_void_p, c_void_p]),
    "spa_stream_wait_event": (c_int, [c_void_p, c_void_p]),
    "spa_event_elapsed_ms": (c_int, [ctypes.POINTER(c_float), c_void_p, c_void_p]),
    "spa_event_synchronize": (c_int, [c_void_p]),
    "spa_mem_info": (c_int, [ctypes.POINTER(c_size_t), ctypes.POINTER(c_size_t)]),
    "spa_copy": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "spa_valu_probe": (c_int, [c_int, c_int64, c_int, c_void_p, c_void_p]),
    "spa_valu_probe_insts": (c_int64, [c_int, c_int64, c_int]),
    "spa_synth_normal_bf16": (c_int, [c_void_p, c_int64, c_uint64, c_float, c_void_p]),
    "spa_perturb_blocks": (c_int, [c_void_p, c_int64, c_int, ctypes.c_uint32, c_uint64, c_void_p]),
    "spa_dequantize": (c_int, [c_int, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "spa_gguf_strings_bytes": (c_uint64, [c_void_p, c_uint64, c_uint64]),
    "spa_crc32": (ctypes.c_uint32, [ctypes.c_uint32, c_void_p, c_size_t]),
    "spa_row_size": (c_size_t, [c_int, c_int64]),
    "spa_type_variants": (c_int, [c_int]),
    "spa_quantize": (c_int, [c_int, c_int, c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_quantize_work_bytes": (c_uint64, [c_int, c_int64, c_int64, c_int]),
    "spa_iq_table_host": (c_int, [c_int, ctypes.POINTER(c_void_p), ctypes.POINTER(c_int), ctypes.POINTER(c_void_p),
                                  ctypes.POINTER(c_int), ctypes.POINTER(c_void_p), ctypes.POINTER(c_int)]),
    "spa_qr_seg_blocks": (c_int, [c_int]),
    "spa_qr_work_bytes": (c_size_t, [c_int, c_int]),
    "spa_qr_hist": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                            c_void_p, c_int, c_void_p, c_void_p]),
    "spa_qr_encode": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                              c_void_p, c_void_p, ctypes.c_uint64, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                              c_void_p]),
    "spa_qr_decode": (c_int, [c_int, c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                              c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "spa_qr_encode_noalloc": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                      c_void_p, c_void_p, c_void_p, ctypes.c_uint64, c_void_p, c_void_p, c_void_p,
                                      c_int, c_void_p]),
    "spa_qr_noalloc_scratch_bytes": (c_size_t, []),
    "spa_qr_gather": (c_int, [c_void_p, ctypes.c_uint64, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_rans_build_lut": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "spa_rans_build_lut32": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "spa_xor": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "spa_xor3": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "spa_diff_count": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "spa_count_every": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
    "spa_m6_scale_hist": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "spa_m6_col_rms": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "spa_m6_pos": (c_int, [c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_m6_segments": (c_int, [c_int]),
    "spa_m6_hist": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_m6_encode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p,
                              c_void_p, c_uint64, c_void_p, c_void_p]),
    "spa_m6_decode": (c_int, [c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p,
                              c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_crans_encode": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                 c_void_p]),
    "spa_crans_decode": (c_int, [c_void_p, c_uint64, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                 c_void_p, c_void_p]),
    "spa_m24_cols": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p]),
    "spa_m24_hist": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_m24_rcp_bytes": (c_size_t, [c_int]),
    "spa_m24_encode": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                               c_void_p, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p, c_void_p]),
    "spa_m24_decode": (c_int, [c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                               c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_pos": (c_int, [c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_q8_row_means": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p]),
    "spa_q8_col_stats": (c_int, [c_void_p, c_int, c_int, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "spa_q8_row_hash": (c_int, [c_void_p, c_int, c_int, c_int64, c_void_p, c_void_p, c_void_p]),
    "spa_q8_rows_equal": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_q8_rcp": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "spa_q8_lut32": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_q8_hist_a": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_enc_a": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p, c_void_p]),
    "spa_q8_dec_a": (c_int, [c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_hist_b": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_q8_enc_b": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p, c_void_p]),
    "spa_q8_dec_b": (c_int, [c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_predict": (c_int, [c_void_p, c_int, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_predict_multi": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_ranks": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_hist_c": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_enc_c": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int] + [c_void_p] * 13 + [c_uint64, c_void_p, c_void_p]),
    "spa_q8_dec_c": (c_int, [c_void_p, c_uint64, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_row_matrix": (c_int, [c_void_p, c_int, c_int, c_int64, c_void_p, c_void_p]),
    "spa_q8_center": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "spa_q8_norm_i8": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "spa_q8_sim8": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "spa_q8_neighbours": (c_int, [c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_fit_rows": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_q8_col_res": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int64, c_void_p, c_void_p]),
    "spa_qr_intervals": (c_int, [c_int, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "spa_qr_grid_h": (c_int, [c_int, c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_qr_weight_equal": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_qr_block_fields": (c_int, [c_int, c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_qr_blocks_from_fields": (c_int, [c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_qr_nfields": (c_int, [c_int]),
    "spa_dm_rows": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "spa_dm_cols": (c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p, c_void_p]),
    "spa_dm_gram": (c_int, [c_void_p, c_int64, c_int, c_int64, c_void_p, c_void_p]),
    "spa_dm_bdot": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int64, c_void_p, c_void_p]),
    "spa_dm_solve": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "spa_dm_log2": (c_int, [c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_dm_exp2": (c_int, [c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_imx_conditions": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                   c_void_p]),
    "spa_est_half_step": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_est_add": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "spa_est_seed": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "spa_blake3_work_bytes": (c_size_t, [c_void_p, c_int]),
    "spa_blake3": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_size_t, c_void_p, c_void_p]),
    "spa_b3h_new": (c_int, [ctypes.POINTER(c_void_p)]),
    "spa_b3h_update": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
    "spa_b3h_final": (c_int, [c_void_p, c_void_p]),
    "spa_b3h_free": (c_int, [c_void_p]),
    "spa_float_pred": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_void_p]),
    "spa_r2_stats": (c_int, [c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p,
                             c_void_p]),
    "spa_r2_stats_work_bytes": (c_uint64, [c_int64, c_int]),
    "spa_r2_hist": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_r2_encode_tables": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_r2_encode": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_uint64, c_void_p, c_void_p]),
    "spa_r2_decode": (c_int, [c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                              c_void_p, c_void_p, c_void_p, c_void_p]),
    "spa_r2_build_dec_tables": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "spa_r2_dec_table_bytes": (c_uint64, []),
    "spa_r2_copy_rows": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p]),
    "spa_rans_build_lut_pb": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
}


class SpaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


# Calls that wait for the device, allocate or free memory, or work on the host for long release the
# interpreter lock; every other entry point only enqueues device work and keeps it: with other threads
# running Python, releasing and re-acquiring the lock around each launch can cost far more than the
# launch itself.
RELEASE = {
    "spa_malloc", "spa_free", "spa_host_alloc", "spa_host_free", "spa_memcpy_h2d", "spa_memcpy_d2h",
    "spa_stream_create", "spa_stream_destroy", "spa_stream_synchronize", "spa_device_synchronize",
    "spa_event_create", "spa_event_destroy", "spa_event_elapsed_ms", "spa_event_synchronize", "spa_mem_info",
    "spa_device_count",
    "spa_set_device", "spa_crc32", "spa_gguf_strings_bytes", "spa_iq_table_host", "spa_blake3",
    "spa_b3h_new", "spa_b3h_update", "spa_b3h_final", "spa_b3h_free",
}


class _Lib:
    """the library's functions: from a handle that releases the interpreter lock for RELEASE, from
    one that keeps it for the rest"""

    def __init__(self, release, keep):
        self._release, self._keep = release, keep

    def __getattr__(self, name):
        f = getattr(self._release if name in RELEASE else self._keep, name)
        setattr(self, name, f)
        return f


def lib():
    """the loaded library (raises if it has not been built)"""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m seedpack_amd.build` "
                                       "(the HIP path has no CPU fallback)")
                handles = (ctypes.CDLL(LIB_PATH), ctypes.PyDLL(LIB_PATH))
                for L in handles:
                    for name, (res, args) in SIGNATURES.items():
                        f = getattr(L, name)
                        f.restype = res
                        f.argtypes = args
                _lib = _Lib(*handles)
    return _lib


def check(code):
    """raise SpaError for a negative status"""
    if code < 0:
        raise SpaError(code, lib().spa_last_error().decode(errors="replace"))
    return code
