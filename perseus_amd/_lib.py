"""ctypes bindings of perseus_amd/libpchip.so (include/pc_hip.h).

The HIP library is the product: nothing here falls back to a CPU path. If the library is missing, importing this
module raises.
"""
import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpchip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "pc_hip.h")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (make -C perseus_amd)")

LIB = C.CDLL(LIB_PATH)

vp = C.c_void_p
u32p = C.POINTER(C.c_uint32)
_SIGS = {
    "pc_table_u32_barrett64": (vp, []),
    "pc_table_u32_logn": (vp, [C.c_uint32]),
    "pc_hip_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "pc_hip_set_device": (C.c_int, [C.c_int]),
    "pc_hip_device_name": (C.c_int, [C.c_int, C.c_char_p, C.c_int]),
    "pc_hip_runtime_version": (C.c_int, [C.POINTER(C.c_int)]),
    "pc_hip_driver_version": (C.c_int, [C.POINTER(C.c_int)]),
    "pc_hip_device_attribute": (C.c_int, [C.POINTER(C.c_int), C.c_int, C.c_int]),
    "pc_hip_mem_get_info": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "pc_hip_profiler_start": (C.c_int, []),
    "pc_hip_profiler_stop": (C.c_int, []),
    "pc_hip_stream_priority_range": (C.c_int, [C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "pc_hip_stream_create_with_priority": (C.c_int, [C.POINTER(vp), C.c_int]),
    "pc_hip_event_create_flags": (C.c_int, [C.POINTER(vp), C.c_uint]),
    "pc_hip_error_name": (C.c_char_p, [C.c_int]),
    "pc_hip_malloc": (C.c_int, [C.POINTER(vp), C.c_size_t]),
    "pc_hip_free": (C.c_int, [vp]),
    "pc_hip_malloc_host": (C.c_int, [C.POINTER(vp), C.c_size_t]),
    "pc_hip_free_host": (C.c_int, [vp]),
    "pc_hip_memcpy_htod": (C.c_int, [vp, vp, C.c_size_t, vp]),
    "pc_hip_memcpy_dtoh": (C.c_int, [vp, vp, C.c_size_t, vp]),
    "pc_hip_memcpy_dtod": (C.c_int, [vp, vp, C.c_size_t, vp]),
    "pc_hip_memset": (C.c_int, [vp, C.c_int, C.c_size_t, vp]),
    "pc_hip_stream_create": (C.c_int, [C.POINTER(vp)]),
    "pc_hip_stream_destroy": (C.c_int, [vp]),
    "pc_hip_stream_sync": (C.c_int, [vp]),
    "pc_hip_stream_wait_event": (C.c_int, [vp, vp]),
    "pc_hip_device_sync": (C.c_int, []),
    "pc_hip_event_create": (C.c_int, [C.POINTER(vp)]),
    "pc_hip_event_destroy": (C.c_int, [vp]),
    "pc_hip_event_record": (C.c_int, [vp, vp]),
    "pc_hip_event_sync": (C.c_int, [vp]),
    "pc_hip_event_elapsed_ms": (C.c_int, [C.POINTER(C.c_float), vp, vp]),
    "pc_hip_graph_begin_capture": (C.c_int, [vp]),
    "pc_hip_graph_end_capture": (C.c_int, [vp, C.POINTER(vp)]),
    "pc_hip_graph_instantiate": (C.c_int, [C.POINTER(vp), vp]),
    "pc_hip_graph_launch": (C.c_int, [vp, vp]),
    "pc_hip_graph_destroy": (C.c_int, [vp]),
    "pc_hip_graph_exec_destroy": (C.c_int, [vp]),
    "pc_hip_error_string": (C.c_char_p, [C.c_int]),
    "pc_hip_last_error": (C.c_int, []),
    "pcx_ctx_new": (vp, [C.c_uint32, C.POINTER(C.c_uint64), C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "pcx_ctx_new_k": (vp, [C.c_uint32, C.POINTER(C.c_uint64), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                           C.POINTER(C.c_int)]),
    "pcx_ctx_free": (None, [vp]),
    "pcx_ctx_table": (vp, [vp]),
    "pcx_ctx_primes": (vp, [vp]),
    "pcx_ctx_twiddle": (vp, [vp, C.c_int]),
    "pcx_ctx_root": (C.c_uint64, [vp, C.c_int]),
    "pcx_ctx_workspace_bytes": (C.c_size_t, [vp]),
    "pcx_ctx_table_only": (C.c_int, [vp, C.c_int]),
    "pcx_ctx_conv_fusion": (C.c_int, [vp, C.c_int]),
    "pcx_rows_new": (vp, [vp, u32p, C.POINTER(C.c_int32), C.c_int]),
    "pcx_rows_free": (None, [vp]),
    "pcx_ntt": (C.c_int, [vp, C.c_int, vp, vp, vp]),
    "pcx_keys_new": (vp, [vp, C.c_int, C.POINTER(C.c_uint64), u32p, C.POINTER(vp), C.c_int, C.POINTER(C.c_int)]),
    "pcx_keys_generate": (vp, [vp, C.c_int, C.POINTER(C.c_uint64), C.POINTER(C.c_int8), u32p,
                               C.POINTER(C.c_int64), C.c_int, C.POINTER(C.c_int)]),
    "pcx_keys_free": (None, [vp]),
    "pcx_keys_resident_a": (C.c_int, [vp, C.c_int, vp]),
    "pcx_keys_resident_bytes": (C.c_size_t, [vp]),
    "pcx_drbg_new": (vp, [u32p, C.c_uint32]),
    "pcx_drbg_free": (None, [vp]),
    "pcx_drbg_u32": (C.c_uint32, [vp]),
    "pcx_drbg_ksk_seed": (C.c_int, [vp, u32p]),
    "pcx_drbg_sparse_ternary": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.POINTER(C.c_int8)]),
    "pcx_drbg_gaussian": (C.c_int, [vp, C.c_double, C.c_uint32, C.POINTER(C.c_int64)]),
    "pcx_keygen_draw": (C.c_int, [vp, C.c_int, C.c_int, C.c_uint32, C.c_double, u32p, C.POINTER(C.c_int64)]),
    "pcx_keys_download_b": (C.c_int, [vp, C.c_int, u32p]),
    "pcx_ct_words": (C.c_size_t, [vp]),
    "pcx_rotate": (C.c_int, [vp, vp, C.c_int, vp, C.c_int, vp, vp]),
    "pcx_rotate_hoisted": (C.c_int, [vp, vp, C.POINTER(C.c_int), C.c_int, vp, C.c_int, vp, vp]),
    "pcx_rotate_sum": (C.c_int, [vp, vp, C.POINTER(C.c_int), C.c_int, vp, C.c_int, vp, vp, vp]),
    "pcx_ntt_one_pass_min": (C.c_int, [C.c_int]),
    "pcx_rotate_many": (C.c_int, [vp, vp, C.POINTER(C.c_int), C.c_int, C.POINTER(vp), C.c_int, vp, vp, vp]),
    "pcx_rotate_and_sum": (C.c_int, [vp, vp, vp, C.c_int, C.c_int64, C.c_int64, C.c_int, vp, vp, vp]),
    "pcx_rotate_and_sum_k": (C.c_int, [vp, vp, vp, C.c_int, C.c_int64, C.c_int64, C.c_int, vp, vp, C.c_int, vp]),
    "pcx_rotate_and_sum_noalloc": (C.c_int, [vp, vp, vp, C.c_int, C.c_int64, C.c_int64, C.c_int, vp, vp]),
    "pcx_cts_stage": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, C.c_int, C.c_uint32, vp, C.c_int, vp,
                                vp]),
    "pcx_cts_stage_hoisted": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, C.c_int, C.c_uint32, vp,
                                        C.c_int, vp, vp, vp]),
    "pcx_moddown_k": (C.c_int, [vp, vp, C.c_int, vp, C.c_int, vp]),
    "pcx_keys_relin": (vp, [vp, C.POINTER(C.c_int8), u32p, C.POINTER(C.c_int64), C.c_int, C.POINTER(C.c_int)]),
    "pcx_rescale": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, vp]),
    "pcx_rescale_k": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, C.c_int, vp]),
    "pcx_mul_relin": (C.c_int, [vp, vp, vp, vp, C.c_int, vp, vp]),
    "pcx_mul_relin_rescale": (C.c_int, [vp, vp, vp, vp, C.c_int, vp, vp]),
    "pcx_mul_relin_rescale_k": (C.c_int, [vp, vp, vp, vp, C.c_int, vp, C.c_int, C.c_int, vp]),
    "pcx_mul_relin_rescale_list": (C.c_int, [vp, vp, C.POINTER(vp), C.POINTER(vp), C.c_int, C.c_int, vp, C.c_int, vp]),
    "pcx_mul_sum_relin_rescale_list": (C.c_int, [vp, vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(C.c_int), C.c_int,
                                                 C.c_int, C.POINTER(vp), C.POINTER(vp), C.c_uint, C.c_int, vp, vp]),
    "pcx_rotate_many_rescale": (C.c_int, [vp, vp, C.POINTER(C.c_int), C.c_int, C.POINTER(vp), C.c_int, vp, vp, vp]),
    "pcx_mul_plain": (C.c_int, [vp, vp, vp, C.c_int, vp, vp]),
    "pcx_mul_plain_k": (C.c_int, [vp, vp, C.POINTER(vp), C.c_int, C.c_int, vp, vp]),
    "pcx_modup": (C.c_int, [vp, vp, C.c_int, vp]),
    "pcx_modup_digits": (vp, [vp]),
    "pcx_dot": (C.c_int, [vp, vp, C.c_int, vp, C.c_int, vp, vp]),
    "pcx_moddown": (C.c_int, [vp, vp, C.c_int, vp, vp]),
    "pcx_timing": (C.c_int, [vp, C.c_int]),
    "pcx_timing_read": (C.c_int, [vp, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_int)]),
    "pcx_copy_probe": (C.c_int, [vp, vp, C.c_size_t, vp]),
    "pcx_valu_probe": (C.c_int, [C.c_int, C.c_int, C.c_int, vp, vp]),
    "pcx_keys_patch_bytes": (C.c_size_t, [vp]),
    "pcx_keys_new_banded": (vp, [vp, C.c_int, C.POINTER(C.c_uint64), u32p, C.POINTER(vp), C.c_int, C.c_int,
                                 C.POINTER(C.c_int)]),
    "pcx_keys_q_top": (C.c_int, [vp]),
    "pcx_decryptor_new": (vp, [vp, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "pcx_decryptor_free": (None, [vp]),
    "pcx_decryptor_load_secret": (C.c_int, [vp, u32p, C.c_int, vp]),
    "pcx_decrypt_rows": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(LIB, _name)
    _f.restype = _res
    _f.argtypes = _args


def header_functions():
    """The function names include/pc_hip.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(pc\w+|pcx\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


class HipError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != 0:
        msg = LIB.pc_hip_error_string(rc)
        raise HipError(f"{what}: {rc} ({msg.decode() if msg else '?'})")
    return rc
