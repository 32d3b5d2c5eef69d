"""ctypes binding of libspx.so (include/spx.h)."""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libspx.so")


class SpxError(RuntimeError):
    pass


P = C.c_void_p
I64 = C.c_int64
_lib = None

SIGNATURES = {
    "spx_last_error": (C.c_char_p, []),
    "spx_create": (C.c_int, [C.c_int, C.POINTER(P)]),
    "spx_destroy": (C.c_int, [P]),
    "spx_sync": (C.c_int, [P]),
    "spx_get_stream": (P, [P]),
    "spx_row_bytes": (I64, [C.c_int, I64]),
    "spx_tensor_upload": (C.c_int, [P, C.c_int, I64, I64, C.c_int, P, C.POINTER(P)]),
    "spx_tensor_download": (C.c_int, [P, P, P]),
    "spx_tensor_free": (C.c_int, [P, P]),
    "spx_q8k_quantize": (C.c_int, [P, P, I64, I64, C.c_int, P, P, P]),
    "spx_matmul_rows_q8k": (C.c_int, [P, P, C.c_int, P, P, P, C.c_int, P, I64, I64, I64]),
    "spx_block_sums_q8k": (C.c_int, [P, P, C.c_int, I64, P, P, P]),
    "spx_matvec": (C.c_int, [P, P, C.c_int, P, I64, C.c_int, P, I64]),
    "spx_matvec_noalloc": (C.c_int, [P, P, C.c_int, P, I64, C.c_int, P, I64]),
    "spx_moe": (C.c_int, [P, P, P, P, P, I64, C.c_int, C.c_int, P, P, P, I64]),
    "spx_moe_dev": (C.c_int, [P, P, P, P, P, I64, C.c_int, C.c_int, P, P, P, I64]),
    "spx_synth_tensor": (C.c_int, [C.c_int, I64, I64, C.c_int, C.c_uint64, C.c_float, C.c_int, P]),
    "spx_engine_create": (C.c_int, [P, P, C.POINTER(P)]),
    "spx_engine_set_tensor": (C.c_int, [P, C.c_char_p, C.c_int, I64, I64, C.c_int, P]),
    "spx_engine_prepare": (C.c_int, [P]),
    "spx_engine_set_graphs": (C.c_int, [P, C.c_int]),
    "spx_engine_set_decode": (C.c_int, [P, C.c_int]),
    "spx_engine_decode_pipeline": (C.c_int, [P, C.POINTER(C.c_int)]),
    "spx_engine_set_mfma": (C.c_int, [P, C.c_int]),
    "spx_engine_set_persist": (C.c_int, [P, C.c_int]),
    "spx_engine_persist_active": (C.c_int, [P, C.POINTER(C.c_int)]),
    "spx_engine_forward": (C.c_int, [P, P, C.c_int, C.c_int, P, P, P]),
    "spx_engine_feed": (C.c_int, [P, P, C.c_int, C.c_int, P, P, P]),
    "spx_engine_last_experts": (C.c_int, [P, P]),
    "spx_engine_debug_read": (C.c_int, [P, C.c_char_p, P, I64]),
    "spx_engine_debug_layers": (C.c_int, [P, C.c_int]),
    "spx_engine_debug_layout": (C.c_int, [P, P]),
    "spx_engine_expert_counts": (C.c_int, [P, P]),
    "spx_engine_kv_download": (C.c_int, [P, P, P]),
    "spx_engine_attention": (C.c_int, [P, C.c_int, P, P, P, C.c_int, C.c_int, P]),
    "spx_engine_shift_kv": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "spx_engine_ensure_kv_room": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "spx_engine_destroy": (C.c_int, [P]),
    "spx_lookup_draft": (C.c_int, [P, C.c_int, C.c_int, P, C.c_int, C.c_int, C.c_int, P, P]),
    "spx_engine_generate": (C.c_int, [P, P, C.c_int, C.c_int, P, P, P]),
    "spx_sampler_create": (C.c_int, [P, P, C.c_int, C.POINTER(P)]),
    "spx_sampler_destroy": (C.c_int, [P]),
    "spx_sampler_reseed": (C.c_int, [P, C.c_uint64]),
    "spx_sample": (C.c_int, [P, P, C.c_float, P, C.c_int, C.c_int, C.c_int, P]),
    "spx_sample_verify": (C.c_int, [P, P, I64, C.c_int, C.c_float, P, C.c_int, P, C.c_int, C.c_int, C.c_int, P, P]),
    "spx_engine_set_sampler": (C.c_int, [P, P]),
    "spx_engine_set_draft": (C.c_int, [P, P]),
    "spx_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "spx_gguf_close": (C.c_int, [P]),
    "spx_gguf_info": (C.c_int, [P, P, P, P, P, P]),
    "spx_gguf_tensor": (C.c_int, [P, I64, P, P, P, P, P]),
    "spx_gguf_find": (I64, [P, C.c_char_p]),
    "spx_gguf_meta_type": (C.c_int, [P, C.c_char_p]),
    "spx_gguf_meta_index": (C.c_int, [P, C.c_char_p, P]),
    "spx_gguf_meta_f32": (C.c_int, [P, C.c_char_p, P]),
    "spx_gguf_meta_bool": (C.c_int, [P, C.c_char_p, P]),
    "spx_gguf_meta_str": (C.c_int, [P, C.c_char_p, P]),
    "spx_gguf_meta_array": (C.c_int, [P, C.c_char_p, P, P]),
    "spx_gguf_vocab_size": (I64, [P]),
    "spx_gguf_token": (C.c_char_p, [P, I64]),
    "spx_gguf_config": (C.c_int, [P, P]),
    "spx_gguf_stop_ids": (C.c_int, [P, P, C.c_int, P]),
    "spx_gguf_think_ids": (C.c_int, [P, P, P]),
    "spx_gguf_check": (C.c_int, [P]),
    "spx_engine_load_gguf": (C.c_int, [P, P, C.c_int, C.c_float, C.POINTER(P)]),
    "spx_spec_create": (P, [C.c_int]),
    "spx_spec_clone": (P, [P]),
    "spx_spec_destroy": (None, [P]),
    "spx_spec_class": (C.c_int, [C.c_int]),
    "spx_spec_accept_rate": (C.c_double, [P, C.c_int]),
    "spx_spec_best_len": (C.c_int, [P, C.c_int, C.c_int]),
    "spx_spec_reset_rates": (None, [P]),
    "spx_spec_record_draft": (C.c_int, [P, C.c_int, C.c_int, C.c_int]),
    "spx_spec_record_step": (None, [P, C.c_uint64]),
    "spx_spec_record_verify": (None, [P, C.c_int, C.c_uint64]),
    "spx_engine_decode": (C.c_int, [P, C.c_int32, C.c_int, C.c_int, P]),
    "spx_engine_profile": (C.c_int, [P, C.c_int]),
    "spx_engine_profile_read": (C.c_int, [P, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_int64), C.POINTER(C.c_double), C.POINTER(C.c_double)]),
}


def load():
    """Loads libspx.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise SpxError(f"{LIB_PATH} is missing: run `python -m spindle_amd.build` (or __graft_entry__.build())")
    lib_ = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib_, name)
        f.restype = res
        f.argtypes = args
    _lib = lib_
    return _lib


class _Lazy:
    def __getattr__(self, name):
        return getattr(load(), name)


lib = _Lazy()


def check(rc):
    if rc != 0:
        msg = load().spx_last_error()
        raise SpxError(msg.decode() if msg else f"spx error {rc}")
    return rc
