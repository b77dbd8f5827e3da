"""ctypes binding of libramforge_hip.so (the C ABI in include/ramforge_hip.h).

The shared library is built in-tree by ``ramforge_amd.build`` and loaded from
the package directory.  There is no CPU fallback: if the library is missing,
importing this module raises, so nothing can silently run without the HIP
kernels.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_NAME = "libramforge_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


class RamforgeError(RuntimeError):
    """Error returned by the C ABI; ``code`` is the RF_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


RF_OK = 0
RF_ERR_INVALID = 1
RF_ERR_BUDGET = 2
RF_ERR_IO = 5
READ_FN = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p)
RF_ERR_HIP = 3
RF_ERR_UNSUPPORTED = 4
RF_ALL_ROWS = 0xFFFFFFFFFFFFFFFF

_vp = C.c_void_p
_u32, _u64, _i32, _i64 = C.c_uint32, C.c_uint64, C.c_int32, C.c_int64
_f32, _f64 = C.c_float, C.c_double
_fp = C.c_void_p  # device float* passed as raw addresses


class ModelConfig(C.Structure):
    """rf_model_config — LlamaConfig (runtime/src/model.rs:26-37)."""

    _fields_ = [
        ("vocab_size", _u64),
        ("context_length", _u64),
        ("embedding_length", _u64),
        ("block_count", _u64),
        ("feed_forward_length", _u64),
        ("head_count", _u64),
        ("head_count_kv", _u64),
        ("head_dim", _u64),
        ("rms_eps", _f32),
        ("rope_freq_base", _f32),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "rf_last_error": (C.c_size_t, [C.c_char_p, C.c_size_t]),
    "rf_version": (C.c_char_p, []),
    "rf_ctx_create": (_i32, [_i32, _u64, C.POINTER(_vp)]),
    "rf_ctx_destroy": (None, [_vp]),
    "rf_ctx_synchronize": (_i32, [_vp]),
    "rf_ctx_reserve": (_i32, [_vp, _u64, _u64, _u64, _i32]),
    "rf_attention_workspace_bytes": (_u64, [_u64, _u32, _u32, _u32]),
    "rf_matmul_workspace_bytes": (_u64, [_u64, _u64, _u64]),
    "rf_ctx_compute_stream": (_vp, [_vp]),
    "rf_ctx_copy_stream": (_vp, [_vp]),
    "rf_ctx_device_info": (_i32, [_vp, C.c_char_p, C.c_size_t, C.POINTER(_i32)]),
    "rf_vram_alloc": (_i32, [_vp, C.c_char_p, _u64, C.POINTER(_vp)]),
    "rf_vram_release": (_i32, [_vp, C.c_char_p]),
    "rf_vram_rename_prefix": (_i32, [_vp, C.c_char_p, C.c_char_p]),
    "rf_vram_charge": (_i32, [_vp, C.c_char_p, C.POINTER(_u64)]),
    "rf_vram_used": (_u64, [_vp]),
    "rf_vram_total": (_u64, [_vp]),
    "rf_vram_peak": (_u64, [_vp]),
    "rf_pinned_alloc": (_i32, [_vp, _u64, C.POINTER(_vp)]),
    "rf_pinned_free": (_i32, [_vp, _vp]),
    "rf_upload_async": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "rf_upload": (_i32, [_vp, _vp, _vp, _u64]),
    "rf_download": (_i32, [_vp, _vp, _vp, _u64]),
    "rf_memset": (_i32, [_vp, _vp, _i32, _u64]),
    "rf_copy_async": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "rf_packed_supported": (_i32, [_u32, _u64]),
    "rf_pack_weights": (_i32, [_vp, _u32, _vp, _u64, _u64, _u64, _vp, _u64, _vp]),
    "rf_matvec_packed": (_i32, [_vp, _u32, _vp, _u64, _u64, _u64, _fp, _fp, _u64, _u64, _vp]),
    "rf_matmul_packed": (_i32, [_vp, _u32, _vp, _u64, _u64, _u64, _fp, _u64, _fp, _vp]),
    "rf_event_create": (_i32, [_vp, C.POINTER(_vp)]),
    "rf_event_destroy": (_i32, [_vp, _vp]),
    "rf_event_record": (_i32, [_vp, _vp, _vp]),
    "rf_stream_wait_event": (_i32, [_vp, _vp, _vp]),
    "rf_event_elapsed_ms": (_i32, [_vp, _vp, _vp, C.POINTER(_f32)]),
    "rf_event_synchronize": (_i32, [_vp, _vp]),
    "rf_matvec": (_i32, [_vp, _u32, _vp, _u64, _u64, _u64, _fp, _fp, _u64, _u64, _vp]),
    "rf_matvec_cache": (_i32, [_vp, _u64]),
    "rf_matvec_cache_forget": (_i32, [_vp, _vp, _u64]),
    "rf_matvec_cache_stats": (_i32, [_vp, C.POINTER(_u64), C.POINTER(_u64), C.POINTER(_u64), C.POINTER(_u64)]),
    "rf_dequantize_rows": (_i32, [_vp, _u32, _vp, _u64, _u64, _u64, _u64, _fp, _vp]),
    "rf_attention_decode": (_i32, [_vp, _fp, _fp, _fp, _fp, _fp, _u32, _u32, _u32, _u32, _fp, _vp]),
    "rf_attention_decode_noalloc": (_i32, [_vp, _fp, _fp, _fp, _fp, _fp, _u32, _u32, _u32, _u32, _fp, _vp]),
    "rf_rope": (_i32, [_vp, _fp, _fp, _u64, _u32, _u32, _u32, _f32, _vp]),
    "rf_rmsnorm": (_i32, [_vp, _fp, _fp, _u64, _f32, _fp, _vp]),
    "rf_add": (_i32, [_vp, _fp, _fp, _u64, _fp, _vp]),
    "rf_bias_add": (_i32, [_vp, _fp, _fp, _u64, _vp]),
    "rf_mul": (_i32, [_vp, _fp, _fp, _u64, _fp, _vp]),
    "rf_silu": (_i32, [_vp, _fp, _u64, _fp, _vp]),
    "rf_swiglu": (_i32, [_vp, _fp, _fp, _u64, _fp, _vp]),
    "rf_softmax": (_i32, [_vp, _fp, _u64, _vp]),
    "rf_argmax": (_i32, [_vp, _fp, _u64, _vp, _vp]),
    "rf_synth_blocks": (_i32, [_vp, _u32, _u64, _u64, _u64, _f64, _vp, _u64, _vp]),
    "rf_model_create": (_i32, [_vp, C.POINTER(ModelConfig), _u64, C.POINTER(_vp)]),
    "rf_model_create_growing": (_i32, [_vp, C.POINTER(ModelConfig), _u64, _u64, C.POINTER(_vp)]),
    "rf_model_destroy": (None, [_vp]),
    "rf_model_set_tensor": (_i32, [_vp, C.c_char_p, _u32, _u64, _u64, _vp, _u64]),
    "rf_model_synth_tensor": (_i32, [_vp, C.c_char_p, _u32, _u64, _u64, _u64, _f64, _f32]),
    "rf_model_reset": (_i32, [_vp]),
    "rf_model_seq_len": (_u64, [_vp]),
    "rf_model_forward": (_i32, [_vp, _u32, _u64, _vp]),
    "rf_model_prefill": (_i32, [_vp, _vp, _u64, _vp]),
    "rf_model_set_prefill": (_i32, [_vp, _i32]),
    "rf_model_logits": (_i32, [_vp, _vp]),
    "rf_model_generate": (_i32, [_vp, _vp, _u64, _u64, _i64, _vp, C.POINTER(_u64)]),
    "rf_model_decode_steps": (_i32, [_vp, _u64]),
    "rf_model_read_tokens": (_i32, [_vp, _vp, _u64]),
    "rf_model_use_graph": (_i32, [_vp, _i32]),
    "rf_model_kv_growth": (_i32, [_vp, _u64]),
    "rf_model_set_reader": (_i32, [_vp, READ_FN, _vp, _u64]),
    "rf_model_set_read_ahead": (_i32, [_vp, _i32]),
    "rf_file_source_open": (_i32, [C.c_char_p, _u32, C.POINTER(_vp)]),
    "rf_file_source_close": (None, [_vp]),
    "rf_model_set_tensor_source": (_i32, [_vp, C.c_char_p, _u32, _u64, _u64, _u64, _u64]),
    "rf_model_read_stats": (_i32, [_vp, _vp]),
    "rf_model_set_persistent_policy": (_i32, [_vp, _i32]),
    "rf_model_persistent_streamed": (_i32, [_vp, _vp]),
    "rf_model_profile": (_i32, [_vp, _i32]),
    "rf_model_profile_read": (_i32, [_vp, _vp, _vp, _i32]),
    "rf_model_kv_capacity": (_i32, [_vp, _vp]),
    "rf_model_paths": (_i32, [_vp, _u64, _vp, _vp, _vp]),
    "rf_model_kernel_name": (_i32, [_vp, _u32, C.c_char_p, _u64]),
    "rf_model_host_bytes": (_i32, [_vp, C.POINTER(_u64)]),
    "rf_model_time_kernel": (_i32, [_vp, _u32, _u32, C.POINTER(_f32), C.POINTER(_u64), C.POINTER(_u64)]),
    "rf_tune_matvec_tile_bytes": (_u32, [_u32]),
    "rf_tune_matvec_kernel": (_i32, [_i32]),
    "rf_tune_matvec_digits": (_i32, [_i32]),
    "rf_tune_packed_inflight": (_i32, [_i32]),
    "rf_tune_attention_merge": (_i32, [_i32]),
    "rf_tune_attention_kernel": (_i32, [_i32]),
    "rf_tune_attention_single": (_i32, [_i32]),
    "rf_tune_prefill_attention": (_i32, [_i32]),
    "rf_tune_packed_weights": (_i32, [_i32]),
    "rf_model_enable_streaming": (_i32, [_vp, _u64]),
    "rf_model_residency_stats": (_i32, [_vp, C.POINTER(_u64)]),
    "rf_model_set_cache_policy": (_i32, [_vp, _i32]),
    "rf_model_set_stream_units": (_i32, [_vp, _i32]),
    "rf_capture_begin": (_i32, [_vp]),
    "rf_capture_end": (_i32, [_vp, C.POINTER(_vp)]),
    "rf_graph_replay": (_i32, [_vp, _vp, _u32, C.POINTER(_f32)]),
    "rf_graph_destroy": (_i32, [_vp, _vp]),
}

_LIB = None


def load() -> C.CDLL:
    """Load the in-tree library once (raises if it was not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the HIP library is required; there is no CPU fallback)"
            )
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def last_error() -> str:
    lib = load()
    buf = C.create_string_buffer(2048)
    lib.rf_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int) -> None:
    if rc != RF_OK:
        raise RamforgeError(rc, last_error())
