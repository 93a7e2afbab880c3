"""ctypes binding of libopenmini_qmm.so (C-ABI in include/openmini_qmm.h).

The library is the only compute path: if it is missing this module raises, there
is no CPU fallback.  Build it with `python openmini-v1_amd/build.py`.
"""
from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "libopenmini_qmm.so")

OK = 0
ERR_MEMORY = -1
ERR_INVALID_PARAM = -2
ERR_MODEL_LOAD = -3
ERR_INFERENCE = -4
ERR_UNSUPPORTED = -5
ERR_HIP = -10
ERR_INSUFFICIENT_DATA = -11
ERR_NOT_FOUND = -12

Q4_0 = 2
Q8_0 = 7


class WeightInfo(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("n_rows", ctypes.c_int64),
        ("k_cols", ctypes.c_int64),
        ("blocks_per_row", ctypes.c_int64),
        ("gguf_bytes", ctypes.c_size_t),
        ("device_bytes", ctypes.c_size_t),
    ]


class GgufHeader(ctypes.Structure):
    _fields_ = [
        ("version", ctypes.c_uint32),
        ("dialect", ctypes.c_int32),
        ("tensor_count", ctypes.c_uint64),
        ("metadata_kv_count", ctypes.c_uint64),
        ("distinct_tensors", ctypes.c_uint64),
        ("distinct_keys", ctypes.c_uint64),
        ("alignment", ctypes.c_uint32),
        ("file_size", ctypes.c_uint64),
    ]


class GgufTensorInfo(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("n_dims", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * 8),
        ("offset", ctypes.c_uint64),
        ("n_elements", ctypes.c_uint64),
        ("data_size", ctypes.c_uint64),
    ]


_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# void (*)(int level, const char* text, void* user_data)
LOG_CALLBACK = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p)
LOG_ERROR = 3

# name -> (restype, argtypes); mirrors include/openmini_qmm.h one to one.
SIGNATURES = {
    "openmini_qmm_version": (ctypes.c_char_p, []),
    "openmini_qmm_init": (_i, [_i]),
    "openmini_qmm_last_error": (ctypes.c_char_p, []),
    "openmini_qmm_set_log_callback": (_i, [LOG_CALLBACK, _p]),
    "openmini_qmm_is_available": (_i, []),
    "openmini_qmm_device_info": (_i, [ctypes.c_char_p, _sz]),
    "openmini_qmm_required_bytes": (_i, [_i, _sz, ctypes.POINTER(_sz)]),
    "openmini_qmm_estimate_memory_usage": (_sz, [_i, _sz]),
    "openmini_qmm_upload": (_i, [_i, _p, _sz, _i64, _i64, ctypes.POINTER(_p)]),
    "openmini_qmm_upload_device": (_i, [_i, _p, _sz, _i64, _i64, _p, ctypes.POINTER(_p)]),
    "openmini_qmm_weight_device_bytes": (_i, [_i, _i64, _i64, ctypes.POINTER(_sz)]),
    "openmini_qmm_upload_device_into": (_i, [_i, _p, _sz, _i64, _i64, _p, _sz, _p, ctypes.POINTER(_p)]),
    "openmini_qmm_free_weight": (None, [_p]),
    "openmini_qmm_weight_info": (_i, [_p, ctypes.POINTER(WeightInfo)]),
    "openmini_qmm_gemv": (_i, [_p, _p, _p, _i64, _p]),
    "openmini_qmm_gemm_bf16": (_i, [_p, _p, _p, _i64, _p]),
    "openmini_qmm_gemm_f32_workspace_bytes": (_sz, [_i64, _i64]),
    "openmini_qmm_gemm_launch_shape": (_i, [_p, _i64, _i]),
    "openmini_qmm_gemm_min_rows": (_i64, [_p]),
    "openmini_qmm_gemm_f32": (_i, [_p, _p, _p, _i64, _p, _sz, _p]),
    "openmini_qmm_gemv_multi": (_i, [ctypes.POINTER(_p), _i, _p, ctypes.POINTER(_p), _i64, _p]),
    "openmini_qmm_ffn_gate_up": (_i, [_p, _p, _p, _p, _i64, _p]),
    "openmini_qmm_ffn_gate_up_bf16": (_i, [_p, _p, _p, _p, _i64, _p]),
    "openmini_qmm_ffn_gate_up_f32": (_i, [_p, _p, _p, _p, _i64, _p, _sz, _p]),
    "openmini_qmm_linear_host": (_i, [_p, _p, _p, _i64]),
    "openmini_qmm_linear_host_noalloc": (_i, [_p, _p, _p, _i64]),
    "openmini_qmm_dequant_weight": (_i, [_p, _p, _p]),
    "openmini_qmm_dequantize_device": (_i, [_i, _p, _sz, _sz, _p, _p, ctypes.POINTER(_sz)]),
    "openmini_qmm_dequantize": (_i, [_i, _p, _sz, _sz, _p, ctypes.POINTER(_sz)]),
    "openmini_qmm_dequantize_any_device": (_i, [_i, _p, _sz, _sz, _p, _p]),
    "openmini_qmm_dequantize_any": (_i, [_i, _p, _sz, _sz, _p]),
    "openmini_qmm_gguf_open": (_i, [ctypes.c_char_p, _i, ctypes.POINTER(_p)]),
    "openmini_qmm_gguf_close": (None, [_p]),
    "openmini_qmm_gguf_header": (_i, [_p, ctypes.POINTER(GgufHeader)]),
    "openmini_qmm_gguf_tensor_name": (_i, [_p, _sz, ctypes.c_char_p, _sz]),
    "openmini_qmm_gguf_tensor_info": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(GgufTensorInfo)]),
    "openmini_qmm_gguf_tensor_data": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(_p), ctypes.POINTER(_sz)]),
    "openmini_qmm_gguf_meta_key": (_i, [_p, _sz, ctypes.c_char_p, _sz]),
    "openmini_qmm_gguf_meta_type": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(_i), ctypes.POINTER(ctypes.c_uint64)]),
    "openmini_qmm_gguf_get_u32": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]),
    "openmini_qmm_gguf_get_u64": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "openmini_qmm_gguf_get_f32": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
    "openmini_qmm_gguf_get_string": (_i, [_p, ctypes.c_char_p, ctypes.c_char_p, _sz, ctypes.POINTER(_sz)]),
    "openmini_qmm_gguf_upload_weight": (_i, [_p, ctypes.c_char_p, _p, ctypes.POINTER(_p)]),
    "openmini_qmm_gguf_dequantize_tensor": (_i, [_p, ctypes.c_char_p, _p, _p]),
    "openmini_qmm_malloc": (_i, [ctypes.POINTER(_p), _sz]),
    "openmini_qmm_free": (_i, [_p]),
    "openmini_qmm_memcpy_h2d": (_i, [_p, _p, _sz, _p]),
    "openmini_qmm_memcpy_d2h": (_i, [_p, _p, _sz, _p]),
    "openmini_qmm_memset": (_i, [_p, _i, _sz, _p]),
    "openmini_qmm_stream_create": (_i, [ctypes.POINTER(_p)]),
    "openmini_qmm_stream_destroy": (_i, [_p]),
    "openmini_qmm_stream_synchronize": (_i, [_p]),
    "openmini_qmm_stream_copy": (_i, [_p, _p, _sz, _p]),
    "openmini_qmm_stream_read": (_i, [_p, _sz, _p, _p]),
    "openmini_qmm_gemm_ceiling": (_i, [_i, _i64, _i64, _i64, _p, _p]),
    "openmini_qmm_soa_bytes": (_i, [_i, _sz, _sz, ctypes.POINTER(_sz)]),
    "openmini_qmm_convert_to_soa_device": (_i, [_i, _p, _sz, _sz, _p, _p]),
    "openmini_qmm_convert_to_soa": (_i, [_i, _p, _sz, _sz, _p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python openmini-v1_amd/build.py` "
                "(the HIP library is the only compute path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().openmini_qmm_last_error()
    return msg.decode() if msg else ""


class QmmError(RuntimeError):
    """A failing C-ABI call: `.status` is the openmini_qmm_status_t value."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


def check(status: int) -> None:
    if status != OK:
        raise QmmError(status, last_error())
