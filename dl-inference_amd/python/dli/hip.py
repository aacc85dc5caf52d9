"""ctypes binding of libdli_hip.so (include/dli_hip.h).

This is what a non-C++ caller of the device layer binds: plain pointers, sizes and int status
codes. Tensors are passed as data pointers; every kernel call is asynchronous on `stream`
(torch's current stream by default).
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import hip_library_path

F32, I64, BF16, F16, I32 = 0, 1, 2, 3, 4
_TORCH_CODES = {torch.float32: F32, torch.int64: I64, torch.bfloat16: BF16, torch.float16: F16,
                torch.int32: I32}

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_float = ctypes.c_float
_size = ctypes.c_size_t

# name -> argument types (return type is int unless listed in _RESTYPES)
_SIGNATURES = {
    "dli_hip_available": [],
    "dli_hip_load_error": [],
    "dli_hip_last_error": [],
    "dli_hip_target_arch": [],
    "dli_hip_device_count": [ctypes.POINTER(_int)],
    "dli_hip_get_device": [ctypes.POINTER(_int)],
    "dli_hip_set_device": [_int],
    "dli_hip_compute_units": [ctypes.POINTER(_int)],
    "dli_hip_module_load": [_c_void_p, _size, ctypes.POINTER(_c_void_p)],
    "dli_hip_code_object": [ctypes.c_char_p, ctypes.POINTER(_c_void_p), ctypes.POINTER(_size)],
    "dli_hip_module_get_function": [_c_void_p, ctypes.c_char_p, ctypes.POINTER(_c_void_p)],
    "dli_hip_module_unload": [_c_void_p],
    "dli_hip_launch": [_c_void_p, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                       ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, _c_void_p,
                       ctypes.POINTER(_c_void_p)],
    "dli_hip_malloc": [_size, ctypes.POINTER(_c_void_p)],
    "dli_hip_free": [_c_void_p],
    "dli_hip_memcpy": [_c_void_p, _c_void_p, _size, _int],
    "dli_hip_memcpy_async": [_c_void_p, _c_void_p, _size, _int, _c_void_p],
    "dli_hip_stream_synchronize": [_c_void_p],
    "dli_hip_device_synchronize": [],
    "dli_hip_event_create": [ctypes.POINTER(_c_void_p)],
    "dli_hip_event_record": [_c_void_p, _c_void_p],
    "dli_hip_event_synchronize": [_c_void_p],
    "dli_hip_event_elapsed_ms": [_c_void_p, _c_void_p, ctypes.POINTER(_float)],
    "dli_hip_event_destroy": [_c_void_p],
    "dli_hip_add": [_int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "dli_hip_mul": [_int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "dli_hip_silu": [_int, _c_void_p, _c_void_p, _i64, _c_void_p],
    "dli_hip_relu": [_int, _c_void_p, _c_void_p, _i64, _c_void_p],
    "dli_hip_rms_norm": [_int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _float, _c_void_p],
    "dli_hip_embedding": [_int, _int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                          _c_void_p],
    "dli_hip_softmax": [_int, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "dli_hip_transpose2d": [_int, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "dli_hip_permute_0213": [_int, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _c_void_p],
    "dli_hip_batch_norm2d": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                             _c_void_p, _i64, _i64, _i64, _float, _c_void_p],
    "dli_hip_max_pool2d": [_int, _c_void_p, _c_void_p] + [_i64] * 12 + [_c_void_p],
    "dli_hip_conv2d": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p] + [_i64] * 13
    + [_c_void_p],
    "dli_hip_conv2d_act": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p] + [_i64] * 13
    + [_int, _c_void_p, _size, _c_void_p],
    "dli_hip_conv2d_workspace": [_int] + [_i64] * 7,
    "dli_hip_linear": [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                       _c_void_p],
    "dli_hip_linear_act": [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                           _i64, _int, _c_void_p, _size, _c_void_p],
    "dli_hip_matmul": [_int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p],
    "dli_hip_rotary": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]
    + [_i64] * 8 + [_c_void_p, _int, _c_void_p],
    "dli_hip_attention": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p] + [_i64] * 6
    + [_int, _float, _c_void_p],
    "dli_hip_attention_bshd": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p] + [_i64] * 6
    + [_int, _float, _c_void_p],
    "dli_hip_kv_append": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]
    + [_i64] * 7 + [_c_void_p, _int, _c_void_p],
    "dli_hip_linear_workspace": [_int, _i64, _i64, _i64],
    "dli_hip_paged_attention_workspace": [_i64] * 5,
    "dli_hip_paged_attention": [_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p]
    + [_i64] * 8 + [_c_void_p, _int, _int, _float, _int, _c_void_p, _size, _c_void_p],
    "dli_hip_argmax": [_int, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "dli_hip_splitk_workspace": [_i64, _i64, _int],
    "dli_hip_qkv_rope_append": [_c_void_p] * 6 + [_i64, _c_void_p, _int] + [_c_void_p] * 4
    + [_i64] * 7 + [_float, _c_void_p],
    "dli_hip_qkv_rope_append_workspace": [_i64] * 5,
    "dli_hip_qkv_rope_append_ws": [_c_void_p] * 6 + [_i64, _c_void_p, _int] + [_c_void_p] * 4
    + [_i64] * 7 + [_float, _c_void_p, _size, _c_void_p],
    "dli_hip_linear_residual": [_c_void_p] * 5 + [_i64] * 3 + [_int, _c_void_p, _size, _c_void_p],
    "dli_hip_linear_residual_norm": [_c_void_p] * 7 + [_i64] * 3
    + [_float, _int, _c_void_p, _size, _c_void_p],
    "dli_hip_gate_up_silu": [_c_void_p] * 4 + [_i64] * 3 + [_float, _c_void_p],
    "dli_hip_qkv_rope_heads": [_c_void_p] * 5 + [_i64] + [_c_void_p] * 3 + [_i64] * 7
    + [_c_void_p],
    "dli_hip_lm_head_argmax_workspace": [_i64, _i64],
    "dli_hip_lm_head_argmax": [_c_void_p] * 3 + [_int, _c_void_p] + [_i64] * 3
    + [_c_void_p, _size, _c_void_p],
    "dli_hip_lm_head_argmax_norm": [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _int,
                                    _c_void_p, _i64, _i64, _i64, _c_void_p, _size, _c_void_p],
    "dli_hip_lm_head_argmax_norm_noalloc": [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p,
                                            _int, _c_void_p, _i64, _i64, _i64, _c_void_p],
    "dli_hip_decoder_stack_workspace": [_int] + [_i64] * 7 + [_int, _int],
    "dli_hip_decoder_stack": [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _int, _c_void_p,
                              _c_void_p] + [_i64] * 9 + [_float, _int, _c_void_p, _size,
                                                         _c_void_p, _c_void_p, _c_void_p],
    "dli_hip_decoder_stack_status": [_c_void_p, ctypes.POINTER(_int), _c_void_p],
    "dli_hip_stream_is_capturing": [_c_void_p, ctypes.POINTER(_int)],
}
_RESTYPES = {
    "dli_hip_load_error": ctypes.c_char_p,
    "dli_hip_last_error": ctypes.c_char_p,
    "dli_hip_target_arch": ctypes.c_char_p,
    "dli_hip_linear_workspace": _size,
    "dli_hip_conv2d_workspace": _size,
    "dli_hip_paged_attention_workspace": _size,
    "dli_hip_splitk_workspace": _size,
    "dli_hip_qkv_rope_append_workspace": _size,
    "dli_hip_lm_head_argmax_workspace": _size,
    "dli_hip_decoder_stack_workspace": _size,
}


class DecoderLayer(ctypes.Structure):
    """DliDecoderLayer: device pointers of one decoder layer (include/dli_hip.h)."""
    _fields_ = [(name, _c_void_p) for name in (
        "input_norm", "w_qkv", "b_qkv", "w_o", "post_norm", "w_gate_up", "w_down", "key_pool",
        "value_pool", "block_table")]


class StackOptions(ctypes.Structure):
    """DliStackOptions: per-call options of dli_hip_decoder_stack (include/dli_hip.h)."""
    _fields_ = [("attention_splits", _int), ("trace", _c_void_p), ("trace_layers", _int),
                ("token_ids", _c_void_p), ("token_ids_dtype", _int), ("embedding", _c_void_p),
                ("vocab", ctypes.c_int64)]


class HipError(RuntimeError):
    pass


def declared_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def load(path: str | None = None) -> ctypes.CDLL:
    lib = ctypes.CDLL(path or hip_library_path(), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, _int)
    return lib


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def dtype_code(t: torch.Tensor) -> int:
    return _TORCH_CODES[t.dtype]


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


def current_stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def call(name: str, *args) -> int:
    """Calls an entry point and raises HipError with dli_hip_last_error() on failure."""
    rc = getattr(lib(), name)(*args)
    if isinstance(rc, int) and rc != 0 and name not in _RESTYPES:
        raise HipError(f"{name} failed ({rc}): {lib().dli_hip_last_error().decode()}")
    return rc
