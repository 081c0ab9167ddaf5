"""ctypes bindings of libw8a8_mi355.so: the argument and return types of every entry point in include/w8a8_mi355.h.

Mirrors how the reference binds its libraries (vllm_turing/w8a8.py:27-35,49-55, vllm_turing/tailoverlap.py:48-54):
pointers as c_void_p, sizes and flags as c_int, the stream last, an int return code.
"""
import ctypes

from . import _build

_vp, _i, _l = ctypes.c_void_p, ctypes.c_int, ctypes.c_long

SIGNATURES = {
    "w8a8_gemv": [_vp] * 6 + [_i] * 6 + [_vp],
    "w8a8_mma": [_vp] * 6 + [_i] * 6 + [_vp],
    "w8a8_big": [_vp] * 5 + [_i] * 4 + [_vp],
    "w8a8_scaled_mm": [_vp] * 6 + [_i] * 6 + [_vp],
    "w8a8_scaled_mm_ws": [_vp] * 6 + [_i] * 6 + [_vp, _l, _vp],
    "w8a8_scaled_mm_ws_size": [_i] * 3,
    "w8a8_scaled_mm_noalloc": [_vp] * 6 + [_i] * 6 + [_vp],
    "w8a8_gemv_quant": [_vp, _l, _vp, _vp] + [_vp] * 4 + [_i] * 5 + [_vp],
    "w8a8_gemv_silu": [_vp] * 6 + [_i] * 6 + [_vp],
    "per_token_quant": [_vp] * 3 + [_i, _i, _l, _i, _vp],
    "silu_mul_quant": [_vp] * 3 + [_i] * 2 + [_vp],
    "silu_mul_quant_bf16": [_vp] * 3 + [_i] * 2 + [_vp],
    "w8a16_gemv": [_vp] * 5 + [_i] * 4 + [_vp],
    "w8a16_gemv_rows": [_vp] * 5 + [_i] * 4 + [_vp, _vp],
    "w8a16_gemv_rows_bounded": [_vp] * 5 + [_i] * 4 + [_vp, _i, _vp],
    "w8a16_mma": [_vp] * 5 + [_i] * 4 + [_vp],
    "ar8_quant": [_vp, _vp, _i, _vp],
    "ar8_dequant_sum": [_vp, _vp, _i, _vp],
    "ar8_dequant_sum_ranks": [_vp, _vp, _i, _i, _vp],
    "rms_norm_quant": [_vp] * 4 + [ctypes.c_float] + [_vp] * 2 + [_i] * 3 + [_vp],
    "w8a8_i32": [_vp] * 3 + [_i] * 4 + [_vp],
    "silu_table": [_vp, _i, _vp],
    "silu_mul_quant_path": [_vp] * 3 + [_i] * 4 + [_vp],
    "f32_to_16": [_vp, _vp, _l, _i, _vp],
    "hbm_read": [_vp, _i, _i, _vp, _vp],
}
RESTYPES = {"w8a8_scaled_mm_ws_size": _l}

_lib = None


def lib():
    """The loaded library with every signature set (built first if needed); raises if it cannot be loaded."""
    global _lib
    if _lib is None:
        L = _build.load()
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def stream_handle(device=None):
    """The current HIP stream of `device` as the void* the C ABI takes."""
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype):
    import torch
    if dtype == torch.float16:
        return 0
    if dtype == torch.bfloat16:
        return 1
    raise ValueError(f"unsupported activation / output dtype {dtype}: float16 or bfloat16")
