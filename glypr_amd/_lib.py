"""ctypes binding of libglypr_hip.so (the C ABI declared in include/glypr_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libglypr_hip.so")

GLYPR_OK = 0
GLYPR_ERR_INVALID_ARG = 1
GLYPR_ERR_SHAPE = 2
GLYPR_ERR_ALIGNMENT = 3
GLYPR_ERR_DEVICE = 4
GLYPR_ERR_HIP = 5
GLYPR_ERR_OOM = 6
GLYPR_ERR_RANGE = 7
GLYPR_ERR_UNSUPPORTED = 8
GLYPR_ERR_NOT_FOUND = 9
GLYPR_ERR_BUSY = 10

INT8_EXACT = 0
BF16_DEQUANT = 1
INT8_FMA = 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); every symbol of include/glypr_hip.h.
SIGNATURES = {
    "glypr_hip_last_error": (ctypes.c_char_p, []),
    "glypr_hip_abi_version": (_int, []),
    "glypr_hip_ctx_create": (_int, [_int, ctypes.POINTER(_vp)]),
    "glypr_hip_ctx_destroy": (_int, [_vp]),
    "glypr_hip_sync": (_int, [_vp, _vp]),
    "glypr_hip_ctx_reserve": (_int, [_vp, _i64]),
    "glypr_hip_q8_0_weight_create": (_int, [_vp, _vp, _i64, _i64, ctypes.POINTER(_vp)]),
    "glypr_hip_q8_0_weight_concat": (_int, [_vp, ctypes.POINTER(_vp), _int, ctypes.POINTER(_vp),
                                            ctypes.POINTER(_vp)]),
    "glypr_hip_q8_0_weight_view": (_int, [_vp, _i64, _i64, ctypes.POINTER(_vp)]),
    "glypr_hip_q8_0_weight_destroy": (_int, [_vp]),
    "glypr_hip_q8_0_weight_shape": (_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "glypr_hip_q8_0_dequantize": (_int, [_vp, _vp, _vp, _vp]),
    "glypr_hip_q8_0_quantize": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_q8_0_matmul": (_int, [_vp, _vp, _vp, _vp, _i64, _int, _vp]),
    "glypr_hip_q8_0_matmul_noalloc": (_int, [_vp, _vp, _vp, _vp, _i64, _int, _vp]),
    "glypr_hip_bf16_weight_create": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "glypr_hip_bf16_weight_destroy": (_int, [_vp]),
    "glypr_hip_bf16_matmul": (_int, [_vp, _vp, _vp, _vp, _i64, _vp]),
    "glypr_hip_rmsnorm": (_int, [_vp, _vp, _vp, _f32, _vp, _i64, _i64, _vp]),
    "glypr_hip_rmsnorm_q8_0_matmul": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _i64, _int, _vp]),
    "glypr_hip_geglu": (_int, [_vp, _vp, _vp, _vp, _i64, _vp]),
    "glypr_hip_mlp": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _int, _vp]),
    "glypr_hip_rmsnorm_mlp": (_int, [_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _int, _vp]),
    "glypr_hip_q8_0_embed_gather": (_int, [_vp, _vp, _vp, _i64, _f32, _vp, _vp]),
    "glypr_hip_pool_normalize": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "glypr_hip_quantize_binary": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_quantize_int8": (_int, [_vp, _vp, _i64, _vp, _vp]),
    "glypr_hip_hamming": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_binary_cosine": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_int8_dot": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_int8_cosine": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_attention": (_int, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _i64, _i64, _i64, _i64,
                                   _i64, _vp, _vp]),
    "glypr_hip_model_create": (_int, [_vp, _vp, ctypes.POINTER(_vp)]),
    "glypr_hip_model_set_tensor": (_int, [_vp, ctypes.c_char_p, _vp, _i64, _i64, _int]),
    "glypr_hip_model_finalize": (_int, [_vp]),
    "glypr_hip_model_embed": (_int, [_vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "glypr_hip_model_embed_batch": (_int, [_vp, _vp, _vp, _i64, _i64, _vp, _vp]),
    "glypr_hip_model_set_variant": (_int, [_vp, _int]),
    "glypr_hip_model_destroy": (_int, [_vp]),
    "glypr_gguf_open": (_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "glypr_gguf_close": (_int, [_vp]),
    "glypr_gguf_version": (_int, [_vp, ctypes.POINTER(ctypes.c_uint32),
                                  ctypes.POINTER(ctypes.c_uint32)]),
    "glypr_gguf_tensor_count": (_int, [_vp, ctypes.POINTER(_i64)]),
    "glypr_gguf_tensor_info": (_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.POINTER(_int), ctypes.POINTER(_int),
                                      ctypes.POINTER(_i64), ctypes.POINTER(_vp),
                                      ctypes.POINTER(_i64)]),
    "glypr_gguf_find_tensor": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_i64)]),
    "glypr_gguf_get_u64": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "glypr_gguf_get_f64": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "glypr_gguf_get_str": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
    "glypr_gguf_get_array": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_int),
                                    ctypes.POINTER(_i64)]),
    "glypr_gguf_get_array_u64": (_int, [_vp, ctypes.c_char_p, _i64,
                                        ctypes.POINTER(ctypes.c_uint64)]),
    "glypr_hip_model_load_gguf": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "glypr_hip_profile_enable": (_int, [_vp, _int]),
    "glypr_hip_profile_read": (_int, [_vp, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(_i64)]),
    "glypr_hip_kernel_name": (ctypes.c_char_p, [_int]),
}

KERNEL_COUNT = 21


class GlyprError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"glypr_hip error {code}: {msg}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Load libglypr_hip.so; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m glypr_amd.build` "
                "(glypr_amd has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return (lib().glypr_hip_last_error() or b"").decode()


def check(rc: int) -> None:
    if rc != GLYPR_OK:
        raise GlyprError(rc, last_error())
