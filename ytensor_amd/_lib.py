"""ctypes binding of libythip.so (include/ythip.h).

The library is loaded from this package directory only. If it is missing the
import fails loudly: there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libythip.so")

F32, F16, BF16 = 0, 1, 2
MASK_NONE, MASK_CAUSAL, MASK_BOOL, MASK_DIAG = 0, 1, 2, 3

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_LP = ctypes.POINTER(ctypes.c_int64)

YT_RAW = -1
YTHIP_EINVAL, YTHIP_EUNSUPPORTED, YTHIP_EIO, YTHIP_EFORMAT, YTHIP_ENOTFOUND = -1, -2, -3, -4, -5


class YtTensorInfo(ctypes.Structure):
    """struct ythip_yt_tensor_info (include/ythip.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_char_p), ("tensor_type", ctypes.c_char_p),
                ("compress", ctypes.c_char_p), ("type_size", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.POINTER(ctypes.c_int32)), ("data_offset", ctypes.c_uint64),
                ("compressed_size", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class YtTensor(ctypes.Structure):
    """struct ythip_yt_tensor (include/ythip.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("dtype_name", ctypes.c_char_p),
                ("type_size", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.POINTER(ctypes.c_int32)), ("data", ctypes.c_void_p)]


_U64 = ctypes.c_uint64

# Every symbol include/ythip.h declares, with its ctypes signature.
SIGNATURES = {
    "ythip_abi_version": (_I, []),
    "ythip_last_error": (ctypes.c_char_p, []),
    "ythip_gemm": (_I, [_I, _I, _I, _I, _I, _I, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _F, _F, _P]),
    "ythip_attn_prefill": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P, _LP, _P, _LP, _P, _LP, _P, _LP,
                                _F, _I, _P, _L, _P, _L, _L, _P]),
    "ythip_attn_prefill_workspace_size": (ctypes.c_size_t, [_I, _I]),
    "ythip_attn_sdpa_workspace_size": (ctypes.c_size_t, [_I, _I, _I, _I, _I]),
    "ythip_attn_prefill_ws": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P, _LP, _P, _LP, _P, _LP, _P, _LP,
                                   _F, _I, _P, _L, _P, _L, _L, _P, ctypes.c_size_t, _P]),
    "ythip_attn_math_workspace_size": (ctypes.c_size_t, [_I, _I, _I, _I, _I]),
    "ythip_attn_math": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P, _LP, _P, _LP, _P, _LP, _P, _LP,
                             _F, _I, _P, _L, _P, _L, _L, _P, ctypes.c_size_t, _P]),
    "ythip_gemm_masked_workspace_size": (ctypes.c_size_t, [_I, _I, _I]),
    "ythip_gemm_masked": (_I, [_I, _I, _I, _I, _I, _I, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _F, _F,
                               _I, _P, _L, _I, _F, _P, ctypes.c_size_t, _P]),
    "ythip_attn_decode_workspace_size": (ctypes.c_size_t, [_I, _I, _I, _I]),
    "ythip_attn_decode_splits": (_I, [_I, _I, _I]),
    "ythip_attn_decode_noalloc_max_bytes": (ctypes.c_size_t, []),
    "ythip_attn_decode_noalloc": (_I, [_I, _I, _I, _I, _I, _I, _P, _LP, _P, _P, _LP, _P, _P, _LP, _F, _P]),
    "ythip_attn_decode_rope": (_I, [_I, _I, _I, _I, _I, _I, _P, _L, _P, _P, _F, _P, _P, _L, _I, _P, _P, _P, _LP, _P,
                                    _LP, _F, _P, ctypes.c_size_t, _P]),
    "ythip_attn_decode": (_I, [_I, _I, _I, _I, _I, _I, _P, _LP, _P, _P, _LP, _P, _P, _LP, _F, _P,
                               ctypes.c_size_t, _P]),
    "ythip_rmsnorm_rope": (_I, [_I, _I, _I, _I, _I, _I, _P, _L, _P, _P, _F, _P, _P, _L, _I, _I,
                                _P, _LP, _P, _LP, _P, _LP, _I, _I, _P, _P]),
    "ythip_rms_norm": (_I, [_I, _I, _I, _I, _P, _L, _P, _F, _P, _L, _P]),
    "ythip_rms_norm_strided": (_I, [_I, _I, _I, _I, _P, _L, _L, _P, _F, _P, _L, _L, _P]),
    "ythip_silu_mul": (_I, [_I, _I, _I, _I, _P, _L, _P, _L, _P]),
    "ythip_embedding": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _L, _P]),
    "ythip_add_bias": (_I, [_I, _I, _I, _P, _L, _P, _P]),
    "ythip_argmax_step": (_I, [_I, _P, _P, _P, _P, _P]),
    "ythip_gemv_fused": (_I, [_I, _I, _I, _I, _I, _I, _P, _L, _P, _F, _P, _L, _P, _L, _F, _F, _P, _P]),
    "ythip_gemv_swiglu": (_I, [_I, _I, _I, _I, _I, _P, _L, _P, _F, _P, _L, _P, _L, _P]),
    "ythip_gemv_attn_merge": (_I, [_I, _I, _I, _I, _I, _I, _I, _P, _L, _P, _L, _P, _L, _F, _F, _P, _I, _P]),
    "ythip_argmax_finish": (_I, [_P, _I, _P, _P, _P, _P]),
    "ythip_rope_tables": (_I, [_I, _I, _F, _P, _P]),
    "ythip_yt_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "ythip_yt_close": (_I, [_P]),
    "ythip_yt_count": (_I, [_P]),
    "ythip_yt_metadata": (ctypes.c_char_p, [_P]),
    "ythip_yt_find": (_I, [_P, ctypes.c_char_p]),
    "ythip_yt_info": (_I, [_P, _I, ctypes.POINTER(YtTensorInfo)]),
    "ythip_yt_load": (_I, [_P, _I, _P, _I, _U64, _P]),
    "ythip_yt_load_many": (_I, [_P, _I, _P, _P, _P, _P, _P]),
    "ythip_yt_sync": (_I, [_P]),
    "ythip_convert_host": (_I, [_I, _I, _P, _P, _L]),
    "ythip_yt_save": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(YtTensor), ctypes.c_char_p, _I, _P]),
}


class YthipError(RuntimeError):
    """A non-zero status from libythip (argument error or HIP error)."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is not built; run `python -m ytensor_amd.build` (hipcc, gfx950). "
            "ytensor_amd has no CPU fallback.")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError here = the library lacks a declared symbol
        fn.restype = res
        fn.argtypes = args
    return lib


_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = load()
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().ythip_last_error().decode(errors="replace")
        raise YthipError(f"{what} failed with status {status}: {msg}")


def i64array(vals) -> ctypes.Array:
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])
