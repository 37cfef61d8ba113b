"""ytensor_amd — MI355X (gfx950) back end for YTensor's GEMM and attention hot path.

The product is libythip.so (C ABI in include/ythip.h; HIP kernels in csrc/).
This package loads it through ctypes and exposes torch-facing operators that
mirror yt::function (see ops.py). Every operator loads the library on first
use and fails loudly when it has not been built: there is no CPU fallback.
"""
from ._lib import YthipError, lib, LIB_PATH  # noqa: F401
from . import io  # noqa: F401  (yt::io: .yt checkpoints to and from device memory)
from .ops import (  # noqa: F401
    argmax_finish,
    argmax_step,
    decode_attention,
    embedding,
    gemm,
    gemm_masked,
    gemv_attn_merge,
    gemv_fused,
    gemv_swiglu,
    linear,
    masked_matmul,
    matmul,
    rms_norm,
    rms_norm_rope,
    scaled_dot_product_attention,
    silu_mul,
)


def load():
    """Load libythip.so now; raises ImportError if it is missing and
    AttributeError if it lacks a symbol that include/ythip.h declares."""
    return lib()


__all__ = [
    "YthipError", "lib", "gemm", "matmul", "linear", "scaled_dot_product_attention",
    "decode_attention", "rms_norm", "rms_norm_rope", "silu_mul", "embedding", "argmax_step",
    "gemv_fused", "gemv_swiglu", "gemv_attn_merge", "argmax_finish", "io", "masked_matmul", "gemm_masked",
]
