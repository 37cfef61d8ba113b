"""Roofline probes for the headline bf16 GEMM (libythip_probe.so, built from
csrc/probe/ceiling.hip by ytensor_amd.build): the GEMM's MFMA stream on register
operands, and its global -> LDS operand stream alone. Measurement support for
bench.py and the tests; not part of the C ABI in include/ythip.h.

The library is loaded from this package directory only; if it is missing the
call fails loudly.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE_LIB_PATH = os.path.join(HERE, "libythip_probe.so")

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(PROBE_LIB_PATH):
            raise RuntimeError(f"{PROBE_LIB_PATH} is not built (python -m ytensor_amd.build)")
        lib = ctypes.CDLL(PROBE_LIB_PATH)
        P, I = ctypes.c_void_p, ctypes.c_int
        lib.ythip_probe_mfma.restype = I
        lib.ythip_probe_mfma.argtypes = [P, P, P, I, I, P]
        lib.ythip_probe_dma.restype = I
        lib.ythip_probe_dma.argtypes = [P, P, I, I, I, P, P]
        _lib = lib
    return _lib


def _stream(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def mfma_ceiling(A, B, out, workgroups: int, steps: int) -> None:
    """out[w] = bf16(steps * A[w] . B[w]^T) for every wave w of `workgroups`
    8-wave workgroups: A bf16 [W, 128, 64], B bf16 [W, 64, 64] ([n][k]), out
    bf16 [W, 128, 64], W = 8 * workgroups, all contiguous on the GPU."""
    import torch
    W = 8 * workgroups
    assert A.dtype == torch.bfloat16 and B.dtype == torch.bfloat16 and out.dtype == torch.bfloat16
    assert tuple(A.shape) == (W, 128, 64) and tuple(B.shape) == (W, 64, 64) and tuple(out.shape) == (W, 128, 64)
    assert A.is_contiguous() and B.is_contiguous() and out.is_contiguous()
    st = load().ythip_probe_mfma(A.data_ptr(), B.data_ptr(), out.data_ptr(), workgroups, steps, _stream(torch))
    if st != 0:
        raise RuntimeError(f"ythip_probe_mfma failed ({st})")


def dma_ceiling(A, B, out) -> None:
    """The GEMM's NN operand stream for A bf16 [M, K] and B bf16 [K, N]
    (row-major, M and N multiples of 256, K a multiple of 64, K >= 128) into
    LDS; out uint8 [tiles, 512, 16] receives each workgroup's per-thread sums of
    its final LDS contents (the last two k steps' A and B slices)."""
    import torch
    M, K = A.shape
    K2, N = B.shape
    assert K == K2 and A.dtype == torch.bfloat16 and B.dtype == torch.bfloat16
    assert A.is_contiguous() and B.is_contiguous() and out.is_contiguous()
    assert out.numel() * out.element_size() == (M // 256) * (N // 256) * 512 * 16
    st = load().ythip_probe_dma(A.data_ptr(), B.data_ptr(), M, N, K, out.data_ptr(), _stream(torch))
    if st != 0:
        raise RuntimeError(f"ythip_probe_dma failed ({st})")
