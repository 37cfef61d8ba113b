"""Write tests/golden/reference_math.npz from the COMPILED REFERENCE (oracle/_ref,
built from /root/reference by `make -C oracle ref`): outputs of
scaledDotProductAttention with sdpaBackend::MATH and FLASH_AVX2 (bool masks,
predicate masks, bias), YTensor::masked_matmul and avx2::sgemm_masked on small
seeded inputs. The inputs are regenerated from `cases()` (numpy seeds), so only
outputs are stored.

    python tests/golden/make_math_fixtures.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

# (name, H, Lq, Lkv, D, Dv, mask form, bias)
SDPA_CASES = [
    ("plain", 2, 7, 9, 16, 16, None, False),
    ("bool", 3, 12, 20, 32, 24, "bool", False),
    ("bool_bias", 2, 16, 16, 64, 64, "bool", True),
    ("causal_pred", 2, 10, 10, 16, 16, 0, False),
    ("offset_pred", 2, 6, 11, 16, 8, 5, True),
    ("neg_pred", 1, 9, 9, 8, 8, -3, False),
    ("long", 1, 40, 620, 16, 16, "bool", False),
]
GEMM_CASES = [  # (name, m, n, k, alpha, beta)
    ("g1", 13, 17, 32, 1.0, 0.0),
    ("g2", 40, 33, 100, 0.5, 2.0),
    ("g3", 7, 70, 16, 1.0, 1.0),
]


def sdpa_inputs(case):
    name, H, Lq, Lkv, D, Dv, mform, with_bias = case
    rng = np.random.default_rng(sum(map(ord, name)))
    Q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    K = rng.standard_normal((H, Lkv, D)).astype(np.float32)
    V = rng.standard_normal((H, Lkv, Dv)).astype(np.float32)
    mask, diag = None, None
    if mform == "bool":
        mask = rng.random((Lq, Lkv)) < 0.6
        mask[min(1, Lq - 1), :] = False  # one row with no visible key
    elif mform is not None:
        diag = int(mform)
    bias = rng.standard_normal((Lq, Lkv)).astype(np.float32) if with_bias else None
    return Q, K, V, mask, bias, diag


def gemm_inputs(case):
    name, m, n, k, alpha, beta = case
    rng = np.random.default_rng(sum(map(ord, name)) + 1000)
    A = rng.standard_normal((m, k)).astype(np.float32)
    B = rng.standard_normal((k, n)).astype(np.float32)
    C = rng.standard_normal((m, n)).astype(np.float32)
    mask = rng.random((m, n)) < 0.5
    return A, B, C, mask


def main() -> None:
    ref = oracle.reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libytref.so is not built (make -C oracle ref)")
    out = {}
    for case in SDPA_CASES:
        Q, K, V, mask, bias, diag = sdpa_inputs(case)
        out[f"math_{case[0]}"] = ref.sdpa_math(Q, K, V, 0.0, mask=mask, bias=bias, diag=diag)
        out[f"flash_{case[0]}"] = ref.sdpa_flash(Q, K, V, 0.0, mask=mask, bias=bias, diag=diag)
    for case in GEMM_CASES:
        A, B, C, mask = gemm_inputs(case)
        out[f"sgemm_masked_{case[0]}"] = ref.sgemm_masked(A, B, C.copy(), mask, case[4], case[5])
        out[f"masked_matmul_{case[0]}"] = ref.masked_matmul(A, B, mask=mask, value=-7.0)
        out[f"masked_matmul_diag_{case[0]}"] = ref.masked_matmul(A, B, diag=1, value=-1e9)
    np.savez(os.path.join(HERE, "reference_math.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
