"""CPU: the oracle's restatements of the MATH attention backend and the masked
matmul, pinned to the compiled reference's outputs (tests/golden/
reference_math.npz, written by make_math_fixtures.py from
scaledDotProductAttention(MATH / FLASH_AVX2), YTensor::masked_matmul and
avx2::sgemm_masked) and to closed forms."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_math_fixtures as mf  # noqa: E402


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(HERE, "golden", "reference_math.npz"))


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _flash_oracle(orc, Q, K, V, mask, bias, diag):
    H, Lq, D = Q.shape
    Lkv = K.shape[1]
    if diag is not None:
        mask = np.arange(Lkv)[None, :] <= np.arange(Lq)[:, None] + diag
    out = np.stack([orc.flash_attention(Q[h], K[h], V[h], 1 / np.sqrt(np.float32(D)), mask, bias)
                    for h in range(H)])
    return out


@pytest.mark.parametrize("case", mf.SDPA_CASES, ids=[c[0] for c in mf.SDPA_CASES])
def test_sdpa_math_matches_reference_bit_exact(orc, gold, case):
    Q, K, V, mask, bias, diag = mf.sdpa_inputs(case)
    got = orc.sdpa_math(Q, K, V, 0.0, mask=mask, bias=bias, diag=diag)
    assert np.array_equal(_bits(got), _bits(gold[f"math_{case[0]}"]))


@pytest.mark.parametrize("case", mf.SDPA_CASES, ids=[c[0] for c in mf.SDPA_CASES])
def test_flash_oracle_matches_reference_predicate_and_bool_masks(orc, gold, case):
    """The reference's FLASH with a predicate functor equals the oracle's flash
    on the same mask written out as bytes (tile skipping changes no value)."""
    Q, K, V, mask, bias, diag = mf.sdpa_inputs(case)
    got = _flash_oracle(orc, Q, K, V, mask, bias, diag)
    assert np.array_equal(_bits(got), _bits(gold[f"flash_{case[0]}"]))


@pytest.mark.parametrize("case", mf.SDPA_CASES, ids=[c[0] for c in mf.SDPA_CASES])
def test_math_and_flash_agree(gold, case):
    m, f = gold[f"math_{case[0]}"], gold[f"flash_{case[0]}"]
    assert np.abs(m - f).max() <= 1e-5 * max(1.0, np.abs(f).max())


def test_sdpa_math_closed_forms(orc):
    rng = np.random.default_rng(3)
    H, Lq, Lkv, D = 2, 5, 8, 16
    Q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    K = rng.standard_normal((H, Lkv, D)).astype(np.float32)
    V = rng.standard_normal((H, Lkv, D)).astype(np.float32)
    # one visible key per row: the output is that key's value row
    mask = np.zeros((Lq, Lkv), bool)
    pick = [3, 0, 7, 7, 2]
    for i, j in enumerate(pick):
        mask[i, j] = True
    out = orc.sdpa_math(Q, K, V, 0.0, mask=mask)
    for i, j in enumerate(pick):
        np.testing.assert_allclose(out[:, i], V[:, j], rtol=0, atol=1e-6)
    # identical keys: uniform weights, the mean of the visible values
    Kc = np.repeat(K[:, :1], Lkv, axis=1)
    out = orc.sdpa_math(Q, Kc, V, 0.0, diag=Lkv - Lq)
    for i in range(Lq):
        vis = Lkv - Lq + i + 1
        np.testing.assert_allclose(out[:, i], V[:, :vis].mean(axis=1), rtol=1e-5, atol=1e-6)
    # no visible key in a row -> zeros; a predicate that hides everything -> all zeros
    mask[2] = False
    assert np.all(orc.sdpa_math(Q, K, V, 0.0, mask=mask)[:, 2] == 0)
    assert np.all(orc.sdpa_math(Q, K, V, 0.0, diag=-Lq - 1) == 0)


@pytest.mark.parametrize("case", mf.GEMM_CASES, ids=[c[0] for c in mf.GEMM_CASES])
def test_masked_matmul_matches_reference(orc, gold, case):
    A, B, C, mask = mf.gemm_inputs(case)
    name, m, n, k, alpha, beta = case
    got = orc.sgemm_masked(A, B, C.copy(), mask, alpha, beta)
    want = gold[f"sgemm_masked_{name}"]
    if (alpha, beta) == (1.0, 0.0) or (alpha, beta) == (0.5, 2.0):
        assert np.array_equal(_bits(got), _bits(want))
    else:  # the reference's full tiles continue the FMA chain from C; one rounding apart
        assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    assert np.array_equal(got[~mask], C[~mask])  # untouched where the mask is clear
    mm = orc.masked_matmul(A, B, mask=mask, value=-7.0)
    assert np.array_equal(_bits(mm), _bits(gold[f"masked_matmul_{name}"]))
    dg = orc.masked_matmul(A, B, diag=1, value=-1e9)
    assert np.array_equal(_bits(dg), _bits(gold[f"masked_matmul_diag_{name}"]))
    # integer-valued operands: the products are exact, so any order gives the same bits
    Ai = np.round(A * 4).astype(np.float32)
    Bi = np.round(B * 4).astype(np.float32)
    ref_int = (Ai.astype(np.float64) @ Bi.astype(np.float64)).astype(np.float32)
    mi = orc.masked_matmul(Ai, Bi, mask=mask, value=0.5)
    assert np.array_equal(mi[mask], ref_int[mask]) and np.all(mi[~mask] == 0.5)


def test_reference_live(orc, ref):
    """Where the reference is built: fresh random cases, bit for bit."""
    rng = np.random.default_rng(11)
    for (H, Lq, Lkv, D) in [(2, 33, 70, 64), (1, 128, 128, 128)]:
        Q = rng.standard_normal((H, Lq, D)).astype(np.float32)
        K = rng.standard_normal((H, Lkv, D)).astype(np.float32)
        V = rng.standard_normal((H, Lkv, D)).astype(np.float32)
        m = rng.random((Lq, Lkv)) < 0.7
        b = rng.standard_normal((Lq, Lkv)).astype(np.float32)
        for kw in (dict(), dict(mask=m, bias=b), dict(diag=Lkv - Lq), dict(diag=2, bias=b)):
            assert np.array_equal(_bits(orc.sdpa_math(Q, K, V, 0.0, **kw)), _bits(ref.sdpa_math(Q, K, V, 0.0, **kw)))
