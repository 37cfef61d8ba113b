"""CPU: the oracle (oracle/ytoracle.cpp) pinned three ways.

1. Golden fixtures written by the compiled reference (tests/golden/
   gen_golden.py): bit-exact equality for every fixture.
2. Live comparison with the compiled reference (oracle/_ref) where it was built.
3. Closed forms that a plausible mistake would break: identity/permutation
   and small-integer GEMMs, one visible key, Q = 0 gives the mean of the
   visible values, decode == last causal row, fp64 brute force, RMSNorm and
   RoPE formulas, the bf16/fp16 bit formulas.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import cases  # noqa: E402

import oracle  # noqa: E402

GOLD = os.path.join(HERE, "golden", "reference_small.npz")
GOLD_Q3 = os.path.join(HERE, "golden", "reference_qwen3_0p6b.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


# ---------------------------------------------------------------- fixtures

@pytest.mark.parametrize("seed", cases.RANDN_SEEDS)
def test_randn_matches_reference(orc, gold, seed):
    orc.seed(seed)
    x = orc.randn(cases.RANDN_N)
    assert bits_equal(x[:64], gold[f"randn{seed}_head"])
    assert cases.digest(x) == str(gold[f"randn{seed}_sha256"])


def test_type_conversions_match_reference(orc, gold):
    kat = gold["kat_in"]
    assert np.array_equal(orc.bf16_round(kat), gold["kat_bf16"])
    assert np.array_equal(orc.f16_round(kat), gold["kat_f16"])
    allh = np.arange(65536, dtype=np.uint16)
    assert bits_equal(orc.bf16_to_f32(allh), gold["kat_bf16_to_f32"])
    assert bits_equal(orc.f16_to_f32(allh), gold["kat_f16_to_f32"])


def test_sgemm_matches_reference(orc, gold):
    for name, (A, B, bt) in cases.gemm_cases(orc).items():
        assert bits_equal(orc.sgemm(A, B, b_trans=bt), gold[f"gemm_{name}"]), name


def test_sgemm_config1_matches_reference(orc, gold):
    A, B = cases.gemm_1024(orc)
    C = orc.sgemm(A, B)
    assert cases.digest(C) == str(gold["gemm1024_sha256"])
    assert bits_equal(C.reshape(-1)[cases.sample_index(C.size)], gold["gemm1024_sample"])


def test_flash_matches_reference(orc, gold):
    for name, (Q, K, V, scale, mask, bias) in cases.flash_cases(orc).items():
        assert bits_equal(orc.flash_attention(Q, K, V, scale, mask, bias), gold[f"flash_{name}"]), name
    Q, K, V = cases.sdpa_case(orc)
    assert bits_equal(orc.sdpa_gqa(Q, K, V, 0.0, True), gold["sdpa_gqa_causal"])
    assert bits_equal(orc.sdpa_gqa(np.ascontiguousarray(Q[:, :, -1:]), K, V, 0.0, True), gold["sdpa_gqa_decode"])


def test_norm_rope_match_reference(orc, gold):
    X, w = cases.norm_case(orc)
    assert bits_equal(orc.rms_norm(X, w, 1e-6), gold["rmsnorm"])
    c, s = orc.rope_tables(128, 4096, 1e6)
    assert cases.digest(c) == str(gold["rope_cos_sha256"])
    assert cases.digest(s) == str(gold["rope_sin_sha256"])
    assert bits_equal(orc.rope(cases.rope_case(orc), c, s), gold["rope"])


def test_qwen3_tiny_matches_reference(orc, gold):
    cfg, W, pr, steps = cases.qwen3_tiny(orc)
    t, m, lg = orc.qwen3_generate(cfg, W, pr, steps)
    assert np.array_equal(t, gold["qwen3_tiny_tokens"])
    assert bits_equal(lg, gold["qwen3_tiny_logits0"])


@pytest.mark.slow
@pytest.mark.skipif(not os.path.exists(GOLD_Q3), reason="configs[4] fixture not generated")
@pytest.mark.skipif(os.environ.get("YT_SLOW_TESTS") != "1", reason="set YT_SLOW_TESTS=1 (about 2 minutes of CPU)")
def test_qwen3_0p6b_matches_reference(orc):
    with np.load(GOLD_Q3, allow_pickle=False) as z:
        tokens, head = z["tokens"], z["logits0_head"]
    cfg = oracle.Qwen3Config()
    W = oracle.qwen3_random_weights(orc, cfg, seed=3)
    t, m, lg = orc.qwen3_generate(cfg, W, oracle.qwen3_prompt(cfg, 512, seed=4), len(tokens))
    assert np.array_equal(t, tokens)
    assert bits_equal(lg[:4096], head)


# ---------------------------------------------------- live reference (here)

def test_live_reference_random_shapes(orc, ref):
    rng = np.random.default_rng(99)
    for _ in range(12):
        m, n, k = (int(v) for v in rng.integers(1, 90, 3))
        A = rng.standard_normal((m, k)).astype(np.float32)
        W = rng.standard_normal((n, k)).astype(np.float32)
        assert bits_equal(orc.sgemm(A, W, b_trans=True), ref.sgemm(A, W, b_trans=True)), (m, n, k)
        B = np.ascontiguousarray(W.T)
        assert bits_equal(orc.sgemm(A, B), ref.sgemm(A, B)), (m, n, k)
    for q, kv in [(3, 50), (20, 20), (1, 200), (40, 90)]:
        Q = rng.standard_normal((q, 64)).astype(np.float32)
        K = rng.standard_normal((kv, 64)).astype(np.float32)
        V = rng.standard_normal((kv, 64)).astype(np.float32)
        mask = np.tril(np.ones((q, kv), bool), kv - q)
        assert bits_equal(orc.flash_attention(Q, K, V, 0.125, mask), ref.flash_attention(Q, K, V, 0.125, mask))


# ----------------------------------------------------------- closed forms

def test_bf16_round_formula(orc):
    # bfloat16.hpp:78-80: (u + ((u & 0x10000) >> 1)) >> 16
    u = np.array([0x3f808000, 0x3f818000, 0x3f807fff, 0x3f80ffff, 0x7f800000, 0x80000000], np.uint32)
    expect = ((u + ((u & 0x10000) >> 1)) >> 16).astype(np.uint16)
    assert np.array_equal(orc.bf16_round(u.view(np.float32)), expect)
    # with bit16 clear the value truncates even above the half-way point, where
    # IEEE round-to-nearest-even would round up: 0x3f80ffff -> 0x3f80 (RNE: 0x3f81)
    assert orc.bf16_round(np.array([0x3f80ffff], np.uint32).view(np.float32))[0] == 0x3f80


def test_f16_round_formula(orc):
    x = np.array([1.0, 65504.0, 65520.0, 6.1035156e-05, 3e-5, -2.5, 0.0], np.float32)
    got = orc.f16_round(x)
    assert got[0] == 0x3c00 and got[1] == 0x7bff and got[2] == 0x7c00  # 65520 rounds up to inf
    assert got[3] == 0x0400 and got[4] == 0x0000  # subnormal range flushes to zero
    assert got[5] == 0xc100 and got[6] == 0


def test_gemm_closed_forms(orc):
    rng = np.random.default_rng(0)
    A = rng.standard_normal((9, 32)).astype(np.float32)
    assert np.array_equal(orc.sgemm(A, np.eye(32, dtype=np.float32)), A)
    perm = rng.permutation(32)
    P = np.eye(32, dtype=np.float32)[:, perm]
    assert np.array_equal(orc.sgemm(A, P), A[:, perm])
    Ai = rng.integers(-8, 9, (13, 40)).astype(np.float32)
    Bi = rng.integers(-8, 9, (40, 11)).astype(np.float32)
    assert np.array_equal(orc.sgemm(Ai, Bi), (Ai.astype(np.int64) @ Bi.astype(np.int64)).astype(np.float32))
    # fp64 brute force on random data, alpha/beta
    B = rng.standard_normal((32, 7)).astype(np.float32)
    C0 = rng.standard_normal((9, 7)).astype(np.float32)
    got = orc.sgemm(A, B, alpha=0.5, beta=-2.0, C=C0)
    exact = 0.5 * (A.astype(np.float64) @ B) - 2.0 * C0
    assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(1)
    S, D = 24, 32
    Q = rng.standard_normal((S, D)).astype(np.float32)
    K = rng.standard_normal((S, D)).astype(np.float32)
    V = rng.standard_normal((S, D)).astype(np.float32)
    one = np.zeros((S, S), bool)
    one[:, 5] = True
    assert np.allclose(orc.flash_attention(Q, K, V, 0.2, one), np.broadcast_to(V[5], (S, D)), atol=1e-6)
    causal = np.tril(np.ones((S, S), bool))
    z = orc.flash_attention(np.zeros_like(Q), K, V, 0.2, causal)
    mean = np.cumsum(V.astype(np.float64), 0) / np.arange(1, S + 1)[:, None]
    assert np.allclose(z, mean, atol=1e-5)
    none = np.zeros((S, S), bool)
    assert np.all(orc.flash_attention(Q, K, V, 0.2, none) == 0.0)  # fully masked rows -> 0
    full = orc.flash_attention(Q, K, V, 0.2, causal)
    dec = orc.flash_attention(Q[-1:], K, V, 0.2, None)
    assert np.abs(full[-1] - dec[0]).max() <= 1e-5
    # fp64 brute force
    s = (Q.astype(np.float64) @ K.T.astype(np.float64)) * 0.2
    s[~causal] = -np.inf
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.abs(full - p @ V).max() <= 1e-5


def test_norm_rope_closed_forms(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    exact = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.abs(orc.rms_norm(x, w, 1e-6) - exact).max() <= 1e-5
    c, s = orc.rope_tables(128, 64, 1e6)
    t, i = 17, 9
    ang = t * (1.0 / 1e6 ** (2.0 * i / 128))
    assert math.isclose(c[t, i], math.cos(ang), abs_tol=1e-6) and c[t, i] == c[t, i + 64]
    X = rng.standard_normal((1, 1, 20, 128)).astype(np.float32)
    R = orc.rope(X, c, s)
    x1, x2 = X[..., :64].astype(np.float64), X[..., 64:].astype(np.float64)
    cc, ss = c[:20, :64], s[:20, :64]
    assert np.abs(R[..., :64] - (x1 * cc - x2 * ss)).max() <= 1e-6
    assert np.abs(R[..., 64:] - (x2 * cc + x1 * ss)).max() <= 1e-6
    assert np.allclose(np.linalg.norm(R, axis=-1), np.linalg.norm(X, axis=-1), rtol=1e-5)  # rotation
