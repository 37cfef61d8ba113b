"""Inputs of the golden fixtures, regenerated from YTensor's RNG (pinned by
the randn fixture) so that only reference OUTPUTS are stored."""
from __future__ import annotations

import numpy as np

import oracle

RANDN_SEEDS = (0, 1, 2, 3)
RANDN_N = 1 << 20

# The discriminating configs[4]-shaped model: configs[4]'s seeded stream,
# layout and prompt, but matrices randn * 0.03 (about 1/sqrt(hidden)) and
# RMSNorm weights 1 + 0.1 * randn, so the greedy stream moves (26 distinct
# tokens in 32, top-2 margins >= 0.044; the literal configs[4] recipe, all
# weights randn * 0.02, repeats one token). Larger matrix scales move the stream
# too but make the 28-layer stack amplify perturbations: at 0.05 a bf16
# activation path is 3e-2 off the fp32 logits, at 0.03 about 1.5e-2.
QWEN3_VAR = {"seed": 3, "scale": 0.03, "norm_spread": 0.1, "prompt_len": 512, "prompt_seed": 4, "steps": 32}


def digest(x: np.ndarray) -> str:
    """SHA-256 of the raw bytes (float32 arrays hash their bit patterns)."""
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(x).tobytes()).hexdigest()


def conversion_inputs() -> np.ndarray:
    """Known-answer inputs for fp32 -> bf16 / fp16: ties, bit16 = 0 with low
    half 0x8000, subnormals, +-inf, NaN, fp16 over/underflow, random bits."""
    special = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 65504.0, 65520.0, 1e5,
                        6.1e-5, 6e-8, 5.96e-8, 1.0000001, 3.0e38, -3.0e38, 0.1, 1 / 3], dtype=np.float32)
    bits = np.array([0x3f808000, 0x3f818000, 0x3f80ffff, 0x3f817fff, 0x7f7fffff, 0x00800000, 0x387fe000,
                     0x38800000, 0x33000000, 0x477fe000, 0x477ff000, 0x7fc00001, 0xff800001], dtype=np.uint32)
    rnd = np.random.default_rng(123).integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([special, bits.view(np.float32), rnd.view(np.float32)])


def gemm_cases(path) -> dict:
    out = {}
    for (m, n, k) in [(7, 13, 5), (6, 16, 500), (37, 41, 1001), (1, 33, 70), (64, 64, 64), (1, 37, 128), (5, 1, 33)]:
        for bt in (False, True):
            path.seed(m * 1000 + n * 10 + k)
            A = path.randn(m, k)
            B = path.randn(n, k) if bt else path.randn(k, n)
            out[f"{m}x{n}x{k}_{'wt' if bt else 'nn'}"] = (A, B, bt)
    return out


def gemm_1024(path):
    """seed 0, A then B ~ N(0,1) [1024,1024]."""
    path.seed(0)
    return path.randn(1024, 1024), path.randn(1024, 1024)


def sample_index(size: int, count: int = 4096) -> np.ndarray:
    return np.random.default_rng(7).choice(size, count, replace=False)


def flash_cases(path) -> dict:
    out = {}
    for (q, kv, d, kind) in [(5, 9, 16, "none"), (13, 13, 128, "causal"), (17, 40, 128, "bool"),
                             (17, 40, 128, "bias"), (1, 37, 128, "none"), (1, 37, 128, "bool"),
                             (33, 70, 64, "causal")]:
        path.seed(q * 100 + kv + d)
        Q, K, V = path.randn(q, d), path.randn(kv, d), path.randn(kv, d)
        mask = bias = None
        if kind == "causal":
            mask = np.tril(np.ones((q, kv), bool), kv - q)
        elif kind == "bool":
            mask = path.randn(q, kv) > -0.3
            mask[min(3, q - 1)] = False
        elif kind == "bias":
            bias = path.randn(q, kv)
        out[f"{q}x{kv}x{d}_{kind}"] = (Q, K, V, 1.0 / np.sqrt(d).astype(np.float32), mask, bias)
    return out


def sdpa_case(path):
    path.seed(11)
    return path.randn(1, 4, 17, 32), path.randn(1, 2, 17, 32), path.randn(1, 2, 17, 32)


def norm_case(path):
    path.seed(12)
    return path.randn(2, 3, 128), path.randn(128)


def rope_case(path):
    path.seed(13)
    return path.randn(2, 3, 50, 128)


def qwen3_tiny(path):
    cfg = oracle.Qwen3Config(hidden=64, layers=2, vocab=97, inter=128, n_heads=4, n_kv=2, head_dim=16, max_pos=64)
    W = oracle.qwen3_random_weights(path, cfg, seed=3)
    return cfg, W, oracle.qwen3_prompt(cfg, 9, seed=4), 8
