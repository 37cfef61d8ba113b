"""GPU: the decode-time linear with fused prologues (ythip_gemv_fused) and the
split argmax (ythip_argmax_finish).

* prologue "none" against the oracle's fp32 sgemm on the up-converted inputs
  (bf16 bar: rel <= 2e-2, MAE <= 1e-3 or 1.1x the output rounding floor);
* "rmsnorm" and "swiglu" against the unfused libythip sequence
  (ythip_rms_norm / ythip_silu_mul, then ythip_gemm): bit-identical, which is
  the fused kernels' contract, plus the oracle's rmsNorm_ + linear chain to the
  bf16 bar (src/function/normalization.inl:256-277, src/function/ops.inl:84-91);
* argmax_finish over the per-tile pairs equals argmax_step over the logits,
  ties included (lowest index wins, qwen3.cpp:465-486 with argmax)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import check16

pytestmark = pytest.mark.gpu


def _bf(x: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev).to(torch.bfloat16)


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@pytest.mark.parametrize("m,n,k", [(1, 3072, 1024), (1, 1024, 2048), (3, 1000, 512), (16, 4096, 1024),
                                   (1, 1024, 3072), (7, 48, 64)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemv_plain_vs_oracle(orc, yt, dev, m, n, k, out_dtype):
    rng = np.random.default_rng(m * 1000 + n + k)
    a = _bf(rng.standard_normal((m, k)), dev)
    w = _bf(rng.standard_normal((n, k)) * 0.02, dev)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    out = torch.from_numpy(c0).to(dev).to(out_dtype)
    yt.gemv_fused(a, w, out, "none", alpha=0.5, beta=1.0)
    torch.cuda.synchronize()
    ref = 0.5 * orc.sgemm(_f32(a), _f32(w), b_trans=True) + _f32(torch.from_numpy(c0).to(out_dtype))
    got = _f32(out)
    if out_dtype == torch.float32:
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    else:
        check16(orc, got, ref, "bf16", True, f"gemv none {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 4096, 1024), (1, 6144, 1024), (4, 1000, 256), (16, 2048, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemv_rmsnorm_fused_equals_unfused(orc, yt, dev, m, n, k, out_dtype):
    rng = np.random.default_rng(n + k + m)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32) * 3).to(dev)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(k)).astype(np.float32)).to(dev)
    w = _bf(rng.standard_normal((n, k)) * 0.02, dev)
    fused = torch.zeros((m, n), dtype=out_dtype, device=dev)
    yt.gemv_fused(x, w, fused, "rmsnorm", nw, 1e-6)
    h = torch.empty((m, k), dtype=torch.bfloat16, device=dev)
    yt.rms_norm(x, nw, 1e-6, out=h)
    unf = torch.zeros((m, n), dtype=out_dtype, device=dev)
    yt.gemm(h, w.t(), unf)
    torch.cuda.synchronize()
    assert torch.equal(fused, unf)
    # the normalised rows against the oracle's rmsNorm_, then the product against
    # the oracle's fp32 sgemm on the up-converted bf16 operands (the GEMM bar)
    hn = orc.rms_norm(_f32(x), _f32(nw), 1e-6)
    check16(orc, _f32(h), hn, "bf16", True, f"rmsnorm rows {m}x{k}")
    ref = orc.sgemm(_f32(h), _f32(w), b_trans=True)
    check16(orc, _f32(fused), ref, "bf16", out_dtype == torch.bfloat16, f"gemv rmsnorm {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 1024, 3072), (2, 512, 1024), (16, 1024, 512)])
def test_gemv_swiglu_fused_equals_unfused(orc, yt, dev, m, n, k):
    rng = np.random.default_rng(7 * n + k)
    gu = _bf(rng.standard_normal((m, 2 * k)) * 2, dev)
    w = _bf(rng.standard_normal((n, k)) * 0.02, dev)
    base = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(dev)
    fused = base.clone()
    yt.gemv_fused(gu, w, fused, "swiglu", beta=1.0)
    act = torch.empty((m, k), dtype=torch.bfloat16, device=dev)
    yt.silu_mul(gu, out=act)
    unf = base.clone()
    yt.gemm(act, w.t(), unf, beta=1.0)
    torch.cuda.synchronize()
    assert torch.equal(fused, unf)
    g, u = _f32(gu)[:, :k].astype(np.float64), _f32(gu)[:, k:].astype(np.float64)
    act_ref = (g / (1 + np.exp(-g)) * u).astype(np.float32)
    ref = orc.sgemm(act_ref, _f32(w), b_trans=True) + _f32(base)
    assert np.abs(_f32(fused) - ref).max() <= 2e-2 * np.abs(ref).max()


def test_lm_head_argmax_parts_match_argmax_step(yt, dev):
    """Final norm + LM head with per-tile argmax pairs; duplicated weight rows
    make exact logit ties, which must resolve to the lowest index."""
    rng = np.random.default_rng(11)
    k, n = 1024, 151936
    w_np = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    x = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float32)).to(dev)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(k)).astype(np.float32)).to(dev)
    h = torch.empty((1, k), dtype=torch.bfloat16, device=dev)
    yt.rms_norm(x, nw, 1e-6, out=h)
    # find the winner, then copy its row to a lower and a higher index to force ties
    w = _bf(w_np, dev)
    logits = torch.empty((1, n), dtype=torch.float32, device=dev)
    yt.gemm(h, w.t(), logits)
    win = int(torch.argmax(logits).item())
    lo, hi = max(win // 3, 1), min(win + 12345, n - 1)
    w[lo] = w[win]
    w[hi] = w[win]
    parts = torch.empty((2 * ((n + 15) // 16),), dtype=torch.float32, device=dev)
    for use_parts in (True, False):
        tok = torch.zeros((1,), dtype=torch.int32, device=dev)
        hist = torch.zeros((8,), dtype=torch.int32, device=dev)
        state = yt.ops.decode_state(40, 64, 64, generated=2, history=8, device=dev)
        lg = torch.empty((1, n), dtype=torch.float32, device=dev)
        if use_parts:
            yt.gemv_fused(x, w, lg, "rmsnorm", nw, 1e-6, argmax_parts=parts)
            yt.argmax_finish(parts, parts.numel() // 2, tok, hist, state)
        else:
            yt.gemm(h, w.t(), lg)
            yt.argmax_step(lg, tok, hist, state)
        torch.cuda.synchronize()
        assert int(tok.item()) == min(lo, win), (use_parts, int(tok.item()), lo, win)
        assert int(hist[2].item()) == int(tok.item())
        st = state.tolist()
        assert (st[yt.ops.ST_GENERATED], st[yt.ops.ST_TOTAL], st[yt.ops.ST_SLOT], st[yt.ops.ST_KV_LEN],
                st[yt.ops.ST_ROPE_POS], st[yt.ops.ST_ERROR]) == (3, 41, 41, 42, 41, 0)
        if use_parts:
            lg_fused = lg.clone()
        else:
            assert torch.equal(lg_fused, lg)


def test_gemv_argument_errors(yt, dev):
    a = torch.zeros((17, 64), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((32, 64), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((17, 32), dtype=torch.bfloat16, device=dev)
    with pytest.raises(yt.YthipError):
        yt.gemv_fused(a, w, out)  # more than 16 rows
    with pytest.raises(ValueError):
        yt.gemv_fused(a[:1], w, out[:1], "rmsnorm")  # needs fp32 A and a norm weight


@pytest.mark.parametrize("m,inter,k", [(1, 3072, 1024), (3, 1000, 512), (16, 520, 256), (1, 12, 64)])
@pytest.mark.parametrize("prologue", ["none", "rmsnorm"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemv_swiglu_epilogue_equals_unfused(orc, yt, dev, m, inter, k, prologue, dtype):
    """gate_up linear + SwiGLU in one launch equals the linear into [m, 2I]
    followed by silu_mul, bit for bit (I not a multiple of 8 included)."""
    rng = np.random.default_rng(m * 31 + inter + k)
    w = torch.from_numpy(rng.standard_normal((2 * inter, k)).astype(np.float32) * 0.05).to(dev).to(dtype)
    if prologue == "rmsnorm":
        a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32) * 3).to(dev)
        nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(k)).astype(np.float32)).to(dev)
    else:
        a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(dtype)
        nw = None
    out = torch.full((m, inter), 7.0, dtype=dtype, device=dev)
    yt.gemv_swiglu(a, w, out, prologue, nw, 1e-6)
    gu = torch.empty((m, 2 * inter), dtype=dtype, device=dev)
    yt.gemv_fused(a, w, gu, prologue, nw, 1e-6)
    act = torch.empty((m, inter), dtype=dtype, device=dev)
    yt.silu_mul(gu, out=act)
    torch.cuda.synchronize()
    assert torch.equal(out, act)
    # against float64 on the rounded gate/up values (the activation bar)
    g, u = _f32(gu)[:, :inter].astype(np.float64), _f32(gu)[:, inter:].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert np.abs(_f32(out) - ref).max() <= 1e-2 * max(1.0, np.abs(ref).max())


def test_gemv_swiglu_argument_errors(yt, dev):
    w = torch.zeros((33, 64), dtype=torch.bfloat16, device=dev)
    a = torch.zeros((1, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        yt.gemv_swiglu(a, w, torch.zeros((1, 16), dtype=torch.bfloat16, device=dev))  # odd row count
    w = torch.zeros((32, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        yt.gemv_swiglu(a, w, torch.zeros((1, 16), dtype=torch.float32, device=dev))  # out dtype
    with pytest.raises(ValueError):
        yt.gemv_swiglu(a, w, torch.zeros((1, 16), dtype=torch.bfloat16, device=dev), "rmsnorm")  # fp32 A needed
