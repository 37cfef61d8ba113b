"""torch-facing operators over libythip.so, mirroring yt::function.

Names and argument meaning follow the reference's operator API
(include/function/ops.hpp:10-70, include/function/normalization.hpp:59-89):

    matmul(a, b)                     YTensor::matmul / yt::function::matmul
    linear(x, weight)                yt::function::linear (weight [out, in])
    scaled_dot_product_attention(q, k, v, scale=0, mask=None, bias=None)
    rms_norm(x, weight, eps)         yt::function::rmsNorm (last axis)
    rms_norm_rope(...)               fused per-head rmsNorm_ + rope (qwen3 example)
    decode_attention(...)            the q_len == 1 SDPA path over a KV cache

Tensors are torch CUDA (HIP) tensors: PyTorch only supplies device memory and
the current stream. All arithmetic runs in the HIP kernels of libythip.so;
errors surface as YthipError (argument problems) or ValueError (shape checks
done here, mirroring src/function/ops.inl:123-128, 382-387).
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import check, i64array

_DT = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; the type set is float32/float16/bfloat16") from None


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("ytensor_amd operators take device (cuda/hip) tensors")


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

def gemm(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """out = alpha * a @ b + beta * out for 2-D or batched 3-D operands, any strides.

    a [M,K] or [Bt,M,K]; b [K,N] (shared) or [Bt,K,N]; out [M,N] or [Bt,M,N].
    """
    _dev(a, b, out)
    if a.dtype != b.dtype:
        raise ValueError("a and b must share a dtype")
    batched = a.dim() == 3
    A = a if batched else a.unsqueeze(0)
    Bm = b if b.dim() == 3 else b.unsqueeze(0)
    C = out if out.dim() == 3 else out.unsqueeze(0)
    bt, m, k = A.shape
    kb, n = Bm.shape[1], Bm.shape[2]
    if kb != k:
        raise ValueError(f"matmul: inner dimensions differ ({k} vs {kb})")
    if C.shape != (bt, m, n):
        raise ValueError(f"matmul: out has shape {tuple(out.shape)}, expected {(bt, m, n)}")
    if Bm.shape[0] not in (1, bt):
        raise ValueError("matmul: batch dimensions do not broadcast")
    sb_b = 0 if Bm.shape[0] == 1 else Bm.stride(0)
    st = _lib.lib().ythip_gemm(
        _code(a), _code(out), bt, m, n, k,
        A.data_ptr(), A.stride(0), A.stride(1), A.stride(2),
        Bm.data_ptr(), sb_b, Bm.stride(1), Bm.stride(2),
        C.data_ptr(), C.stride(0), C.stride(1), C.stride(2),
        float(alpha), float(beta), _stream())
    check(st, "ythip_gemm")
    return out


def matmul(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """YTensor::matmul: a [..., M, K] @ b [K, N] (or same-batch [..., K, N])."""
    out_dtype = out_dtype or a.dtype
    lead = a.shape[:-2]
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    if b.dim() == 2:
        # Batch-flatten fast path (src/ytensor_math.inl:960-1017) when rows are uniform.
        if a.dim() > 2 and a.is_contiguous():
            a2 = a.reshape(-1, k)
            out = torch.empty((a2.shape[0], n), dtype=out_dtype, device=a.device)
            gemm(a2, b, out)
            return out.reshape(*lead, m, n)
        a3 = a.reshape(-1, m, k) if a.dim() > 2 else a
        out = torch.empty((*a3.shape[:-1], n), dtype=out_dtype, device=a.device)
        gemm(a3, b, out)
        return out.reshape(*lead, m, n)
    a3 = a.reshape(-1, m, k)
    b3 = b.reshape(-1, k, n)
    out = torch.empty((a3.shape[0], m, n), dtype=out_dtype, device=a.device)
    gemm(a3, b3, out)
    return out.reshape(*lead, m, n)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """yt::function::linear: x [..., in] @ weight[out, in]^T (+ bias)."""
    k = x.shape[-1]
    if weight.shape[1] != k:
        raise ValueError(f"linear: weight has in_features {weight.shape[1]}, input has {k}")
    x2 = x.reshape(-1, k)
    out = torch.empty((x2.shape[0], weight.shape[0]), dtype=out_dtype or x.dtype, device=x.device)
    if bias is not None:
        out.copy_(bias.to(out.dtype).expand_as(out))
        gemm(x2, weight.t(), out, beta=1.0)
    else:
        gemm(x2, weight.t(), out)
    return out.reshape(*x.shape[:-1], weight.shape[0])


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------

def scaled_dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = 0.0,
                                 mask=None, bias: torch.Tensor | None = None,
                                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill SDPA over [B, Hq, Sq, D] queries and [B, Hkv, Skv, D] keys/values.

    mask: None (all visible), "causal" (key j visible to query i iff
    j <= Skv - Sq + i), or a bool/uint8 tensor [Sq, Skv] (True = visible).
    bias: optional float32 [Sq, Skv] added after scaling. GQA: query head h
    reads key/value head h // (Hq // Hkv).
    """
    _dev(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("scaled_dot_product_attention expects 4-D [B, H, S, D] tensors")
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    if k.shape[3] != D:
        raise ValueError("query/key head dims differ")  # ops.inl:382-384
    if v.shape[2] != Skv or v.shape[1] != Hkv:
        raise ValueError("key/value lengths differ")  # ops.inl:385-387
    if Hq % Hkv != 0:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    dv = v.shape[3]
    if out is None:
        out = torch.empty((B, Hq, Sq, dv), dtype=q.dtype, device=q.device)
    mask_kind, mptr, mld, mask_keep = _lib.MASK_NONE, None, 0, None
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask kind {mask!r}")
        mask_kind = _lib.MASK_CAUSAL
    elif mask is not None:
        if tuple(mask.shape) != (Sq, Skv):
            raise ValueError(f"mask shape {tuple(mask.shape)} != {(Sq, Skv)}")
        mask_keep = mask.to(torch.uint8)
        if mask_keep.stride(1) != 1:
            mask_keep = mask_keep.contiguous()
        mask_kind, mptr, mld = _lib.MASK_BOOL, mask_keep.data_ptr(), mask_keep.stride(0)
    bptr, brs, bcs, bias_keep = None, 0, 0, None
    if bias is not None:
        if tuple(bias.shape) != (Sq, Skv):
            raise ValueError(f"bias shape {tuple(bias.shape)} != {(Sq, Skv)}")
        bias_keep = bias.to(torch.float32)
        bptr, brs, bcs = bias_keep.data_ptr(), bias_keep.stride(0), bias_keep.stride(1)
    st = _lib.lib().ythip_attn_prefill(
        _code(q), B, Hq, Hkv, Sq, Skv, D, dv,
        q.data_ptr(), i64array(q.stride()), k.data_ptr(), i64array(k.stride()),
        v.data_ptr(), i64array(v.stride()), out.data_ptr(), i64array(out.stride()),
        float(scale), mask_kind, mptr, mld, bptr, brs, bcs, _stream())
    check(st, "ythip_attn_prefill")
    return out


def decode_workspace_bytes(B: int, Hq: int, max_ctx: int, d: int) -> int:
    return int(_lib.lib().ythip_attn_decode_workspace_size(B, Hq, max_ctx, d))


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     kv_len: torch.Tensor | None = None, scale: float = 0.0,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Single-query attention: q [B, Hq, D] (or [B, Hq, 1, D]) over caches
    [B, Hkv, max_ctx, D]; kv_len int32 [B] on device (None = max_ctx)."""
    _dev(q, k_cache, v_cache)
    q3 = q.reshape(q.shape[0], q.shape[1], q.shape[-1]) if q.dim() == 4 else q
    B, Hq, D = q3.shape
    Hkv, ctx = k_cache.shape[1], k_cache.shape[2]
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    o3 = out.reshape(B, Hq, D)
    ws_need = decode_workspace_bytes(B, Hq, ctx, D)
    if workspace is None or workspace.numel() * workspace.element_size() < ws_need:
        workspace = torch.empty(max(ws_need, 1), dtype=torch.uint8, device=q.device)
    if kv_len is not None:
        kv_len = kv_len.to(torch.int32).contiguous()
    st = _lib.lib().ythip_attn_decode(
        _code(q), B, Hq, Hkv, D, ctx,
        q3.data_ptr(), i64array(q3.stride()[:2]),
        k_cache.data_ptr(), v_cache.data_ptr(), i64array(k_cache.stride()[:3]),
        None if kv_len is None else kv_len.data_ptr(),
        o3.data_ptr(), i64array(o3.stride()[:2]), float(scale),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream())
    check(st, "ythip_attn_decode")
    return out.reshape(q.shape)


# ---------------------------------------------------------------------------
# RMSNorm / RoPE
# ---------------------------------------------------------------------------

def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """yt::function::rmsNorm over the last axis; weight float32 [n]; `out` may
    have another dtype than x (e.g. fp32 residual in, bf16 out)."""
    _dev(x, weight)
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    if out is None:
        out = torch.empty_like(x)
    o2 = out.reshape(-1, n)
    w = weight.to(torch.float32).contiguous()
    st = _lib.lib().ythip_rms_norm(_code(x), _code(out), x2.shape[0], n, x2.data_ptr(), x2.stride(0), w.data_ptr(),
                                   float(eps), o2.data_ptr(), o2.stride(0), _stream())
    check(st, "ythip_rms_norm")
    return out


def rms_norm_rope(qkv: torch.Tensor, Hq: int, Hkv: int, d: int, wq: torch.Tensor | None, wk: torch.Tensor | None,
                  eps: float, cos: torch.Tensor | None, sin: torch.Tensor | None, pos0: int = 0,
                  q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None,
                  v_out: torch.Tensor | None = None, cache_pos: int = 0, dev_pos: torch.Tensor | None = None):
    """Fused per-head RMSNorm + RoPE on qkv [B, S, (Hq+2*Hkv)*d].

    Returns (q [B,Hq,S,d], k, v) where k/v are written to rows
    cache_pos..cache_pos+S-1 of k_out/v_out [B,Hkv,*,d] when given (KV cache),
    else to new [B,Hkv,S,d] tensors.
    """
    _dev(qkv)
    B, S, W = qkv.shape
    if W != (Hq + 2 * Hkv) * d:
        raise ValueError(f"qkv width {W} != (Hq + 2*Hkv)*d = {(Hq + 2 * Hkv) * d}")
    if qkv.stride(2) != 1 or qkv.stride(0) != S * qkv.stride(1):
        qkv = qkv.contiguous()
    dev, dt = qkv.device, qkv.dtype
    if q_out is None:
        q_out = torch.empty((B, Hq, S, d), dtype=dt, device=dev)
    if k_out is None:
        k_out = torch.empty((B, Hkv, S, d), dtype=dt, device=dev)
    if v_out is None:
        v_out = torch.empty((B, Hkv, S, d), dtype=dt, device=dev)
    for name, t, h in (("q_out", q_out, Hq), ("k_out", k_out, Hkv), ("v_out", v_out, Hkv)):
        rows_needed = S if (name == "q_out" or dev_pos is not None) else cache_pos + S
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != h or t.shape[3] != d or t.shape[2] < rows_needed:
            raise ValueError(f"{name} has shape {tuple(t.shape)}; needs [{B}, {h}, >={rows_needed}, {d}]")
        if t.stride(3) != 1 or t.dtype != dt:
            raise ValueError(f"{name} must have a contiguous last dim and dtype {dt}")
    if cos is not None and dev_pos is None and (cos.shape[0] < pos0 + S or cos.shape[1] < d):
        raise ValueError(f"RoPE tables {tuple(cos.shape)} too small for positions {pos0}..{pos0 + S - 1}")
    keep = []

    def f32(t):
        if t is None:
            return None
        t = t.to(torch.float32).contiguous()
        keep.append(t)
        return t

    wq, wk, cos, sin = f32(wq), f32(wk), f32(cos), f32(sin)
    ld_tab = cos.stride(0) if cos is not None else 0
    st = _lib.lib().ythip_rmsnorm_rope(
        _code(qkv), B, S, Hq, Hkv, d, qkv.data_ptr(), qkv.stride(1),
        None if wq is None else wq.data_ptr(), None if wk is None else wk.data_ptr(), float(eps),
        None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(), ld_tab, int(pos0),
        q_out.data_ptr(), i64array(q_out.stride()[:3]),
        k_out.data_ptr(), i64array(k_out.stride()[:3]),
        v_out.data_ptr(), i64array(v_out.stride()[:3]),
        int(cache_pos), None if dev_pos is None else dev_pos.data_ptr(), _stream())
    check(st, "ythip_rmsnorm_rope")
    return q_out, k_out, v_out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SwiGLU on a fused [rows, 2n] gate_up projection -> [rows, n]."""
    _dev(gate_up)
    g2 = gate_up.reshape(-1, gate_up.shape[-1])
    n = g2.shape[1] // 2
    if out is None:
        out = torch.empty((*gate_up.shape[:-1], n), dtype=gate_up.dtype, device=gate_up.device)
    o2 = out.reshape(-1, n)
    check(_lib.lib().ythip_silu_mul(_code(gate_up), _code(out), g2.shape[0], n, g2.data_ptr(), g2.stride(0),
                                    o2.data_ptr(), o2.stride(0), _stream()), "ythip_silu_mul")
    return out


def embedding(table: torch.Tensor, ids: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[r] = table[ids[r]] with ids an int32 device tensor."""
    _dev(table, ids, out)
    if ids.dtype != torch.int32:
        raise ValueError("ids must be int32")
    check(_lib.lib().ythip_embedding(_code(table), _code(out), ids.numel(), table.shape[1], table.data_ptr(),
                                     ids.data_ptr(), out.data_ptr(), out.stride(0), _stream()), "ythip_embedding")
    return out


def argmax_step(logits: torch.Tensor, token: torch.Tensor, history: torch.Tensor | None = None,
                state: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy token (first max index) into token[0]; optionally history/state updates."""
    _dev(logits, token)
    if logits.dtype != torch.float32:
        raise ValueError("logits must be float32")
    check(_lib.lib().ythip_argmax_step(logits.numel(), logits.data_ptr(), token.data_ptr(),
                                       None if history is None else history.data_ptr(),
                                       None if state is None else state.data_ptr(), _stream()), "ythip_argmax_step")
    return token


GEMV_PROLOGUE = {"none": 0, "rmsnorm": 1, "swiglu": 2}


def gemv_fused(a: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, prologue: str = "none",
               norm_weight: torch.Tensor | None = None, eps: float = 1e-6, alpha: float = 1.0, beta: float = 0.0,
               argmax_parts: torch.Tensor | None = None) -> torch.Tensor:
    """Decode-time linear for at most 16 rows, out = alpha * A' @ weight.T + beta * out,
    weight [N, K] (the `linear` layout). prologue "none": A' = a [m, K];
    "rmsnorm": A' = rms_norm(a fp32 [m, K], norm_weight, eps) rounded to the weight
    type; "swiglu": A' = silu(gate) * up of a = [m, 2K] (gate | up). argmax_parts
    (fp32, 2 * ceil(N/16) values) receives per-tile (max, index) pairs of row 0."""
    _dev(a, weight, out)
    if prologue not in GEMV_PROLOGUE:
        raise ValueError(f"prologue must be one of {sorted(GEMV_PROLOGUE)}")
    pro = GEMV_PROLOGUE[prologue]
    n, k = weight.shape
    a2 = a.reshape(-1, a.shape[-1])
    o2 = out.reshape(-1, out.shape[-1])
    m = a2.shape[0]
    if o2.shape != (m, n):
        raise ValueError(f"out must be [{m}, {n}], got {tuple(o2.shape)}")
    if weight.stride(1) != 1 or a2.stride(1) != 1 or o2.stride(1) != 1:
        raise ValueError("gemv_fused needs unit column strides")
    want_a = torch.float32 if pro == 1 else weight.dtype
    if a.dtype != want_a:
        raise ValueError(f"A must be {want_a} for prologue {prologue!r}")
    if a2.shape[1] != (2 * k if pro == 2 else k):
        raise ValueError("A's width does not match the weight (2K for swiglu)")
    if pro == 1 and (norm_weight is None or norm_weight.dtype != torch.float32):
        raise ValueError("the rmsnorm prologue needs an fp32 norm_weight")
    if argmax_parts is not None and (argmax_parts.dtype != torch.float32 or argmax_parts.numel() < 2 * ((n + 15) // 16)):
        raise ValueError("argmax_parts must be fp32 with 2 * ceil(N/16) values")
    check(_lib.lib().ythip_gemv_fused(pro, _code(weight), _code(out), m, n, k, a2.data_ptr(), a2.stride(0),
                                      None if norm_weight is None else norm_weight.data_ptr(), float(eps),
                                      weight.data_ptr(), weight.stride(0), o2.data_ptr(), o2.stride(0),
                                      float(alpha), float(beta),
                                      None if argmax_parts is None else argmax_parts.data_ptr(), _stream()),
          "ythip_gemv_fused")
    return out


def argmax_finish(parts: torch.Tensor, n_parts: int, token: torch.Tensor, history: torch.Tensor | None = None,
                  state: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy token from gemv_fused's per-tile (max, index) pairs; as argmax_step."""
    _dev(parts, token)
    check(_lib.lib().ythip_argmax_finish(parts.data_ptr(), int(n_parts), token.data_ptr(),
                                         None if history is None else history.data_ptr(),
                                         None if state is None else state.data_ptr(), _stream()), "ythip_argmax_finish")
    return token


def default_scale(d: int) -> float:
    """scale = 0 -> 1/sqrt(d) (src/function/ops.inl:378-381)."""
    return 1.0 / math.sqrt(d)
