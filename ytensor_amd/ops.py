"""torch-facing operators over libythip.so, mirroring yt::function.

Names and argument meaning follow the reference's operator API
(include/function/ops.hpp:10-70, include/function/normalization.hpp:59-89):

    matmul(a, b)                     YTensor::matmul / yt::function::matmul
    linear(x, weight)                yt::function::linear (weight [out, in])
    scaled_dot_product_attention(q, k, v, scale=0, mask=None, bias=None, backend="flash"|"math")
    masked_matmul(a, b, mask, masked_value)   YTensor::masked_matmul
    gemm_masked(a, b, out, mask, alpha, beta) yt::kernel::avx2::sgemm_masked
    rms_norm(x, weight, eps)         yt::function::rmsNorm (last axis)
    rms_norm_rope(...)               fused per-head rmsNorm_ + rope (qwen3 example)
    decode_attention(...)            the q_len == 1 SDPA path over a KV cache

Tensors are torch CUDA (HIP) tensors: PyTorch only supplies device memory and
the current stream. All arithmetic runs in the HIP kernels of libythip.so;
errors surface as YthipError (argument problems) or ValueError (shape checks
done here, mirroring src/function/ops.inl:123-128, 382-387).
"""
from __future__ import annotations

import itertools
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
    """YTensor::matmul (src/ytensor_math.inl:284-316, 954-1051): a [..., M, K] @
    b [..., K, N] over the last two dims, the leading dims broadcast against each
    other (a size-1 dim repeats; unequal sizes raise, as computeBroadcastShape
    does). Output [broadcast lead..., M, N]."""
    if a.dim() < 2 or b.dim() < 2:
        raise ValueError("matmul: both operands need at least 2 dimensions")
    out_dtype = out_dtype or a.dtype
    m, k = a.shape[-2], a.shape[-1]
    kb, n = b.shape[-2], b.shape[-1]
    if kb != k:
        raise ValueError(f"matmul: inner dimensions differ ({k} vs {kb})")
    try:
        lead = tuple(torch.broadcast_shapes(a.shape[:-2], b.shape[:-2]))
    except RuntimeError:
        raise ValueError(f"matmul: batch dimensions {tuple(a.shape[:-2])} and {tuple(b.shape[:-2])} "
                         "do not broadcast") from None
    b_is_2d = all(s == 1 for s in b.shape[:-2])
    if b_is_2d:
        b2 = b.reshape(k, n) if b.dim() > 2 else b
        # Batch-flatten fast path (src/ytensor_math.inl:960-1017): a's rows are
        # uniform, so [..., M, K] is one [prod(lead) * M, K] product.
        if a.dim() > 2 and a.is_contiguous() and tuple(a.shape[:-2]) == lead:
            a2 = a.reshape(-1, k)
            out = torch.empty((a2.shape[0], n), dtype=out_dtype, device=a.device)
            gemm(a2, b2, out)
            return out.reshape(*lead, m, n)
    out = torch.empty((*lead, m, n), dtype=out_dtype, device=a.device)
    if not lead:
        gemm(a, b, out)
        return out
    ae = a.expand(*lead, m, k)
    be = b.expand(*lead, k, n)
    # One batched launch over the last lead dim per index of the others (an
    # expanded dim has stride 0, i.e. a shared operand).
    outer = lead[:-1]
    for idx in itertools.product(*[range(s) for s in outer]):
        gemm(ae[idx], be[idx], out[idx])
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """yt::function::linear: x [..., in] @ weight[out, in]^T (+ bias)."""
    k = x.shape[-1]
    if weight.shape[1] != k:
        raise ValueError(f"linear: weight has in_features {weight.shape[1]}, input has {k}")
    out_dtype = out_dtype or x.dtype
    if bias is not None:
        if bias.dim() != 1 or bias.shape[0] != weight.shape[0]:
            raise ValueError("linear: bias size must match weight.shape(0)")
        if bias.dtype != out_dtype:
            raise ValueError(f"linear: bias has dtype {bias.dtype}, the output {out_dtype}")
        _dev(bias)
    x2 = x.reshape(-1, k)
    out = torch.empty((x2.shape[0], weight.shape[0]), dtype=out_dtype, device=x.device)
    gemm(x2, weight.t(), out)
    if bias is not None:
        # ops.inl:93-104: the product is rounded to the output type first, then
        # the bias is added in that type
        b = bias.contiguous()
        check(_lib.lib().ythip_add_bias(_code(out), out.shape[0], out.shape[1], out.data_ptr(), out.stride(0),
                                        b.data_ptr(), _stream()), "ythip_add_bias")
    return out.reshape(*x.shape[:-1], weight.shape[0])


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------

def _predicate_mask(f, m: int, n: int, device) -> torch.Tensor:
    """A predicate f(row, col) -> bool evaluated into a [m, n] byte mask, as the
    reference calls it per element (src/kernel/avx2/flash_attention.inl:14-49).
    Tried once on index grids (numpy broadcasting), else element by element."""
    import numpy as np
    ii, jj = np.arange(m)[:, None], np.arange(n)[None, :]
    try:
        r = np.broadcast_to(np.asarray(f(ii, jj), dtype=bool), (m, n))
    except Exception:
        r = np.array([[bool(f(i, j)) for j in range(n)] for i in range(m)], dtype=bool).reshape(m, n)
    return torch.from_numpy(np.ascontiguousarray(r, dtype=np.uint8)).to(device)


def _mask_args(mask, m: int, n: int, device):
    """-> (kind, pointer, ld, keep-alive) for the C ABI's mask arguments.
    mask: None, "causal" (j <= i + n - m), ("diag", offset) (j <= i + offset),
    a bool / uint8 tensor [m, n] (True = visible), or a predicate f(i, j)."""
    if mask is None:
        return _lib.MASK_NONE, None, 0, None
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask kind {mask!r}")
        return _lib.MASK_CAUSAL, None, 0, None
    if isinstance(mask, tuple):
        if len(mask) != 2 or mask[0] != "diag":
            raise ValueError(f"unknown mask {mask!r}; use ('diag', offset)")
        return _lib.MASK_DIAG, None, int(mask[1]), None
    if callable(mask) and not isinstance(mask, torch.Tensor):
        mask = _predicate_mask(mask, m, n, device)
    if tuple(mask.shape) != (m, n):
        raise ValueError(f"mask shape {tuple(mask.shape)} != {(m, n)}")  # ops.inl:390-393
    if mask.dtype == torch.bool and mask.device == torch.device(device):
        keep = mask.view(torch.uint8)  # one 0/1 byte per element already: read in place, no copy
    else:
        keep = mask.to(device=device, dtype=torch.uint8)
    if keep.stride(1) != 1:
        keep = keep.contiguous()
    return _lib.MASK_BOOL, keep.data_ptr(), keep.stride(0), keep


def _fold(shape, strides):
    """(size, stride) of dims read as one, or None when their strides do not nest."""
    dims = [(sz, st) for sz, st in zip(shape, strides) if sz != 1]
    total = 1
    for sz, _ in dims:
        total *= sz
    for (s0, st0), (s1, st1) in zip(dims, dims[1:]):
        if st0 != st1 * s1:
            return None
    return total, (dims[-1][1] if dims else 0)


def scaled_dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = 0.0,
                                 mask=None, bias: torch.Tensor | None = None,
                                 out: torch.Tensor | None = None, backend: str = "flash",
                                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """yt::function::scaledDotProductAttention (src/function/ops.inl:368-503).

    q [..., Sq, D], k [..., Skv, D], v [..., Skv, Dv]: the leading dims
    broadcast against each other as the reference's matView does (0-stride
    views such as the examples' repeat_kv are read in place; the innermost
    leading dims over which k and v are broadcast become the GQA group). The
    Qwen3 form q [B, Hq, Sq, D] with k/v [B, Hkv, Skv, D], Hq a multiple of Hkv,
    is accepted directly: query head h reads key/value head h // (Hq // Hkv).
    Any element strides, including transposed keys (a [..., D, Skv] cache seen
    through .transpose(-1, -2)).
    mask: None, "causal" (key j visible to query i iff j <= Skv - Sq + i),
    ("diag", off) (j <= i + off), a bool / uint8 tensor [Sq, Skv] (True =
    visible) or a predicate f(i, j) -> bool (evaluated into a bool mask here).
    bias: optional float32 [Sq, Skv] added after scaling. Rows with no visible
    key come out zero. backend: "flash" (FLASH_AVX2's counterpart, online
    softmax, no score matrix; Sq == 1 runs the split-K decode kernel for every
    mask kind, as flash_attention's q_len == 1 branch does; with a bool mask or
    Sq == 1, a workspace of ythip_attn_sdpa_workspace_size bytes for the mask's
    tile classes or the decode partials) or
    "math" (MATH: materialised scores in a workspace of
    ythip_attn_math_workspace_size bytes). A workspace not given or too small
    is allocated.
    """
    _dev(q, k, v)
    if backend not in ("flash", "math"):
        raise ValueError(f"unknown backend {backend!r}")  # throwNotSupport (ops.inl:423)
    if q.dim() < 2 or k.dim() < 2 or v.dim() < 2:
        raise ValueError("scaled_dot_product_attention expects [..., S, D] tensors")
    Sq, D = q.shape[-2], q.shape[-1]
    Skv, dv = k.shape[-2], v.shape[-1]
    if k.shape[-1] != D:
        raise ValueError("Query and key head dim must match.")  # ops.inl:382-384
    if v.shape[-2] != Skv:
        raise ValueError("Key/value sequence length must match.")  # ops.inl:385-387
    gqa = (q.dim() == 4 and k.dim() == 4 and v.dim() == 4 and q.shape[0] == k.shape[0] == v.shape[0]
           and k.shape[1] == v.shape[1] and k.shape[1] != q.shape[1] and q.shape[1] % k.shape[1] == 0)
    if gqa:
        lead = tuple(q.shape[:2])
        B, Hq, Hkv = q.shape[0], q.shape[1], k.shape[1]
        qv, kv_, vv = q, k, v
    else:
        lead = tuple(torch.broadcast_shapes(q.shape[:-2], k.shape[:-2], v.shape[:-2]))
        qv = q.expand(*lead, Sq, D)
        kv_ = k.expand(*lead, Skv, D)
        vv = v.expand(*lead, Skv, dv)
    if out is None:
        out = torch.empty((*lead, Sq, dv), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (*lead, Sq, dv):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {(*lead, Sq, dv)}")
    kind, mptr, mld, mask_keep = _mask_args(mask, Sq, Skv, q.device)
    bptr, brs, bcs, bias_keep = None, 0, 0, None
    if bias is not None:
        if tuple(bias.shape) != (Sq, Skv):
            raise ValueError("Bias shape must match the last two dimensions of the score tensor.")
        bias_keep = bias.to(torch.float32)
        bptr, brs, bcs = bias_keep.data_ptr(), bias_keep.stride(0), bias_keep.stride(1)

    def call(qt, kt, vt, ot, B, Hq, Hkv, qs, ks, vs, os_):
        if backend == "math":
            need = int(_lib.lib().ythip_attn_math_workspace_size(_code(q), B, Hq, Sq, Skv))
            ws = workspace
            if ws is None or ws.numel() * ws.element_size() < need:
                ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
            st = _lib.lib().ythip_attn_math(
                _code(q), B, Hq, Hkv, Sq, Skv, D, dv, qt.data_ptr(), i64array(qs), kt.data_ptr(), i64array(ks),
                vt.data_ptr(), i64array(vs), ot.data_ptr(), i64array(os_), float(scale), kind, mptr, mld,
                bptr, brs, bcs, ws.data_ptr(), ws.numel() * ws.element_size(), _stream())
            check(st, "ythip_attn_math")
        elif kind == _lib.MASK_BOOL or Sq == 1:
            # room for the mask's tile classes (the long-sequence path lists the
            # key blocks each query block sees from them) and, for one query
            # row, the split-K partials of the decode kernel that row runs on
            need = int(_lib.lib().ythip_attn_sdpa_workspace_size(B, Hq, Sq, Skv, D))
            ws = workspace
            if ws is None or ws.numel() * ws.element_size() < need:
                ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
            st = _lib.lib().ythip_attn_prefill_ws(
                _code(q), B, Hq, Hkv, Sq, Skv, D, dv, qt.data_ptr(), i64array(qs), kt.data_ptr(), i64array(ks),
                vt.data_ptr(), i64array(vs), ot.data_ptr(), i64array(os_), float(scale), kind, mptr, mld,
                bptr, brs, bcs, ws.data_ptr(), ws.numel() * ws.element_size(), _stream())
            check(st, "ythip_attn_prefill_ws")
        else:
            st = _lib.lib().ythip_attn_prefill(
                _code(q), B, Hq, Hkv, Sq, Skv, D, dv, qt.data_ptr(), i64array(qs), kt.data_ptr(), i64array(ks),
                vt.data_ptr(), i64array(vs), ot.data_ptr(), i64array(os_), float(scale), kind, mptr, mld,
                bptr, brs, bcs, _stream())
            check(st, "ythip_attn_prefill")

    if gqa:
        call(qv, kv_, vv, out, B, Hq, Hkv, qv.stride(), kv_.stride(), vv.stride(), out.stride())
        return out
    # (batch, kv-head, group) from the leading dims: the innermost dims over
    # which k and v do not move form the group, the first dim is the batch.
    n = len(lead)
    p = n
    while p > 0 and (lead[p - 1] == 1 or (kv_.stride(p - 1) == 0 and vv.stride(p - 1) == 0)):
        p -= 1
    bdims = 1 if p >= 1 else 0
    fq = _fold(lead[bdims:], qv.stride()[bdims:n])
    fo = _fold(lead[bdims:], out.stride()[bdims:n])
    fk = _fold(lead[bdims:p], kv_.stride()[bdims:p])
    fv = _fold(lead[bdims:p], vv.stride()[bdims:p])
    if None not in (fq, fo, fk, fv) and n >= 1:
        B = lead[0] if bdims else 1
        s0 = lambda t: t.stride(0) if bdims else 0  # noqa: E731
        Hq, Hkv = fq[0], fk[0]
        call(qv, kv_, vv, out, B, Hq, Hkv,
             (s0(qv), fq[1], qv.stride(-2), qv.stride(-1)), (s0(kv_), fk[1], kv_.stride(-2), kv_.stride(-1)),
             (s0(vv), fv[1], vv.stride(-2), vv.stride(-1)), (s0(out), fo[1], out.stride(-2), out.stride(-1)))
        return out
    # leading dims that do not fold: one matrix per call
    import itertools
    for idx in itertools.product(*[range(x) for x in lead]):
        qt, kt, vt, ot = qv[idx], kv_[idx], vv[idx], out[idx]
        call(qt, kt, vt, ot, 1, 1, 1, (0, 0, qt.stride(0), qt.stride(1)), (0, 0, kt.stride(0), kt.stride(1)),
             (0, 0, vt.stride(0), vt.stride(1)), (0, 0, ot.stride(0), ot.stride(1)))
    return out


def masked_gemm_workspace_bytes(batch: int, m: int, n: int) -> int:
    return int(_lib.lib().ythip_gemm_masked_workspace_size(batch, m, n))


def gemm_masked(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, mask, alpha: float = 1.0, beta: float = 0.0,
                fill: float | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """sgemm_masked (src/kernel/avx2/sgemm.inl:342-584) on 2-D or batched 3-D
    operands: where `mask` ([m, n], shared by the batch; forms as for attention)
    is set, out = alpha * a @ b + beta * out; elsewhere out is kept, or set to
    `fill` when given (masked_matmul's maskedValue)."""
    _dev(a, b, out)
    if a.dtype != b.dtype:
        raise ValueError("a and b must share a dtype")
    A = a if a.dim() == 3 else a.unsqueeze(0)
    Bm = b if b.dim() == 3 else b.unsqueeze(0)
    C = out if out.dim() == 3 else out.unsqueeze(0)
    bt, m, k = A.shape
    n = Bm.shape[2]
    if Bm.shape[1] != k:
        raise ValueError(f"masked_matmul: inner dimensions differ ({k} vs {Bm.shape[1]})")
    if tuple(C.shape) != (bt, m, n) or Bm.shape[0] not in (1, bt):
        raise ValueError("masked_matmul: shapes do not match")
    kind, mptr, mld, keep = _mask_args(mask, m, n, a.device)
    need = masked_gemm_workspace_bytes(bt, m, n)
    ws = workspace
    if ws is None or ws.numel() * ws.element_size() < need:
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=a.device)
    st = _lib.lib().ythip_gemm_masked(
        _code(a), _code(out), bt, m, n, k,
        A.data_ptr(), A.stride(0), A.stride(1), A.stride(2),
        Bm.data_ptr(), 0 if Bm.shape[0] == 1 else Bm.stride(0), Bm.stride(1), Bm.stride(2),
        C.data_ptr(), C.stride(0), C.stride(1), C.stride(2), float(alpha), float(beta),
        kind, mptr, mld, int(fill is not None), float(fill or 0.0), ws.data_ptr(), ws.numel() * ws.element_size(),
        _stream())
    check(st, "ythip_gemm_masked")
    return out


def masked_matmul(a: torch.Tensor, b: torch.Tensor, mask, masked_value: float = 0.0) -> torch.Tensor:
    """YTensor::masked_matmul (src/ytensor_math.inl:318-410): a [..., m, k] @
    b [k, n] or [..., k, n] where `mask` [m, n] is set, masked_value elsewhere."""
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    lead = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    a3 = a.expand(*lead, m, k).reshape(-1, m, k)
    b3 = b if b.dim() == 2 else b.expand(*lead, k, n).reshape(-1, k, n)
    out = torch.empty((a3.shape[0], m, n), dtype=a.dtype, device=a.device)
    gemm_masked(a3, b3, out, mask, fill=masked_value)
    return out.reshape(*lead, m, n)


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
        if kv_len.dtype != torch.int32 or kv_len.numel() < B:
            raise ValueError(f"kv_len must be an int32 device tensor with {B} entries")
        kv_len = kv_len.contiguous()
    st = _lib.lib().ythip_attn_decode(
        _code(q), B, Hq, Hkv, D, ctx,
        q3.data_ptr(), i64array(q3.stride()[:2]),
        k_cache.data_ptr(), v_cache.data_ptr(), i64array(k_cache.stride()[:3]),
        None if kv_len is None else kv_len.data_ptr(),
        o3.data_ptr(), i64array(o3.stride()[:2]), float(scale),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream())
    check(st, "ythip_attn_decode")
    return out.reshape(q.shape)


def decode_splits(B: int, Hq: int, max_ctx: int) -> int:
    return int(_lib.lib().ythip_attn_decode_splits(B, Hq, max_ctx))


def decode_attention_rope(qkv: torch.Tensor, Hq: int, Hkv: int, d: int, wq: torch.Tensor | None,
                          wk: torch.Tensor | None, eps: float, cos: torch.Tensor | None, sin: torch.Tensor | None,
                          dev_state: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          out: torch.Tensor | None, workspace: torch.Tensor, scale: float = 0.0):
    """One decode step of a Qwen3 attention layer: the new token's qkv row
    [B, (Hq + 2 Hkv) d] gets per-head RMSNorm + RoPE at the record's RoPE row,
    k/v are written to the ring caches [B, Hkv, max_ctx, d] at its slot, and
    out [B, Hq, d] = attention over the record's KV_LEN cache rows -- the same
    bits as rms_norm_rope followed by decode_attention. With out=None the
    result stays as split-K partials in `workspace` (decode_workspace_bytes)."""
    _dev(qkv, k_cache, v_cache, workspace, dev_state)
    if dev_state.dtype != torch.int32 or dev_state.numel() < ST_WORDS:
        raise ValueError("dev_state must be the int32[16] decode-state record")
    B = qkv.shape[0]
    ctx = k_cache.shape[2]
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if qkv.shape[-1] != (Hq + 2 * Hkv) * d or qkv.stride(-1) != 1:
        raise ValueError("qkv rows must hold (Hq + 2 Hkv) * d contiguous elements")
    o3 = None if out is None else out.reshape(B, Hq, d)
    st = _lib.lib().ythip_attn_decode_rope(
        _code(qkv), B, Hq, Hkv, d, ctx, qkv.data_ptr(), qkv.stride(0),
        None if wq is None else wq.data_ptr(), None if wk is None else wk.data_ptr(), float(eps),
        None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(),
        0 if cos is None else cos.stride(0), 0 if cos is None else cos.shape[0], dev_state.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), i64array(k_cache.stride()[:3]),
        None if o3 is None else o3.data_ptr(), None if o3 is None else i64array(o3.stride()[:2]), float(scale),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream())
    check(st, "ythip_attn_decode_rope")
    return out


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


# Decode-state record fields (include/ythip.h, ythip_decode_state_field).
ST_GENERATED, ST_ROPE_POS, ST_KV_LEN, ST_SLOT, ST_TOTAL, ST_RING, ST_MAX_POS, ST_HISTORY, ST_ERROR = range(9)
ST_WORDS = 16
ST_ERR_CACHE, ST_ERR_ROPE, ST_ERR_HISTORY = 1, 2, 4


def decode_state_fields(total: int, ring: int, max_pos: int) -> tuple[int, int, int]:
    """(slot, kv_len, rope_pos) of the next token once `total` tokens were
    written to a ring KV cache of `ring` rows: KVCache::append / get_mask and
    Qwen3Model::forward's start rule (example/qwen3/src/qwen3.cpp:70-126,
    365-375) for a one-token step; the device derives the same values
    (csrc/common.hpp, decode_state_derive)."""
    cur = min(total, ring)
    rope = total if total + 1 <= max_pos else (cur if cur + 1 <= max_pos else 0)
    return total % ring, min(total + 1, ring), rope


def decode_state(total: int, ring: int, max_pos: int, generated: int = 0, history: int = 0,
                 device="cuda", out: torch.Tensor | None = None) -> torch.Tensor:
    """The device decode-state record (int32[16]) for a next token after `total`
    written tokens; written into `out` when given (a captured graph's record)."""
    slot, kv_len, rope = decode_state_fields(total, ring, max_pos)
    vals = [0] * ST_WORDS
    vals[ST_GENERATED], vals[ST_ROPE_POS], vals[ST_KV_LEN], vals[ST_SLOT] = generated, rope, kv_len, slot
    vals[ST_TOTAL], vals[ST_RING], vals[ST_MAX_POS], vals[ST_HISTORY] = total, ring, max_pos, history
    t = torch.tensor(vals, dtype=torch.int32)
    if out is None:
        return t.to(device)
    out.copy_(t)
    return out


def rms_norm_rope(qkv: torch.Tensor, Hq: int, Hkv: int, d: int, wq: torch.Tensor | None, wk: torch.Tensor | None,
                  eps: float, cos: torch.Tensor | None, sin: torch.Tensor | None, pos0: int = 0,
                  q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None,
                  v_out: torch.Tensor | None = None, cache_pos: int = 0, dev_state: torch.Tensor | None = None):
    """Fused per-head RMSNorm + RoPE on qkv [B, S, (Hq+2*Hkv)*d].

    Returns (q [B,Hq,S,d], k, v) where k/v are written to rows
    (cache_pos + s) % rows of k_out/v_out [B,Hkv,rows,d] when given (a ring KV
    cache), else to new [B,Hkv,S,d] tensors. dev_state: the decode-state record,
    whose RoPE row and cache slot replace pos0 / cache_pos when the kernel runs.
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
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != h or t.shape[3] != d or t.shape[2] < S:
            raise ValueError(f"{name} has shape {tuple(t.shape)}; needs [{B}, {h}, >={S}, {d}]")
        if t.stride(3) != 1 or t.dtype != dt:
            raise ValueError(f"{name} must have a contiguous last dim and dtype {dt}")
    cache_rows = k_out.shape[2]
    if v_out.shape[2] != cache_rows:
        raise ValueError("k_out and v_out must have the same number of rows")
    if dev_state is None and not 0 <= cache_pos < cache_rows:
        raise ValueError(f"cache_pos {cache_pos} outside the {cache_rows} cache rows")
    if cos is not None and dev_state is None and (cos.shape[0] < pos0 + S or cos.shape[1] < d):
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
        None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(), ld_tab,
        0 if cos is None else cos.shape[0], int(pos0),
        q_out.data_ptr(), i64array(q_out.stride()[:3]),
        k_out.data_ptr(), i64array(k_out.stride()[:3]),
        v_out.data_ptr(), i64array(v_out.stride()[:3]),
        cache_rows, int(cache_pos), None if dev_state is None else dev_state.data_ptr(), _stream())
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
    check(_lib.lib().ythip_embedding(_code(table), _code(out), ids.numel(), table.shape[1], table.shape[0],
                                     table.data_ptr(), ids.data_ptr(), out.data_ptr(), out.stride(0), _stream()),
          "ythip_embedding")
    return out


def _check_state(state: torch.Tensor | None) -> None:
    """The argmax kernels advance a whole decode-state record (int32[16]);
    its HISTORY field must not exceed the history buffer handed with it."""
    if state is not None and (state.dtype != torch.int32 or state.numel() < ST_WORDS or not state.is_contiguous()):
        raise ValueError("state must be the contiguous int32[16] decode-state record (ops.decode_state)")


def argmax_step(logits: torch.Tensor, token: torch.Tensor, history: torch.Tensor | None = None,
                state: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy token (first max index) into token[0]; optionally the history
    entry and the decode-state record's advance (ythip_argmax_step)."""
    _dev(logits, token)
    _check_state(state)
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


def gemv_attn_merge(workspace: torch.Tensor, B: int, Hq: int, d: int, max_ctx: int, weight: torch.Tensor,
                    out: torch.Tensor, alpha: float = 1.0, beta: float = 0.0,
                    dev_state: torch.Tensor | None = None) -> torch.Tensor:
    """Decode-step o projection straight from the split-K partials that
    decode_attention_rope(out=None) left in `workspace`: out [B, N] = alpha *
    merge(partials) @ weight.T + beta * out, weight [N, Hq*d]. Same bits as
    decode_attention_rope(out=attn) followed by gemv_fused(attn, weight, out).
    dev_state: the decode-state record that call ran with; only the splits
    holding keys are then read (None: all of them, same bits)."""
    _dev(workspace, weight, out)
    if dev_state is not None:
        _dev(dev_state)
        if dev_state.dtype != torch.int32 or not dev_state.is_contiguous():
            raise ValueError("dev_state must be a contiguous int32 decode-state record")
    splits = decode_splits(B, Hq, max_ctx)
    n, k = weight.shape
    if k != Hq * d:
        raise ValueError(f"weight must be [N, {Hq * d}]")
    o2 = out.reshape(-1, out.shape[-1])
    if o2.shape != (B, n) or o2.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError(f"out must be [{B}, {n}] with unit column stride")
    ld = Hq * splits * (d + 2)
    if workspace.numel() * workspace.element_size() < B * ld * 4:
        raise ValueError("workspace smaller than the partials")
    check(_lib.lib().ythip_gemv_attn_merge(_code(weight), _code(out), B, n, Hq, d, splits, workspace.data_ptr(), ld,
                                           weight.data_ptr(), weight.stride(0), o2.data_ptr(), o2.stride(0),
                                           float(alpha), float(beta),
                                           None if dev_state is None else dev_state.data_ptr(), int(max_ctx),
                                           _stream()), "ythip_gemv_attn_merge")
    return out


def gemv_swiglu(a: torch.Tensor, gate_up: torch.Tensor, out: torch.Tensor, prologue: str = "none",
                norm_weight: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """Qwen3MLP's gate_up linear + SwiGLU for at most 16 rows (qwen3.cpp:193-200):
    out [m, I] = silu(A' @ gate.T) * (A' @ up.T), gate_up = [gate | up] ([2I, K], the
    fused weight), both products rounded to the weight type first. prologue "none":
    A' = a [m, K]; "rmsnorm": A' = rms_norm(a fp32 [m, K], norm_weight, eps). Same
    bits as gemv_fused into a [m, 2I] buffer followed by silu_mul."""
    _dev(a, gate_up, out)
    if prologue not in ("none", "rmsnorm"):
        raise ValueError("prologue must be 'none' or 'rmsnorm'")
    pro = GEMV_PROLOGUE[prologue]
    n2, k = gate_up.shape
    if n2 % 2:
        raise ValueError("gate_up must have an even number of rows ([gate | up])")
    inter = n2 // 2
    a2 = a.reshape(-1, a.shape[-1])
    o2 = out.reshape(-1, out.shape[-1])
    m = a2.shape[0]
    if o2.shape != (m, inter) or a2.shape[1] != k:
        raise ValueError(f"a must be [m, {k}] and out [m, {inter}]")
    if gate_up.stride(1) != 1 or a2.stride(1) != 1 or o2.stride(1) != 1:
        raise ValueError("gemv_swiglu needs unit column strides")
    if out.dtype != gate_up.dtype:
        raise ValueError("out must have the weight's dtype")
    if a.dtype != (torch.float32 if pro == 1 else gate_up.dtype):
        raise ValueError(f"A has the wrong dtype for prologue {prologue!r}")
    if pro == 1 and (norm_weight is None or norm_weight.dtype != torch.float32):
        raise ValueError("the rmsnorm prologue needs an fp32 norm_weight")
    check(_lib.lib().ythip_gemv_swiglu(pro, _code(gate_up), m, inter, k, a2.data_ptr(), a2.stride(0),
                                       None if norm_weight is None else norm_weight.data_ptr(), float(eps),
                                       gate_up.data_ptr(), gate_up.stride(0), o2.data_ptr(), o2.stride(0),
                                       _stream()), "ythip_gemv_swiglu")
    return out


def argmax_finish(parts: torch.Tensor, n_parts: int, token: torch.Tensor, history: torch.Tensor | None = None,
                  state: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy token from gemv_fused's per-tile (max, index) pairs; as argmax_step."""
    _dev(parts, token)
    _check_state(state)
    check(_lib.lib().ythip_argmax_finish(parts.data_ptr(), int(n_parts), token.data_ptr(),
                                         None if history is None else history.data_ptr(),
                                         None if state is None else state.data_ptr(), _stream()), "ythip_argmax_finish")
    return token


def default_scale(d: int) -> float:
    """scale = 0 -> 1/sqrt(d) (src/function/ops.inl:378-381)."""
    return 1.0 / math.sqrt(d)
