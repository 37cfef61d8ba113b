"""GPU: the MATH attention backend (ythip_attn_math), masked matmul
(ythip_gemm_masked), predicate / diagonal masks and strided or broadcast K/V
on the flash path, against the oracle's restatements (pinned to the reference
in test_oracle_math.py).

Bars: fp32 max|g - r| <= 1e-4 * max|r| (attention outputs: 1e-4 absolute on
O(1) values); bf16 / fp16 the 2e-2 / MAE 1e-3 bar of check16, with the oracle
run on the same 16-bit-rounded inputs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import check16

pytestmark = pytest.mark.gpu


def _t(x, dev, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev).to(dt)


def _f(t):
    return t.float().cpu().numpy()


def _ref_heads(orc, Q, K, V, kw, backend):
    """Q [H, Lq, D] etc. -> oracle output, MATH restatement or flash."""
    if backend == "math":
        return orc.sdpa_math(Q, K, V, 0.0, **kw)
    mask, diag, bias = kw.get("mask"), kw.get("diag"), kw.get("bias")
    Lq, Lkv = Q.shape[1], K.shape[1]
    if diag is not None:
        mask = np.arange(Lkv)[None, :] <= np.arange(Lq)[:, None] + diag
    return np.stack([orc.flash_attention(Q[h], K[h], V[h], 1 / np.sqrt(np.float32(Q.shape[2])), mask, bias)
                     for h in range(Q.shape[0])])


def _mask_arg(kw, Lq, Lkv):
    if "diag" in kw:
        return ("diag", kw["diag"])
    if "pred" in kw:
        off = kw["pred"]
        return lambda i, j: j <= i + off
    return kw.get("mask_t")


CASES = [  # (H, Lq, Lkv, D, Dv, mask form)
    (2, 7, 9, 16, 16, None),
    (3, 40, 70, 64, 64, "bool"),
    (2, 64, 64, 128, 128, "causal"),
    (2, 33, 50, 64, 32, "diag5"),
    (1, 20, 20, 32, 32, "pred0"),
    (2, 16, 24, 64, 64, "bool_bias"),
    (1, 9, 9, 8, 8, "diag-3"),
]


def _case(orc, case, seed):
    H, Lq, Lkv, D, Dv, form = case
    rng = np.random.default_rng(seed)
    Q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    K = rng.standard_normal((H, Lkv, D)).astype(np.float32)
    V = rng.standard_normal((H, Lkv, Dv)).astype(np.float32)
    kw, arg = {}, {}
    if form in ("bool", "bool_bias"):
        m = rng.random((Lq, Lkv)) < 0.6
        m[1] = False
        kw["mask"] = m
        arg["mask_t"] = torch.from_numpy(m)
        if form == "bool_bias":
            b = rng.standard_normal((Lq, Lkv)).astype(np.float32)
            kw["bias"] = b
            arg["bias"] = b
    elif form == "causal":
        kw["diag"] = Lkv - Lq
        arg["causal"] = True
    elif form is not None and form.startswith("diag"):
        kw["diag"] = int(form[4:])
        arg["diag"] = kw["diag"]
    elif form is not None and form.startswith("pred"):
        kw["diag"] = int(form[4:])
        arg["pred"] = kw["diag"]
    return Q, K, V, kw, arg


@pytest.mark.parametrize("backend", ["math", "flash"])
@pytest.mark.parametrize("case", CASES)
def test_sdpa_backends_fp32_vs_oracle(orc, yt, dev, backend, case):
    Q, K, V, kw, arg = _case(orc, case, 5)
    mask = "causal" if arg.get("causal") else _mask_arg(arg, Q.shape[1], K.shape[1])
    bias = _t(arg["bias"], dev) if "bias" in arg else None
    got = yt.scaled_dot_product_attention(_t(Q, dev), _t(K, dev), _t(V, dev), 0.0, mask=mask, bias=bias,
                                          backend=backend)
    torch.cuda.synchronize()
    ref = _ref_heads(orc, Q, K, V, kw, backend)
    assert np.abs(_f(got) - ref).max() <= 1e-4, (backend, case)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", [CASES[1], CASES[2], CASES[3], CASES[5]])
def test_sdpa_math_16bit_vs_oracle(orc, yt, dev, dt, case):
    Q, K, V, kw, arg = _case(orc, case, 6)
    rnd = (lambda x: orc.bf16_to_f32(orc.bf16_round(x))) if dt == torch.bfloat16 else \
        (lambda x: orc.f16_to_f32(orc.f16_round(x)))
    Q, K, V = rnd(Q), rnd(K), rnd(V)
    mask = "causal" if arg.get("causal") else _mask_arg(arg, Q.shape[1], K.shape[1])
    bias = _t(arg["bias"], dev) if "bias" in arg else None
    got = yt.scaled_dot_product_attention(_t(Q, dev, dt), _t(K, dev, dt), _t(V, dev, dt), 0.0, mask=mask,
                                          bias=bias, backend="math")
    torch.cuda.synchronize()
    ref = orc.sdpa_math(Q, K, V, 0.0, **kw)
    check16(orc, _f(got), ref, "bf16" if dt == torch.bfloat16 else "f16", True, f"math {case}")


@pytest.mark.parametrize("backend", ["math", "flash"])
def test_ymodel2_pega2_layout(orc, yt, dev, backend):
    """The ymodel2 example's attention (example/ymodel2-s-2/ymodel2.cpp:188-262):
    q [b, 2, hh, l, hd]; k = repeat_kv of a [b, 2, L, hd] cache (0-stride over
    hh); v = the cache's second half repeated over the first axis (0-stride);
    the cache stored transposed ([b, 2, hd, L], read through .transpose) and a
    ring-wrapped bool causal mask."""
    rng = np.random.default_rng(8)
    b, hh, l, L, hd = 2, 4, 5, 23, 64
    q = rng.standard_normal((b, 2, hh, l, hd)).astype(np.float32)
    cache_t = rng.standard_normal((b, 2, hd, L)).astype(np.float32)  # transposed storage
    wp = 7  # ring write position: logical order starts at wp
    mask = np.zeros((l, L), bool)
    for qi in range(l):
        for ki in range(L):
            mask[qi, ki] = (ki - wp + L) % L <= L - l + qi
    kvc = torch.from_numpy(cache_t).to(dev)
    kv = kvc.transpose(-1, -2)                          # [b, 2, L, hd], d-stride L
    k5 = kv.unsqueeze(2).expand(b, 2, hh, L, hd)        # repeat_kv: 0-stride over hh
    v5 = kv[:, 1:2].expand(b, 2, L, hd).unsqueeze(2).expand(b, 2, hh, L, hd)
    out = yt.scaled_dot_product_attention(_t(q, dev), k5, v5, 0.125, mask=torch.from_numpy(mask), backend=backend)
    torch.cuda.synchronize()
    kv_np = np.swapaxes(cache_t, -1, -2)
    for bi in range(b):
        for s in range(2):
            for j in range(hh):
                K = kv_np[bi, s][None]
                Vv = kv_np[bi, 1][None]
                if backend == "math":
                    ref = orc.sdpa_math(q[bi, s, j][None], K, Vv, 0.125, mask=mask)[0]
                else:
                    ref = orc.flash_attention(q[bi, s, j], K[0], Vv[0], 0.125, mask)
                assert np.abs(_f(out[bi, s, j]) - ref).max() <= 1e-4


def test_flash_transposed_keys_decode_and_prefill(orc, yt, dev):
    """K and V stored [B, H, D, L] (d-major) on the flash path: the row-wise
    kernel reads them through their strides (the reference copies to contiguous
    for q_len > 1 and reads strided for q_len == 1, ops.inl:176-189)."""
    rng = np.random.default_rng(9)
    B, H, L, D = 1, 2, 300, 64
    kt = rng.standard_normal((B, H, D, L)).astype(np.float32)
    vt = rng.standard_normal((B, H, D, L)).astype(np.float32)
    for Lq in (1, 17):
        q = rng.standard_normal((B, H, Lq, D)).astype(np.float32)
        kd, vd = _t(kt, dev), _t(vt, dev)
        out = yt.scaled_dot_product_attention(_t(q, dev), kd.transpose(-1, -2), vd.transpose(-1, -2), 0.0,
                                              mask="causal")
        torch.cuda.synchronize()
        K, V = np.swapaxes(kt, -1, -2)[0], np.swapaxes(vt, -1, -2)[0]
        ref = orc.sdpa_math(q[0], K, V, 0.0, diag=L - Lq)
        assert np.abs(_f(out[0]) - ref).max() <= 1e-4


def test_flash_diag_masks_on_mfma_path_bf16(orc, yt, dev):
    """Diagonal offsets on the 16-bit MFMA kernel (offset 0 on a rectangular
    problem, negative offsets with rows that see no key)."""
    rng = np.random.default_rng(10)
    H, Lq, Lkv, D = 2, 200, 300, 128
    rnd = lambda x: orc.bf16_to_f32(orc.bf16_round(x))  # noqa: E731
    Q = rnd(rng.standard_normal((H, Lq, D)).astype(np.float32))
    K = rnd(rng.standard_normal((H, Lkv, D)).astype(np.float32))
    V = rnd(rng.standard_normal((H, Lkv, D)).astype(np.float32))
    for off in (0, -40, 150, 10000, -10000):
        got = yt.scaled_dot_product_attention(_t(Q, dev, torch.bfloat16)[None], _t(K, dev, torch.bfloat16)[None],
                                              _t(V, dev, torch.bfloat16)[None], 0.0, mask=("diag", off))
        torch.cuda.synchronize()
        ref = orc.sdpa_math(Q, K, V, 0.0, diag=off)
        check16(orc, _f(got[0]), ref, "bf16", True, f"diag {off}")
        if off <= -Lq:
            assert torch.count_nonzero(got) == 0


@pytest.mark.parametrize("m,n,k", [(13, 17, 32), (256, 384, 128), (1000, 520, 64), (3, 4096, 256)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0)])
def test_gemm_masked_fp32(orc, yt, dev, m, n, k, alpha, beta):
    rng = np.random.default_rng(m + n + k)
    A = rng.standard_normal((m, k)).astype(np.float32)
    B = rng.standard_normal((k, n)).astype(np.float32)
    C = rng.standard_normal((m, n)).astype(np.float32)
    mask = rng.random((m, n)) < 0.5
    out = _t(C, dev)
    yt.gemm_masked(_t(A, dev), _t(B, dev), out, torch.from_numpy(mask), alpha, beta)
    torch.cuda.synchronize()
    ref = orc.sgemm_masked(A, B, C.copy(), mask, alpha, beta)
    got = _f(out)
    assert np.array_equal(got[~mask], C[~mask])
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_masked_matmul_16bit_batched_predicates(orc, yt, dev, dt):
    rng = np.random.default_rng(12)
    bt, m, n, k = 3, 96, 130, 64
    rnd = (lambda x: orc.bf16_to_f32(orc.bf16_round(x))) if dt == torch.bfloat16 else \
        (lambda x: orc.f16_to_f32(orc.f16_round(x)))
    A = rnd(rng.standard_normal((bt, m, k)).astype(np.float32))
    B = rnd(rng.standard_normal((k, n)).astype(np.float32))
    for mask, diag in ((None, 3), (lambda i, j: (i + j) % 3 != 0, None), ("causal", n - m)):
        got = yt.masked_matmul(_t(A, dev, dt), _t(B, dev, dt), mask if mask is not None else ("diag", diag),
                               masked_value=-8192.0)
        torch.cuda.synchronize()
        if callable(mask):
            mk = np.fromfunction(lambda i, j: (i + j) % 3 != 0, (m, n), dtype=int)
            refs = [orc.masked_matmul(A[i], B, mask=mk, value=-8192.0) for i in range(bt)]
        else:
            refs = [orc.masked_matmul(A[i], B, diag=diag, value=-8192.0) for i in range(bt)]
        ref = np.stack(refs)
        vis = ref != -8192.0
        g = _f(got)
        assert np.all(g[~vis] == -8192.0)
        check16(orc, g[vis], ref[vis], "bf16" if dt == torch.bfloat16 else "f16", True, f"masked {mask}")


def test_math_edge_cases(yt, dev):
    q = torch.randn(1, 2, 4, 16, device=dev)
    k = torch.randn(1, 2, 0, 16, device=dev)
    v = torch.randn(1, 2, 0, 8, device=dev)
    out = yt.scaled_dot_product_attention(q, k, v, backend="math")
    torch.cuda.synchronize()
    assert out.shape == (1, 2, 4, 8) and torch.count_nonzero(out) == 0
    with pytest.raises(ValueError):
        yt.scaled_dot_product_attention(q, k, v, backend="eigen")
    k = torch.randn(1, 2, 6, 16, device=dev)
    v = torch.randn(1, 2, 6, 8, device=dev)
    with pytest.raises(ValueError):
        yt.scaled_dot_product_attention(q, k, v, mask=torch.ones(3, 6, dtype=torch.bool), backend="math")


@pytest.mark.parametrize("Lkv", [1500, 4096, 5000])
def test_math_long_rows(orc, yt, dev, Lkv):
    """Rows of up to 1024 / 4096 keys are read once into registers; longer
    rows take the three-pass softmax. Both against the oracle."""
    rng = np.random.default_rng(Lkv)
    H, Lq, D = 2, 8, 64
    Q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    K = rng.standard_normal((H, Lkv, D)).astype(np.float32)
    V = rng.standard_normal((H, Lkv, D)).astype(np.float32)
    m = rng.random((Lq, Lkv)) < 0.5
    m[3] = False
    b = rng.standard_normal((Lq, Lkv)).astype(np.float32)
    got = yt.scaled_dot_product_attention(_t(Q, dev), _t(K, dev), _t(V, dev), 0.0, mask=torch.from_numpy(m),
                                          bias=_t(b, dev), backend="math")
    torch.cuda.synchronize()
    ref = orc.sdpa_math(Q, K, V, 0.0, mask=m, bias=b)
    assert np.abs(_f(got) - ref).max() <= 1e-4
    assert torch.count_nonzero(got[:, 3]) == 0
