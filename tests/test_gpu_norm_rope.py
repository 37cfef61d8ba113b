"""GPU parity: RMSNorm and fused RMSNorm+RoPE against the oracle's rmsNorm_ and
rope (src/function/normalization.inl:256-267; example/qwen3/src/qwen3.cpp:522-559).
fp32: rel <= 1e-4; bf16: rel <= 2e-2 and MAE <= 1e-3 vs the fp32 CPU path on the
up-converted input."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err
from helpers import check16, dev_f32, host_f32, make_input

pytestmark = pytest.mark.gpu


def _oracle_norm_rope(orc, qkv, B, S, Hq, Hkv, d, wq, wk, eps, cos, sin, pos0):
    x = qkv.reshape(B, S, Hq + 2 * Hkv, d)
    q = np.ascontiguousarray(x[:, :, :Hq].transpose(0, 2, 1, 3))
    k = np.ascontiguousarray(x[:, :, Hq:Hq + Hkv].transpose(0, 2, 1, 3))
    v = np.ascontiguousarray(x[:, :, Hq + Hkv:].transpose(0, 2, 1, 3))
    q = orc.rms_norm(q, wq, eps)
    k = orc.rms_norm(k, wk, eps)
    q = orc.rope(q, cos[pos0:pos0 + S], sin[pos0:pos0 + S])
    k = orc.rope(k, cos[pos0:pos0 + S], sin[pos0:pos0 + S])
    return q, k, v


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("B,S,pos0", [(1, 7, 0), (2, 33, 5), (1, 512, 0)])
def test_norm_rope(orc, yt, dtype, B, S, pos0):
    Hq, Hkv, d = 16, 8, 128
    rng = np.random.default_rng(B * 100 + S)
    qkv = rng.standard_normal((B, S, (Hq + 2 * Hkv) * d)).astype(np.float32)
    wq = (rng.standard_normal(d) * 0.02 + 1.0).astype(np.float32)
    wk = (rng.standard_normal(d) * 0.02 + 1.0).astype(np.float32)
    cos, sin = orc.rope_tables(d, 4096, 1e6)
    qd, qh = make_input(orc, qkv, dtype)
    rq, rk, rv = _oracle_norm_rope(orc, qh, B, S, Hq, Hkv, d, wq, wk, 1e-6, cos, sin, pos0)
    gq, gk, gv = yt.rms_norm_rope(qd, Hq, Hkv, d, dev_f32(wq), dev_f32(wk), 1e-6, dev_f32(cos), dev_f32(sin),
                                  pos0=pos0)
    for name, g, r in (("q", gq, rq), ("k", gk, rk), ("v", gv, rv)):
        g = host_f32(g)
        if dtype == "f32":
            assert rel_err(g, r) <= 1e-4, name
        else:
            check16(orc, g, r, dtype, True, f"{name} B={B} S={S}")


def test_norm_rope_into_cache(orc, yt):
    """K/V land in cache rows cache_pos.. of a [B,Hkv,max,d] buffer; other rows untouched."""
    B, S, Hq, Hkv, d, cache_pos, maxlen = 2, 9, 4, 2, 128, 17, 64
    rng = np.random.default_rng(2)
    qkv = rng.standard_normal((B, S, (Hq + 2 * Hkv) * d)).astype(np.float32)
    w = np.ones(d, np.float32)
    cos, sin = orc.rope_tables(d, 128, 1e6)
    kc = torch.full((B, Hkv, maxlen, d), 7.0, device="cuda")
    vc = torch.full((B, Hkv, maxlen, d), 7.0, device="cuda")
    q, k, v = yt.rms_norm_rope(dev_f32(qkv), Hq, Hkv, d, dev_f32(w), dev_f32(w), 1e-6, dev_f32(cos), dev_f32(sin),
                               pos0=cache_pos, k_out=kc, v_out=vc, cache_pos=cache_pos)
    rq, rk, rv = _oracle_norm_rope(orc, qkv, B, S, Hq, Hkv, d, w, w, 1e-6, cos, sin, cache_pos)
    kh, vh = host_f32(kc), host_f32(vc)
    assert rel_err(kh[:, :, cache_pos:cache_pos + S], rk) <= 1e-4
    assert np.array_equal(vh[:, :, cache_pos:cache_pos + S], rv)
    assert np.all(kh[:, :, :cache_pos] == 7.0) and np.all(kh[:, :, cache_pos + S:] == 7.0)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,n", [(1, 1024), (37, 1024), (512, 1024), (5, 100), (3, 2048), (2, 4000), (2, 5000)])
def test_rms_norm_rows(orc, yt, dtype, rows, n):
    rng = np.random.default_rng(rows + n)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    xd, xh = make_input(orc, x, dtype)
    r = orc.rms_norm(xh, w, 1e-6)
    g = host_f32(yt.rms_norm(xd, dev_f32(w), 1e-6))
    if dtype == "f32":
        assert rel_err(g, r) <= 1e-4
    else:
        check16(orc, g, r, dtype, True, f"rms {rows}x{n}")
