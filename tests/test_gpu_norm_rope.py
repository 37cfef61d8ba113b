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


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("d", [64, 128])
def test_norm_rope_long_prompt(orc, yt, dtype, d):
    """65568 (token, head) rows at d = 64 and 128; 2049 tokens leave a partly
    filled last workgroup."""
    B, S, pos0, Hq, Hkv = 1, 2049, 3, 16, 8
    rng = np.random.default_rng(d + 7)
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
            check16(orc, g, r, dtype, True, f"{name} d={d} S={S}")


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


def test_norm_rope_ring_write_wraps(orc, yt):
    """K/V rows go to (cache_pos + s) % rows, the ring write of KVCache::append
    (example/qwen3/src/qwen3.cpp:70-88): 9 tokens from row 15 of a 20-row cache
    land in rows 15..19 and 0..3; rows 4..14 are untouched."""
    B, S, Hq, Hkv, d, cache_pos, rows = 1, 9, 4, 2, 128, 15, 20
    rng = np.random.default_rng(44)
    qkv = rng.standard_normal((B, S, (Hq + 2 * Hkv) * d)).astype(np.float32)
    w = (rng.standard_normal(d) * 0.1 + 1.0).astype(np.float32)
    cos, sin = orc.rope_tables(d, 64, 1e6)
    kc = torch.full((B, Hkv, rows, d), 7.0, device="cuda")
    vc = torch.full((B, Hkv, rows, d), 7.0, device="cuda")
    yt.rms_norm_rope(dev_f32(qkv), Hq, Hkv, d, dev_f32(w), dev_f32(w), 1e-6, dev_f32(cos), dev_f32(sin),
                     pos0=30, k_out=kc, v_out=vc, cache_pos=cache_pos)
    rq, rk, rv = _oracle_norm_rope(orc, qkv, B, S, Hq, Hkv, d, w, w, 1e-6, cos, sin, 30)
    kh, vh = host_f32(kc), host_f32(vc)
    order = [(cache_pos + s) % rows for s in range(S)]
    assert rel_err(kh[:, :, order], rk) <= 1e-4
    assert np.array_equal(vh[:, :, order], rv)
    assert np.all(kh[:, :, 4:15] == 7.0) and np.all(vh[:, :, 4:15] == 7.0)
    with pytest.raises(ValueError):  # a host cache_pos outside the ring is refused before any launch
        yt.rms_norm_rope(dev_f32(qkv), Hq, Hkv, d, None, None, 1e-6, None, None, k_out=kc, v_out=vc, cache_pos=rows)


@pytest.mark.parametrize("fused", [False, True])
def test_decode_state_out_of_range_flags_and_skips(orc, yt, fused):
    """A decode-state record whose cache slot or RoPE row lies outside the cache
    / table sets the ERROR bits and neither writes the cache row nor reads the
    table row. The cache and the tables are views into larger buffers with a
    sentinel slab right behind them, so an access past the end would land in
    owned memory and show up as a changed sentinel."""
    ops = yt.ops
    Hq, Hkv, d, rows, tab = 4, 2, 64, 32, 40
    rng = np.random.default_rng(45)
    big_k = torch.full((1, Hkv, rows + 4, d), 3.0, dtype=torch.bfloat16, device="cuda")
    big_v = torch.full_like(big_k, 3.0)
    kc, vc = big_k[:, :, :rows], big_v[:, :, :rows]
    cos, sin = orc.rope_tables(d, tab + 4, 1e6)
    cos_d, sin_d = dev_f32(cos), dev_f32(sin)
    qkv = torch.from_numpy(rng.standard_normal((1, (Hq + 2 * Hkv) * d)).astype(np.float32)).cuda().to(torch.bfloat16)
    ws = torch.empty(ops.decode_workspace_bytes(1, Hq, rows, d), dtype=torch.uint8, device="cuda")
    for field, bad, bit in ((ops.ST_SLOT, rows, ops.ST_ERR_CACHE), (ops.ST_ROPE_POS, tab, ops.ST_ERR_ROPE)):
        st = ops.decode_state(5, rows, tab)
        st[field] = bad
        before_k, before_v = big_k.clone(), big_v.clone()
        if fused:
            o = torch.empty((1, Hq, d), dtype=torch.bfloat16, device="cuda")
            ops.decode_attention_rope(qkv, Hq, Hkv, d, None, None, 1e-6, cos_d[:tab], sin_d[:tab], st, kc, vc, o, ws)
        else:
            qd = torch.empty((1, Hq, 1, d), dtype=torch.bfloat16, device="cuda")
            yt.rms_norm_rope(qkv.view(1, 1, -1), Hq, Hkv, d, None, None, 1e-6, cos_d[:tab], sin_d[:tab], q_out=qd,
                             k_out=kc, v_out=vc, dev_state=st)
        torch.cuda.synchronize()
        assert int(st[ops.ST_ERROR]) & bit, (field, st.tolist())
        assert torch.equal(big_k[:, :, rows:], before_k[:, :, rows:]) and torch.equal(big_v[:, :, rows:],
                                                                                     before_v[:, :, rows:])
        if field == ops.ST_SLOT:  # no cache row changed at all
            assert torch.equal(big_k, before_k) and torch.equal(big_v, before_v)


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
