"""Qwen3 decoder: the device-resident model on libythip.so against
the oracle's restatement of the example's fp32 CPU model (which the CPU test
pins bit-exactly to the compiled reference's own qwen3.cpp), on identical
bf16-rounded weights. Bar: greedy argmax tokens identical for the first 32
steps; top-2 margins are logged."""
from __future__ import annotations

import numpy as np
import pytest

import oracle

SMALL = dict(hidden=256, layers=2, vocab=1000, inter=512, n_heads=4, n_kv=2, head_dim=64, max_pos=256)


def _small_weights(orc, cfg, seed=5):
    """Matrices ~ N(0, 0.05), norm weights ~ 1 + N(0, 0.1): larger logit margins
    than the configs[4] recipe, so the small case checks the plumbing with
    margins far above bf16 noise."""
    orc.seed(seed)
    parts = []
    for name, shp in oracle.qwen3_weight_layout(cfg):
        x = orc.randn(int(np.prod(shp)))
        if "norm" in name:
            x = (1.0 + 0.1 * x).astype(np.float32)
        else:
            x = (0.05 * x).astype(np.float32)
        parts.append(orc.bf16_to_f32(orc.bf16_round(x)))
    return np.concatenate(parts)


def test_oracle_qwen3_matches_reference(orc, ref):
    """CPU: the restatement equals the compiled reference's Qwen3ForCausalLM
    bit for bit (first-step logits) and in its greedy tokens."""
    for kw, plen, steps in [(dict(hidden=64, layers=2, vocab=97, inter=128, n_heads=4, n_kv=2, head_dim=16,
                                  max_pos=64), 9, 8), (SMALL, 40, 6)]:
        cfg = oracle.Qwen3Config(**kw)
        W = oracle.qwen3_random_weights(orc, cfg, seed=3)
        pr = oracle.qwen3_prompt(cfg, plen, seed=4)
        to, mo, lo = orc.qwen3_generate(cfg, W, pr, steps)
        tr, mr, lr = ref.qwen3_generate(cfg, W, pr, steps)
        assert np.array_equal(to, tr)
        assert np.array_equal(lo.view(np.uint32), lr.view(np.uint32))


@pytest.mark.gpu
def test_qwen3_small_gpu_tokens_and_logits(orc):
    import torch

    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    kw = SMALL
    cfg_o = oracle.Qwen3Config(**kw)
    W = _small_weights(orc, cfg_o)
    pr = oracle.qwen3_prompt(cfg_o, 37, seed=4)
    steps = 12
    to, mo, lo = orc.qwen3_generate(cfg_o, W, pr, steps)
    m = Qwen3(Qwen3Config(**kw), W, max_ctx=64, max_prompt=64)
    tg = m.generate(pr, steps)
    print("oracle", to, "margins", np.round(mo, 4), "\ngpu   ", tg, flush=True)
    m2 = Qwen3(Qwen3Config(**kw), W, max_ctx=64, max_prompt=64)
    m2.prefill(pr)
    torch.cuda.synchronize()
    lg = m2.logits.float().cpu().numpy()[0]
    rel = np.abs(lg - lo).max() / np.abs(lo).max()
    print("first-step logits rel err", rel, flush=True)
    assert rel <= 2e-2
    assert np.array_equal(tg, to)
    # the graph-replayed decode equals the eager one
    m3 = Qwen3(Qwen3Config(**kw), W, max_ctx=64, max_prompt=64)
    assert np.array_equal(m3.generate(pr, steps, use_graph=False), tg)


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_config5_qwen3_0p6b_greedy_32(orc):
    """Qwen3-0.6B shape, all weights randn*0.02 from seed 3 in the
    layout order, bf16-rounded; 512-token prompt; first 32 greedy tokens must
    equal the fp32 CPU model's on the same (up-converted) weights."""
    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    cfg_o = oracle.Qwen3Config()
    W = oracle.qwen3_random_weights(orc, cfg_o, seed=3)
    pr = oracle.qwen3_prompt(cfg_o, 512, seed=4)
    to, mo, _ = orc.qwen3_generate(cfg_o, W, pr, 32)
    m = Qwen3(Qwen3Config(), W, max_ctx=1024, max_prompt=512)
    tg = m.generate(pr, 32)
    print("oracle", to.tolist(), "\ngpu   ", tg.tolist(), "\nmargins", np.round(mo, 6).tolist(), flush=True)
    assert np.array_equal(tg, to)


@pytest.mark.gpu
def test_qwen3_small_fp16_end_to_end(orc):
    """The whole decoder in fp16 (weights rounded with yt::float16's rule,
    activations, KV cache and GEMM inputs fp16; residual and norms fp32):
    greedy tokens equal the oracle's on the same fp16-representable weights,
    first-step logits within the 16-bit bar, graph replay == eager."""
    import torch

    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    kw = SMALL
    cfg_o = oracle.Qwen3Config(**kw)
    W = _small_weights(orc, cfg_o)
    W16 = orc.f16_to_f32(orc.f16_round(W))  # what the device holds for the matrices
    names = [n for n, _ in oracle.qwen3_weight_layout(cfg_o)]
    sizes = [int(np.prod(s)) for _, s in oracle.qwen3_weight_layout(cfg_o)]
    Wo = W.copy()
    off = 0
    for n, sz in zip(names, sizes):
        if "norm" not in n:
            Wo[off:off + sz] = W16[off:off + sz]
        off += sz
    pr = oracle.qwen3_prompt(cfg_o, 37, seed=4)
    steps = 12
    to, mo, lo = orc.qwen3_generate(cfg_o, Wo, pr, steps)
    m = Qwen3(Qwen3Config(**kw), W, max_ctx=64, max_prompt=64, dtype=torch.float16)
    assert m.embed.dtype == torch.float16 and m.kc.dtype == torch.float16
    tg = m.generate(pr, steps)
    print("oracle", to, "margins", np.round(mo, 4), "\ngpu   ", tg, flush=True)
    m2 = Qwen3(Qwen3Config(**kw), W, max_ctx=64, max_prompt=64, dtype=torch.float16)
    m2.prefill(pr)
    torch.cuda.synchronize()
    lg = m2.logits.float().cpu().numpy()[0]
    rel = np.abs(lg - lo).max() / np.abs(lo).max()
    print("fp16 first-step logits rel err", rel, flush=True)
    assert rel <= 2e-2
    assert np.array_equal(tg, to)
    m3 = Qwen3(Qwen3Config(**kw), W, max_ctx=64, max_prompt=64, dtype=torch.float16)
    assert np.array_equal(m3.generate(pr, steps, use_graph=False), tg)
    # the matrices on the device are exactly yt::float16(w)
    assert np.array_equal(m.embed.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1),
                          orc.f16_round(W[:sizes[0]]))


@pytest.mark.gpu
def test_qwen3_prefill_graph_equals_eager(orc):
    """The captured prefill (one HIP graph per prompt length, replayed) gives
    the eager prefill's bits: logits, residual stream, KV caches and the first
    token, for three prompts of one length through the same graph with eager
    work between the replays, and the decode that follows is unchanged."""
    import torch

    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    cfg_o = oracle.Qwen3Config(**SMALL)
    W = _small_weights(orc, cfg_o)
    a = Qwen3(Qwen3Config(**SMALL), W, max_ctx=64, max_prompt=64)
    b = Qwen3(Qwen3Config(**SMALL), W, max_ctx=64, max_prompt=64)
    for seed in (6, 7, 8):
        pr = oracle.qwen3_prompt(cfg_o, 29, seed=seed)
        a.prefill(pr, use_graph=True)
        b.prefill(pr)
        torch.cuda.synchronize()
        P = len(pr)
        assert torch.equal(a.logits, b.logits), seed
        assert torch.equal(a.x[:P], b.x[:P]), seed
        assert torch.equal(a.kc[:, :, :, :P], b.kc[:, :, :, :P]) and torch.equal(a.vc[:, :, :, :P], b.vc[:, :, :, :P])
        assert torch.equal(a.history[:1], b.history[:1]) and torch.equal(a.state, b.state), seed
    assert len(a.prefill_graphs) == 1
    pr = oracle.qwen3_prompt(cfg_o, 29, seed=9)
    a.prefill(pr, use_graph=True)
    ta = a.generate(pr, 8)  # the prefill graph again, then the decode graph
    assert np.array_equal(ta, b.generate(pr, 8, use_graph=False))


@pytest.mark.gpu
def test_qwen3_fused_decode_equals_unfused(orc):
    """The fused decode step (GEMV prologues, one-kernel attention with q/k
    norm + RoPE + cache append + merge) gives the same bits as the unfused
    per-operator sequence: identical tokens, logits and KV caches."""
    import torch

    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    cfg_o = oracle.Qwen3Config(**SMALL)
    W = _small_weights(orc, cfg_o)
    pr = oracle.qwen3_prompt(cfg_o, 21, seed=5)
    a = Qwen3(Qwen3Config(**SMALL), W, max_ctx=64, max_prompt=64, fused=True)
    b = Qwen3(Qwen3Config(**SMALL), W, max_ctx=64, max_prompt=64, fused=False)
    ta = a.generate(pr, 10)
    tb = b.generate(pr, 10, use_graph=False)
    assert np.array_equal(ta, tb)
    assert torch.equal(a.kc, b.kc) and torch.equal(a.vc, b.vc)
    # one more step each, eager, then compare the logits of the fused head with the unfused head's
    a._decode_step()
    b._decode_step()
    torch.cuda.synchronize()
    assert torch.equal(a.token, b.token)
