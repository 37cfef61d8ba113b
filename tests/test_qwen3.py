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


def test_qwen3_rejects_bad_requests_before_device_work():
    """Prompt ids outside [0, vocab), empty or oversize prompts and oversize
    generate() requests raise ValueError before anything is uploaded or run:
    the model's buffers live on the CPU here, so any launch would fail
    differently, and the decode-state record and TOTAL stay untouched."""
    torch = pytest.importorskip("torch")
    from ytensor_amd.qwen3 import Qwen3, Qwen3Config, weight_layout
    cfg = Qwen3Config(hidden=64, layers=1, vocab=100, inter=128, n_heads=2, n_kv=1, head_dim=32, max_pos=64)
    total = sum(int(np.prod(s)) for _, s in weight_layout(cfg))
    m = Qwen3(cfg, np.zeros(total, np.float32), device="cpu", max_prompt=16, max_tokens=8)
    state0 = m.state.clone()
    for prompt in ([5, 100], [-1, 3], [7, 2**31 - 1]):
        with pytest.raises(ValueError, match="token ids must lie in"):
            m.prefill(prompt)
    with pytest.raises(ValueError, match="prompt of 0 tokens"):
        m.prefill([])
    with pytest.raises(ValueError, match="prompt of 17 tokens"):
        m.prefill(list(range(17)))
    with pytest.raises(ValueError, match="n_tokens=9"):
        m.generate([1, 2], 9)
    with pytest.raises(ValueError, match="token ids must lie in"):
        m.generate([1, 200], 2)
    assert m.total == 0 and torch.equal(m.state, state0)
    assert int(m.ids.abs().sum()) == 0


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


def _ring_case(orc):
    """A model whose ring KV cache (max_pos = 48 rows, the reference's sizing)
    wraps during the first turn and is full for the next two: 20-token prompt
    + 40 steps, then a 9-token and a 30-token prompt continuing the same
    cache (a full-ring prefill: get_mask's logical-order mask). Seeds picked
    for margins >= 0.017 at every one of the 82 steps."""
    cfg = oracle.Qwen3Config(**dict(SMALL, max_pos=48))
    W = _small_weights(orc, cfg, seed=6)
    rng = np.random.default_rng(6)
    turns = [(rng.integers(0, cfg.vocab, n).astype(np.int32), steps) for n, steps in ((20, 40), (9, 30), (30, 12))]
    return cfg, W, turns


def test_oracle_qwen3_ring_and_turns_match_reference(orc, ref):
    """CPU: past the ring's end and across turns over one cache, the
    restatement equals the compiled reference's Qwen3ForCausalLM bit for bit
    (tokens, margins, logits at the last step of each turn)."""
    cfg, W, turns = _ring_case(orc)
    steps = [39, 69, 81]
    a = orc.qwen3_run(cfg, W, turns, logit_steps=steps)
    b = ref.qwen3_run(cfg, W, turns, logit_steps=steps)
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    assert np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32))
    assert len(set(a[0].tolist())) >= 16 and a[1].min() > 0.015


@pytest.mark.gpu
def test_qwen3_ring_wrap_multi_turn(orc):
    """The device decoder past the ring's end (decode slots wrap, every row
    visible, RoPE row 0 once max_pos is passed) and in two more turns over the
    full ring (continued prefill with the logical-order bool mask): all 82
    greedy tokens equal the oracle's (pinned to the reference's KVCache by the
    CPU test), the last logits of each turn within the 16-bit bar, fused ==
    unfused decode, and the decode-state record ends error-free at TOTAL = 138."""
    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    cfg_o, W, turns = _ring_case(orc)
    steps = [39, 69, 81]
    to, mo, lo = orc.qwen3_run(cfg_o, W, turns, logit_steps=steps)
    for fused in (True, False):
        m = Qwen3(Qwen3Config(**dict(SMALL, max_pos=48)), W, max_prompt=64, fused=fused)
        assert m.max_ctx == 48
        got = []
        for t, (pr, n) in enumerate(turns):
            tg = m.generate(pr, n, reset=(t == 0), use_graph=fused)
            got.append(tg)
            lg = m.logits.float().cpu().numpy()[0]
            rel = np.abs(lg - lo[t]).max() / np.abs(lo[t]).max()
            print(f"fused={fused} turn {t}: logits rel err {rel:.3e}", flush=True)
            assert rel <= 2e-2
        tg = np.concatenate(got)
        print("oracle", to.tolist(), "\ngpu   ", tg.tolist(), "\nmargins", np.round(mo, 4).tolist(), flush=True)
        assert np.array_equal(tg, to), f"first difference at step {int(np.argmax(tg != to))}"
        assert m.total == sum(len(p) + n - 1 for p, n in turns) == 138


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
@pytest.mark.timeout(600)
def test_config5_discriminating_0p6b_greedy_32(orc):
    """configs[4]'s shape, seeded stream, layout and 512-token prompt with the
    discriminating init (matrices randn * 0.03, RMSNorm weights 1 + 0.1 *
    randn; tests/golden/cases.py QWEN3_VAR), against the fixture the compiled
    reference's own Qwen3ForCausalLM wrote (qwen3.cpp:365-457, 506-516): its
    32-token greedy stream holds 26 distinct tokens. All 32 device tokens must
    equal the reference's, and at every step the device logits at the
    reference's 16 largest and at 1024 fixed entries must be within
    max|g - r| / max|r| <= 2e-2 (the bf16 bar). Margins and errors are printed."""
    import os

    import torch

    from tests.golden import cases
    from ytensor_amd.qwen3 import Qwen3, Qwen3Config
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_qwen3_0p6b_var.npz"))
    r = cases.QWEN3_VAR
    cfg_o = oracle.Qwen3Config()
    W = oracle.qwen3_random_weights(orc, cfg_o, seed=r["seed"], scale=r["scale"], norm_spread=r["norm_spread"])
    pr = oracle.qwen3_prompt(cfg_o, r["prompt_len"], seed=r["prompt_seed"])
    assert np.array_equal(pr, fx["prompt"])
    ref_tok = fx["tokens"]
    assert len(set(ref_tok.tolist())) >= 8
    m = Qwen3(Qwen3Config(), W, max_ctx=1024, max_prompt=512)
    del W
    m.prefill(pr, use_graph=True)
    m.capture()
    worst = 0.0
    for k in range(r["steps"]):
        if k > 0:
            m.graph.replay()
        torch.cuda.synchronize()
        lg = m.logits.float().cpu().numpy()[0]
        ri = np.concatenate([fx["top_idx"][k], fx["sample_idx"]])
        rv = np.concatenate([fx["top_val"][k], fx["sample_val"][k]])
        rel = float(np.abs(lg[ri] - rv).max() / np.abs(rv).max())
        worst = max(worst, rel)
        print(f"step {k:2d}: ref token {int(ref_tok[k]):6d} margin {float(fx['margins'][k]):.4f} "
              f"gpu token {int(lg.argmax()):6d} logits rel err {rel:.3e}", flush=True)
        assert rel <= 2e-2, k
    m.total += r["steps"] - 1
    m.check_state()
    tg = m.history[:r["steps"]].cpu().numpy()
    print("reference", ref_tok.tolist(), "\ngpu      ", tg.tolist(), f"\nworst logits rel err {worst:.3e}",
          flush=True)
    assert np.array_equal(tg, ref_tok), f"first difference at step {int(np.argmax(tg != ref_tok))}"


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
