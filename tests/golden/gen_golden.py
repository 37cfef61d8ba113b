"""Write the golden fixtures under tests/golden/ from the COMPILED REFERENCE.

Runs only where /root/reference exists and `make -C oracle ref` built
oracle/_ref/libytref.so (the reference's own sources compiled as they lie).
The reference ships no tests or vectors of its own, so these fixtures are
the pins: every output below comes from the reference's functions
(yt::YTensor::seed/randn, yt::bfloat16, yt::float16, avx2::sgemm,
avx2::flash_attention, scaledDotProductAttention(FLASH_AVX2), rmsNorm_,
qwen3::RoPECache / ops::rope_k, qwen3::Qwen3ForCausalLM). Inputs are
regenerated in the tests from the pinned RNG, so only outputs are stored.

    python tests/golden/gen_golden.py            # small fixtures
    python tests/golden/gen_golden.py --qwen3    # + the configs[4] 0.6B run (minutes)
    python tests/golden/gen_golden.py --qwen3-var  # only the discriminating 0.6B run (minutes)
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
sys.path.insert(0, HERE)
import cases  # noqa: E402


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--qwen3", action="store_true")
    ap.add_argument("--qwen3-var", action="store_true")
    args = ap.parse_args()
    ref = oracle.reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libytref.so is not built (make -C oracle ref)")
    if args.qwen3_var:
        qwen3_var(ref)
        return
    out = {}
    for s in cases.RANDN_SEEDS:
        ref.seed(s)
        x = ref.randn(cases.RANDN_N)
        out[f"randn{s}_head"] = x[:64]
        out[f"randn{s}_sha256"] = np.array(cases.digest(x))
    kat = cases.conversion_inputs()
    out["kat_in"] = kat
    out["kat_bf16"] = ref.bf16_round(kat)
    out["kat_f16"] = ref.f16_round(kat)
    allh = np.arange(65536, dtype=np.uint16)
    out["kat_bf16_to_f32"] = ref.bf16_to_f32(allh)
    out["kat_f16_to_f32"] = ref.f16_to_f32(allh)
    for name, (A, B, bt) in cases.gemm_cases(ref).items():
        out[f"gemm_{name}"] = ref.sgemm(A, B, b_trans=bt)
    A, B = cases.gemm_1024(ref)
    C = ref.sgemm(A, B)
    out["gemm1024_sha256"] = np.array(cases.digest(C))
    out["gemm1024_sample"] = C.reshape(-1)[cases.sample_index(C.size)]
    for name, (Q, K, V, scale, mask, bias) in cases.flash_cases(ref).items():
        out[f"flash_{name}"] = ref.flash_attention(Q, K, V, scale, mask, bias)
    Q, K, V = cases.sdpa_case(ref)
    out["sdpa_gqa_causal"] = ref.sdpa_gqa(Q, K, V, 0.0, True)
    out["sdpa_gqa_decode"] = ref.sdpa_gqa(np.ascontiguousarray(Q[:, :, -1:]), K, V, 0.0, True)
    X, w = cases.norm_case(ref)
    out["rmsnorm"] = ref.rms_norm(X, w, 1e-6)
    c, s = ref.rope_tables(128, 4096, 1e6)
    out["rope_cos_sha256"] = np.array(cases.digest(c))
    out["rope_sin_sha256"] = np.array(cases.digest(s))
    out["rope_cos_rows"] = c[[0, 1, 7, 511, 4095]]
    X = cases.rope_case(ref)
    out["rope"] = ref.rope(X, c, s)
    cfg, W, pr, steps = cases.qwen3_tiny(ref)
    t, m, lg = ref.qwen3_generate(cfg, W, pr, steps)
    out["qwen3_tiny_tokens"], out["qwen3_tiny_margins"], out["qwen3_tiny_logits0"] = t, m, lg
    np.savez_compressed(os.path.join(HERE, "reference_small.npz"), **out)
    print("wrote reference_small.npz:", len(out), "arrays")
    if args.qwen3:
        cfg = oracle.Qwen3Config()
        W = oracle.qwen3_random_weights(ref, cfg, seed=3)
        pr = oracle.qwen3_prompt(cfg, 512, seed=4)
        t, m, lg = ref.qwen3_generate(cfg, W, pr, 32)
        np.savez_compressed(os.path.join(HERE, "reference_qwen3_0p6b.npz"), tokens=t, margins=m,
                            logits0_head=lg[:4096], logits0_sha256=np.array(cases.digest(lg)),
                            prompt=pr)
        print("wrote reference_qwen3_0p6b.npz", t)


def qwen3_var(ref) -> None:
    """The configs[4] shape with a discriminating random init: the same seeded
    stream and layout as configs[4], matrices randn * 0.03 and every RMSNorm
    weight 1 + 0.1 * randn (cases.QWEN3_VAR), the same 512-token prompt, 32
    greedy steps through the reference's Qwen3ForCausalLM. Stored per step: the
    token, the top-1 - top-2 margin, the logits' SHA-256, the 16 largest logits
    (index, value) and the logits at 1024 fixed indices."""
    cfg = oracle.Qwen3Config()
    r = cases.QWEN3_VAR
    W = oracle.qwen3_random_weights(ref, cfg, seed=r["seed"], scale=r["scale"], norm_spread=r["norm_spread"])
    pr = oracle.qwen3_prompt(cfg, r["prompt_len"], seed=r["prompt_seed"])
    steps = r["steps"]
    t, m, lg = ref.qwen3_run(cfg, W, [(pr, steps)], logit_steps=list(range(steps)))
    idx = cases.sample_index(cfg.vocab, 1024)
    top = np.argsort(-lg, axis=1, kind="stable")[:, :16]
    np.savez_compressed(os.path.join(HERE, "reference_qwen3_0p6b_var.npz"), tokens=t, margins=m,
                        logits_sha256=np.array([cases.digest(x) for x in lg]),
                        top_idx=top.astype(np.int32), top_val=np.take_along_axis(lg, top, 1),
                        sample_idx=idx.astype(np.int32), sample_val=lg[:, idx], prompt=pr,
                        recipe=np.array(repr(sorted(r.items()))))
    print("wrote reference_qwen3_0p6b_var.npz", t.tolist(), "min margin", float(m.min()))


if __name__ == "__main__":
    main()
