"""configs[4] through the C++ host: the Qwen3 decoder of include/yt/qwen3.hpp
(the example's Qwen3ForCausalLM, example/qwen3/src/qwen3.cpp:193-516, over
include/yt/ytensor.hpp and libythip.so), built into ytensor_amd/bin/yt_qwen3
from tests/cpp/qwen3_host.cpp.

The program draws the Qwen3-0.6B weights itself with YTensor::seed / randn in
the model's layout order (the discriminating recipe of tests/golden/cases.py
QWEN3_VAR), runs the fixture's 512-token prompt through the prompt graph and 31
replays of the captured decode step, and writes every step's logits. Checked
against the fixture the compiled reference's own Qwen3ForCausalLM wrote: all 32
greedy tokens equal, and at every step the logits at the reference's 16 largest
and at 1024 fixed entries within max|g - r| / max|r| <= 2e-2 (the bf16 bar).
Its generate() on a fresh cache must return the same 32 tokens."""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "ytensor_amd", "bin", "yt_qwen3")


@pytest.mark.timeout(600)
def test_cpp_host_qwen3_0p6b_matches_reference_fixture(tmp_path):
    from tests.golden import cases
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built (python -m ytensor_amd.build)")
    fx = np.load(os.path.join(ROOT, "tests", "golden", "reference_qwen3_0p6b_var.npz"))
    r = cases.QWEN3_VAR
    prompt = fx["prompt"].astype(np.int32)
    pf = tmp_path / "prompt.i32"
    prompt.tofile(pf)
    steps = r["steps"]
    p = subprocess.run([EXE, "fixture", str(pf), str(tmp_path), str(steps), str(r["seed"]), str(r["scale"]),
                        str(r["norm_spread"])], capture_output=True, text=True, timeout=540)
    print(p.stdout, p.stderr, flush=True)
    assert p.returncode == 0, p.stderr
    tokens = np.fromfile(tmp_path / "tokens.i32", dtype=np.int32)
    gen = np.fromfile(tmp_path / "generate.i32", dtype=np.int32)
    logits = np.fromfile(tmp_path / "logits.f32", dtype=np.float32).reshape(steps, -1)
    ref_tok = fx["tokens"]
    worst = 0.0
    for k in range(steps):
        ri = np.concatenate([fx["top_idx"][k], fx["sample_idx"]])
        rv = np.concatenate([fx["top_val"][k], fx["sample_val"][k]])
        rel = float(np.abs(logits[k][ri] - rv).max() / np.abs(rv).max())
        worst = max(worst, rel)
        print(f"step {k:2d}: ref token {int(ref_tok[k]):6d} C++ token {int(tokens[k]):6d} "
              f"argmax {int(logits[k].argmax()):6d} logits rel err {rel:.3e}", flush=True)
        assert rel <= 2e-2, k
    print(f"worst logits rel err {worst:.3e}", flush=True)
    assert np.array_equal(tokens, ref_tok), f"first difference at step {int(np.argmax(tokens != ref_tok))}"
    assert np.array_equal(gen, ref_tok), "generate() on a fresh cache differs from the step-by-step run"
