"""The C++ host boundary on the GPU: tests/cpp/host_parity.cpp (built into
ytensor_amd/bin by the package build) drives the reference's own operator
signatures -- YTensor::matmul with MatmulBackend::HIP, yt::function::linear,
scaledDotProductAttention in the Qwen3 example's call form (5-D q, repeat_kv'd
K/V, bool causal mask, FLASH_AVX2), with a CausalMask predicate and FLASH_HIP,
through MATH, the q_len == 1 decode, and rmsNorm_ -- over include/yt/ytensor.hpp
and libythip.so, on inputs from YTensor::seed / randn. Its outputs are checked
here against the reference's golden fixtures (randn, configs[0] GEMM samples,
rmsNorm_) and against the oracle (pinned to the reference) at the north-star
tolerances: fp32 rel <= 1e-4; bf16 rel <= 2e-2 and MAE <= 1e-3 (or 1.1x the
bf16 output-rounding floor)."""
from __future__ import annotations

import math
import os
import subprocess

import numpy as np
import pytest

from conftest import rel_err
from helpers import check16

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "ytensor_amd", "bin", "yt_host_parity")


@pytest.fixture(scope="module")
def outputs(tmp_path_factory):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built (python -m ytensor_amd.build)")
    d = tmp_path_factory.mktemp("host_parity")
    p = subprocess.run([EXE, str(d)], capture_output=True, text=True, timeout=300)
    print(p.stdout, p.stderr, flush=True)
    assert p.returncode == 0, p.stderr
    shapes = {}
    for line in p.stdout.splitlines():
        if ":" in line:
            k, v = line.split(":", 1)
            shapes[k] = tuple(int(x) for x in v.split())
    out = {}
    for k, shp in shapes.items():
        out[k] = np.fromfile(os.path.join(d, k + ".f32"), dtype=np.float32).reshape(shp)
    return out


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(ROOT, "tests", "golden", "reference_small.npz"))


def _bf16(orc, x):
    return orc.bf16_to_f32(orc.bf16_round(x))


def test_randn_is_the_references(outputs, golden):
    assert np.array_equal(outputs["randn0_head"].view(np.uint32), golden["randn0_head"].view(np.uint32))


def test_config1_fp32_matmul_hip_backend(outputs, golden):
    from tests.golden import cases
    g = outputs["c0"].reshape(-1)
    idx = cases.sample_index(1024 * 1024)
    assert rel_err(g[idx], golden["gemm1024_sample"]) <= 1e-4


def test_config2_bf16_matmul_and_linear(orc, outputs):
    M, N, K = 128, 3072, 1024
    orc.seed(0)
    A = _bf16(orc, orc.randn(M, K))
    B = _bf16(orc, (orc.randn(K, N) * np.float32(0.02)).astype(np.float32))
    check16(orc, outputs["c1_nn"], orc.sgemm(A, B), "bf16", True, "C++ matmul NN")
    orc.seed(0)
    A = _bf16(orc, orc.randn(M, K))
    W = _bf16(orc, (orc.randn(N, K) * np.float32(0.02)).astype(np.float32))
    check16(orc, outputs["c1_nt"], orc.sgemm(A, W, b_trans=True), "bf16", True, "C++ linear")


def test_linear_with_bias_fp32(orc, outputs):
    orc.seed(5)
    x, w, b = orc.randn(33, 64), orc.randn(40, 64), orc.randn(40)
    r = (orc.sgemm(x, w, b_trans=True) + b[None, :]).astype(np.float32)
    assert rel_err(outputs["c1_bias"], r) <= 1e-4


def _prefill_ref(orc):
    S, D = 256, 128
    orc.seed(1)
    Q = _bf16(orc, orc.randn(1, 16, S, D))
    K = _bf16(orc, orc.randn(1, 8, S, D))
    V = _bf16(orc, orc.randn(1, 8, S, D))
    return orc.sdpa_gqa(Q, K, V, 1.0 / math.sqrt(D), True)


@pytest.mark.parametrize("name", ["prefill", "prefill_pred", "prefill_math"])
def test_causal_gqa_prefill_qwen3_call_form(orc, outputs, name):
    r = _prefill_ref(orc)
    g = outputs[name]
    assert g.shape == (1, 8, 2, 256, 128)
    check16(orc, g.reshape(1, 16, 256, 128), r, "bf16", True, f"C++ {name}")


def test_decode_one_query(orc, outputs):
    D, ctx = 128, 1024
    orc.seed(2)
    K = _bf16(orc, orc.randn(1, 8, ctx, D))
    V = _bf16(orc, orc.randn(1, 8, ctx, D))
    Q = _bf16(orc, orc.randn(1, 16, 1, D))
    r = orc.sdpa_gqa(Q, K, V, 1.0 / math.sqrt(D), False)
    g = outputs["decode"]
    assert g.shape == (1, 8, 2, 1, 128)
    check16(orc, g.reshape(1, 16, 1, 128), r, "bf16", True, "C++ decode")


def test_rmsnorm_inplace(outputs, golden):
    assert rel_err(outputs["rmsnorm"], golden["rmsnorm"]) <= 1e-4
