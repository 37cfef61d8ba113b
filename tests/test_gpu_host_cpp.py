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


def _decode_case(orc, B, ctx):
    orc.seed(2)
    K = _bf16(orc, orc.randn(B, 8, ctx, 128))
    V = _bf16(orc, orc.randn(B, 8, ctx, 128))
    Q = _bf16(orc, orc.randn(B, 16, 1, 128))
    return Q, K, V


@pytest.mark.parametrize("B,ctx", [(1, 1024), (1, 8192), (16, 1024), (16, 8192)])
def test_decode_qwen3_per_token_call_form(orc, outputs, B, ctx):
    """configs[3] in the example's per-token form (qwen3.cpp:250-264): 5-D q,
    repeat_kv'd K/V, the wrapped ring's get_mask bool mask, FLASH_AVX2 -- the
    q_len == 1 branch of flash_attention (flash_attention.inl:469-499)."""
    Q, K, V = _decode_case(orc, B, ctx)
    r = orc.sdpa_gqa(Q, K, V, 1.0 / math.sqrt(128), False)
    g = outputs[f"dec_B{B}_c{ctx}"]
    assert g.shape == (B, 8, 2, 1, 128)
    check16(orc, g.reshape(B, 16, 1, 128), r, "bf16", True, f"C++ decode call form B={B} ctx={ctx}")


def _per_head(orc, Q, K, V, mask, bias):
    """flash_attention per (batch, head) over the GQA mapping h -> h // G."""
    B, Hq = Q.shape[:2]
    G = Hq // K.shape[1]
    out = np.zeros((B, Hq, Q.shape[2], V.shape[3]), np.float32)
    for b in range(B):
        for h in range(Hq):
            out[b, h] = orc.flash_attention(Q[b, h], K[b, h // G], V[b, h // G], 1.0 / math.sqrt(Q.shape[3]),
                                            mask, bias)
    return out


def test_decode_random_mask_and_bias(orc, outputs):
    Q, K, V = _decode_case(orc, 1, 1024)
    orc.seed(21)
    mask = orc.randn(1, 1024) > np.float32(-0.5)
    bias = _bf16(orc, orc.randn(1, 1024))
    assert 0.5 < mask.mean() < 0.9
    r = _per_head(orc, Q, K, V, mask, bias)
    check16(orc, outputs["dec_rand"].reshape(1, 16, 1, 128), r, "bf16", True, "C++ decode mask+bias")


def test_decode_all_masked_is_zero(outputs):
    assert not outputs["dec_none"].any()


def test_decode_predicate(orc, outputs):
    Q, K, V = _decode_case(orc, 1, 1024)
    mask = np.arange(1024)[None, :] <= 512
    r = _per_head(orc, Q, K, V, mask, None)
    check16(orc, outputs["dec_pred"].reshape(1, 16, 1, 128), r, "bf16", True, "C++ decode CausalMask{512}")


def test_decode_group_of_five(orc, outputs):
    orc.seed(22)
    K = _bf16(orc, orc.randn(1, 8, 512, 128))
    V = _bf16(orc, orc.randn(1, 8, 512, 128))
    Q = _bf16(orc, orc.randn(1, 40, 1, 128))
    r = orc.sdpa_gqa(Q, K, V, 1.0 / math.sqrt(128), False)
    check16(orc, outputs["dec_g5"].reshape(1, 40, 1, 128), r, "bf16", True, "C++ decode G=5")


def test_decode_two_threads_two_streams(outputs):
    """Two std::threads, each with its own stream, decoding at once: every one of
    their 24 results has the serial bits (each thread and stream has its own
    split-K workspace)."""
    assert outputs["concurrent"][0] == 0


def test_rmsnorm_out_of_place_and_axes(orc, outputs, golden):
    assert np.array_equal(outputs["rmsnorm_oop"], outputs["rmsnorm"])
    assert rel_err(outputs["rmsnorm_oop"], golden["rmsnorm"]) <= 1e-4
    orc.seed(13)
    x, w = orc.randn(2, 64, 3), orc.randn(64)
    r = orc.rms_norm(np.ascontiguousarray(x.transpose(0, 2, 1)).reshape(-1, 64), w, 1e-6)
    r = r.reshape(2, 3, 64).transpose(0, 2, 1)
    assert rel_err(outputs["rmsnorm_ax1"], r) <= 1e-4
    orc.seed(14)
    x, w = orc.randn(2, 4, 32), orc.randn(4, 32)
    r = orc.rms_norm(x.reshape(2, 128), w.reshape(128), 1e-6).reshape(2, 4, 32)
    assert rel_err(outputs["rmsnorm_ax12"], r) <= 1e-4
