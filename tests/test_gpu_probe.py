"""The roofline probes of libythip_probe.so (ytensor_amd/probe.py) compute what
they claim: the MFMA probe's output is bf16(steps * A . B^T) per wave, and
the DMA probe's LDS holds exactly the headline GEMM's A and B slices of the last
two k steps for each tile, in the GEMM's XCD-aware tile order."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ytensor_amd import probe
    probe.load()
    return torch, torch.device("cuda", 0)


def tile_coords(w: int, tiles_m: int, tiles_n: int) -> tuple[int, int]:
    """The GEMM grids' tile order (common.hpp tile_coords)."""
    T = tiles_m * tiles_n
    if T % 8 == 0:
        w = (w % 8) * (T // 8) + w // 8
    in_group = 4 * tiles_n
    g = w // in_group
    first = 4 * g
    gsize = min(tiles_m - first, 4)
    r = w - g * in_group
    return first + r % gsize, r // gsize


@pytest.mark.parametrize("workgroups,steps", [(1, 1), (3, 5), (256, 2)])
def test_mfma_probe_is_steps_times_the_product(torch_dev, workgroups, steps):
    torch, dev = torch_dev
    from ytensor_amd import probe
    W = 8 * workgroups
    g = torch.Generator(device="cpu").manual_seed(workgroups * 100 + steps)
    A = torch.randn(W, 128, 64, generator=g).to(torch.bfloat16)
    B = torch.randn(W, 64, 64, generator=g).to(torch.bfloat16)
    out = torch.full((W, 128, 64), float("nan"), device=dev, dtype=torch.bfloat16)
    probe.mfma_ceiling(A.to(dev), B.to(dev), out, workgroups, steps)
    torch.cuda.synchronize()
    a, b = A.double(), B.double()
    ref = steps * torch.bmm(a, b.transpose(1, 2).contiguous())
    # fp32 accumulation, then one rounding to bf16: half an ulp, at most 2^-8
    # of the value (8 significant bits)
    bound = 2.0 ** -8 * ref.abs() + 1e-5 * steps * torch.bmm(a.abs(), b.abs().transpose(1, 2).contiguous()) + 1e-30
    err = (out.cpu().double() - ref).abs()
    assert torch.isfinite(out).all()
    assert (err <= bound).all(), float((err / bound).max())


def _slice_sums(a_u32: np.ndarray, b_u32: np.ndarray, m0: int, n0: int, k: int) -> np.ndarray:
    """Component-wise uint32 sums (mod 2^32) over the 16-byte chunks of A's rows
    m0..m0+255 and B's columns n0..n0+255 for the last two 64-wide k steps."""
    kt = k // 64
    sa = a_u32[m0:m0 + 256, (kt - 2) * 32:kt * 32].reshape(-1, 4).astype(np.uint64).sum(0)
    sb = b_u32[(kt - 2) * 64:kt * 64, n0 // 2:n0 // 2 + 128].reshape(-1, 4).astype(np.uint64).sum(0)
    return ((sa + sb) % (1 << 32)).astype(np.uint64)


@pytest.mark.parametrize("M,N,K", [(512, 768, 256), (1024, 512, 192), (4096, 4096, 4096)])
def test_dma_probe_lands_the_gemm_slices(torch_dev, M, N, K):
    torch, dev = torch_dev
    from ytensor_amd import probe
    g = torch.Generator(device="cpu").manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = torch.randn(K, N, generator=g).to(torch.bfloat16)
    tm_, tn_ = M // 256, N // 256
    out = torch.zeros(tm_ * tn_, 512, 16, dtype=torch.uint8, device=dev)
    probe.dma_ceiling(A.to(dev), B.to(dev), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(tm_ * tn_, 512, 4).astype(np.uint64).sum(1) % (1 << 32)
    a_u32 = A.view(torch.int16).numpy().view(np.uint32).reshape(M, K // 2)
    b_u32 = B.view(torch.int16).numpy().view(np.uint32).reshape(K, N // 2)
    for w in range(tm_ * tn_):
        tm, tn = tile_coords(w, tm_, tn_)
        np.testing.assert_array_equal(got[w], _slice_sums(a_u32, b_u32, tm * 256, tn * 256, K), err_msg=f"wg {w}")

