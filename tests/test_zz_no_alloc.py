"""ythip_attn_decode_noalloc: the decode attention entry point that takes no
workspace (its split-K partials live in a fixed per-GPU array of the library).
Checked through the C ABI against ythip_attn_decode with a caller workspace:
same kernels, so the outputs must be identical bit for bit -- on two calls in a
row, the second with a smaller input, and after other work on the GPU."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from ytensor_amd import _lib


def _decode_pair(torch, dev, B, Hq, Hkv, ctx, D, lens, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Hkv, ctx, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, ctx, D, generator=g).to(torch.bfloat16).to(dev)
    kv_len = torch.tensor(lens, dtype=torch.int32, device=dev)
    return q, k, v, kv_len


def _call(lib, fn, q, k, v, kv_len, out, ws, stream):
    B, Hq, D = q.shape
    Hkv, ctx = k.shape[1], k.shape[2]
    args = [_lib.BF16, B, Hq, Hkv, D, ctx, q.data_ptr(), _lib.i64array(q.stride()[:2]), k.data_ptr(),
            v.data_ptr(), _lib.i64array(k.stride()[:3]), kv_len.data_ptr(), out.data_ptr(),
            _lib.i64array(out.stride()[:2]), 0.0]
    if fn == "ythip_attn_decode":
        args += [ws.data_ptr(), ws.numel()]
    st = getattr(lib, fn)(*args, stream)
    _lib.check(st, fn)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(dev):
    import torch
    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # first call: B=16 at ctx 2048 (4 splits); second, smaller: B=1 at ctx 700 (6 splits, ragged length)
    for (B, ctx, lens, seed) in [(16, 2048, [2048 - 37 * i for i in range(16)], 11), (1, 700, [613], 12)]:
        q, k, v, kv_len = _decode_pair(torch, dev, B, 16, 8, ctx, 128, lens, seed)
        need = int(lib.ythip_attn_decode_workspace_size(B, 16, ctx, 128))
        assert need <= int(lib.ythip_attn_decode_noalloc_max_bytes())
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        ref = torch.empty(B, 16, 128, dtype=torch.bfloat16, device=dev)
        got = torch.full_like(ref, float("nan"))
        _call(lib, "ythip_attn_decode", q, k, v, kv_len, ref, ws, stream)
        _call(lib, "ythip_attn_decode_noalloc", q, k, v, kv_len, got, None, stream)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"B={B} ctx={ctx}"
        assert torch.isfinite(got.float()).all()
