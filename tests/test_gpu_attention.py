"""GPU parity: ythip_attn_prefill / ythip_attn_decode against the oracle's
restatement of YTensor's FLASH_AVX2 path (src/kernel/avx2/flash_attention.inl).

Tolerances: fp32 max|g-r|/max|r| <= 1e-4; bf16/fp16 <= 2e-2 and MAE <= 1e-3
(16-bit outputs: max(1e-3, 1.1 * output-rounding floor)) against the fp32 CPU
result on the up-converted inputs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import rel_err
from helpers import TORCH_DT, check16, dev_f32, host_f32, make_input

pytestmark = pytest.mark.gpu


def _check(orc, g, r, dtype, label):
    if dtype == "f32":
        e = rel_err(g, r)
        print(f"{label}: rel={e:.3e}", flush=True)
        assert e <= 1e-4, f"{label}: {e}"
    else:
        check16(orc, g, r, dtype, True, label)


@pytest.mark.parametrize("S", [512, 2048, 8192])
def test_config3_causal_prefill_bf16(orc, yt, S):
    """B=1, 16 q heads, 8 kv heads, d=128, Q,K,V ~ N(0,1) from seed 1
    (drawn in that order), [B,H,S,D], scale 1/sqrt(128), causal."""
    orc.seed(1)
    Q = orc.randn(1, 16, S, 128)
    K = orc.randn(1, 8, S, 128)
    V = orc.randn(1, 8, S, 128)
    Qd, Qh = make_input(orc, Q, "bf16")
    Kd, Kh = make_input(orc, K, "bf16")
    Vd, Vh = make_input(orc, V, "bf16")
    r = orc.sdpa_gqa(Qh, Kh, Vh, 1.0 / math.sqrt(128), True)
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, 1.0 / math.sqrt(128), mask="causal"))
    check16(orc, g, r, "bf16", True, f"prefill S={S}")


def _causal_rows_ref(orc, Qh, Kh, Vh, rows, diag_off):
    """The reference's flash_attention on a subset of query rows of every head
    (rows i see keys j <= i + diag_off), q head h on kv head h // G."""
    B, Hq, S, D = Qh.shape
    G = Hq // Kh.shape[1]
    Skv = Kh.shape[2]
    m = np.arange(Skv)[None, :] <= (rows[:, None] + diag_off)
    out = np.zeros((B, Hq, len(rows), D), np.float32)
    for b in range(B):
        for h in range(Hq):
            out[b, h] = orc.flash_attention(Qh[b, h, rows], Kh[b, h // G], Vh[b, h // G], 1.0 / math.sqrt(D), m)
    return out


@pytest.mark.parametrize("S", [2048, 8192])
def test_config3_causal_prefill_fp32_mfma(orc, yt, S):
    """configs[2]'s shapes in fp32 -- the dtype of the reference's flash path
    (src/function/ops.inl:119-121) -- on the v_mfma_f32_16x16x4_f32 kernel: Q,
    K, V ~ N(0,1) from seed 1 in that order, causal, rel <= 1e-4 against the
    reference's fp32 flash_attention. S=2048: every row; S=8192: the first and
    last 96 rows and 96 rows around the middle of every head."""
    orc.seed(1)
    Q = orc.randn(1, 16, S, 128)
    K = orc.randn(1, 8, S, 128)
    V = orc.randn(1, 8, S, 128)
    g = host_f32(yt.scaled_dot_product_attention(dev_f32(Q), dev_f32(K), dev_f32(V), 1.0 / math.sqrt(128),
                                                 mask="causal"))
    if S <= 2048:
        r = orc.sdpa_gqa(Q, K, V, 1.0 / math.sqrt(128), True)
        e = rel_err(g, r)
    else:
        rows = np.concatenate([np.arange(96), np.arange(S // 2 - 48, S // 2 + 48), np.arange(S - 96, S)])
        r = _causal_rows_ref(orc, Q, K, V, rows, 0)
        e = rel_err(g[:, :, rows], r)
    print(f"fp32 causal prefill S={S}: rel={e:.3e}", flush=True)
    assert e <= 1e-4


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kind", ["none", "diag", "bool", "bias", "bool_bias"])
@pytest.mark.parametrize("grid", ["split", "whole"])
def test_prefill_fp32_mfma_mask_kinds(orc, yt, D, kind, grid):
    """The fp32 MFMA kernel's mask forms against the reference's flash_attention:
    ragged q / kv lengths (not multiples of the query and 64-key blocks), GQA
    4:1, B = 2; a diagonal predicate with a negative offset (leading rows see no
    key -> zeros), a bool mask with a fully masked row, an additive bias. "split":
    a grid short of two 128-query blocks per CU, which runs 64-query blocks with
    each staged key block split between the two wave groups; "whole": 640
    128-query blocks, one wave group per query block."""
    if grid == "split":
        B, Hq, Hkv, Sq, Skv = 2, 8, 2, 201, 333
    else:
        B, Hq, Hkv, Sq, Skv = 2, 64, 16, 520, 601
    rng = np.random.default_rng(D + len(kind))
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    mask = bias = None
    mnp = bnp = None
    if kind == "none":
        mnp = None
    elif kind == "diag":
        mask = ("diag", -5)
        mnp = np.arange(Skv)[None, :] <= np.arange(Sq)[:, None] - 5
    if kind in ("bool", "bool_bias"):
        mnp = rng.random((Sq, Skv)) > 0.35
        mnp[7] = False
        mask = torch.from_numpy(mnp).cuda()
    if kind in ("bias", "bool_bias"):
        bnp = rng.standard_normal((Sq, Skv)).astype(np.float32)
        bias = torch.from_numpy(bnp).cuda()
    g = host_f32(yt.scaled_dot_product_attention(dev_f32(Q), dev_f32(K), dev_f32(V), 0.0, mask=mask, bias=bias))
    r = np.zeros_like(g)
    for b in range(B):
        for h in range(Hq):
            r[b, h] = orc.flash_attention(Q[b, h], K[b, h // 4], V[b, h // 4], 1.0 / math.sqrt(D), mnp, bnp)
    e = rel_err(g, r)
    print(f"fp32 mfma {kind} D={D}: rel={e:.3e}", flush=True)
    assert e <= 1e-4
    if kind in ("bool", "bool_bias"):
        assert not g[:, :, 7].any()
    if kind == "diag":
        assert not g[:, :, :5].any()


CASES = [
    # (B, Hq, Hkv, Sq, Skv, D, mask)
    (1, 2, 1, 5, 9, 64, None),
    (1, 4, 2, 13, 13, 128, "causal"),
    (2, 4, 4, 70, 70, 128, "causal"),
    (1, 2, 1, 33, 70, 128, "causal"),     # kv longer than q: causal offset kv-q
    (1, 2, 2, 130, 130, 64, "causal"),
    (1, 2, 1, 200, 333, 128, None),
    (1, 2, 1, 17, 40, 128, "bool"),       # bool mask with a fully masked row
    (1, 2, 1, 17, 40, 128, "bias"),       # additive bias
    (1, 4, 1, 64, 64, 128, "causal"),     # GQA 4:1
]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_prefill_cases(orc, yt, case, dtype):
    B, Hq, Hkv, Sq, Skv, D, mk = case
    rng = np.random.default_rng(Sq * 7 + Skv)
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    scale = 1.0 / math.sqrt(D)
    mask = bias = None
    mask_np = None
    bias_np = None
    if mk == "causal":
        mask = "causal"
        mask_np = np.tril(np.ones((Sq, Skv), bool), Skv - Sq)
    elif mk == "bool":
        mask_np = rng.random((Sq, Skv)) > 0.4
        mask_np[3] = False
        mask = torch.from_numpy(mask_np).cuda()
    elif mk == "bias":
        bias_np = rng.standard_normal((Sq, Skv)).astype(np.float32)
        bias = dev_f32(bias_np)
    r = np.zeros((B, Hq, Sq, D), np.float32)
    for b in range(B):
        for h in range(Hq):
            kh = h // (Hq // Hkv)
            r[b, h] = orc.flash_attention(Qh[b, h], Kh[b, kh], Vh[b, kh], scale, mask_np, bias_np)
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask=mask, bias=bias))
    if mk == "bool":
        assert np.all(g[:, :, 3] == 0.0)  # fully masked row -> zeros (flash_attention.inl:327-331)
    _check(orc, g, r, dtype, f"{case} {dtype}")


def _staged_mask(kind, Sq, Skv, rng):
    if kind == "random":
        m = rng.random((Sq, Skv)) > 0.4
    elif kind == "blocks":
        # 64-key blocks wholly hidden from some row groups, whole for others, and an empty row
        m = np.zeros((Sq, Skv), bool)
        for qb in range(0, Sq, 16):
            for kb in range(0, Skv, 64):
                sel = (qb // 16 + kb // 64) % 3
                if sel == 1:
                    m[qb:qb + 16, kb:kb + 64] = True
                elif sel == 2:
                    m[qb:qb + 16, kb:kb + 64] = rng.random((min(16, Sq - qb), min(64, Skv - kb))) > 0.5
        m[5] = False
    elif kind == "wgblocks":
        # whole 128-row x 64-key regions hidden, whole or mixed in turn: a workgroup's
        # next key block alternates between skipped (no K/V staged) and loaded
        m = np.zeros((Sq, Skv), bool)
        for qb in range(0, Sq, 128):
            for kb in range(0, Skv, 64):
                sel = (qb // 128 + kb // 64) % 3
                if sel == 1:
                    m[qb:qb + 128, kb:kb + 64] = True
                elif sel == 2:
                    m[qb:qb + 128, kb:kb + 64] = rng.random((min(128, Sq - qb), min(64, Skv - kb))) > 0.5
        m[200] = False
    elif kind == "ring":
        # KVCache::get_mask once the ring is full (example/qwen3/src/qwen3.cpp:115-123):
        # physical key ki has logical position (ki - write_pos) mod max_len
        wp = 77
        ki = np.arange(Skv)[None, :]
        qi = np.arange(Sq)[:, None]
        m = ((ki - wp + Skv) % Skv) <= (Skv - Sq) + qi
    else:
        m = np.tril(np.ones((Sq, Skv), bool), Skv - Sq)
    return m


STAGED_CASES = [(d, k, sq, skv, hq, hkv, 1) for d in ("bf16", "f16")
                for (k, sq, skv, hq, hkv) in [("random", 200, 336, 2, 1), ("blocks", 300, 512, 4, 2),
                                              ("ring", 96, 256, 4, 2), ("causal", 513, 1024, 2, 2),
                                              ("blocks", 1100, 1040, 2, 1)]]
# GQA pairs with >= 512 paired workgroups: two heads per workgroup, the mask staged
# one key block ahead of K/V, key blocks no row of a workgroup sees skipped whole
STAGED_CASES += [("bf16", k, 2048, 2048, 16, 8, 4) for k in ("causal", "ring", "wgblocks")]
# the same shapes through the tile-class list (ops passes the workspace): every
# tile mixed, a partial last key block and query block, 16-row regions
STAGED_CASES += [("bf16", "random", 2048, 2096, 16, 8, 4), ("f16", "blocks", 2000, 2096, 16, 8, 4)]
STAGED_CASES = [c + (128,) for c in STAGED_CASES]
# the tile-class path at head dim 64 (its DMA slot count and swizzle masks differ)
STAGED_CASES += [("bf16", "random", 2048, 2096, 16, 8, 4, 64), ("f16", "blocks", 2000, 2096, 16, 8, 4, 64)]


@pytest.mark.parametrize("dtype,kind,Sq,Skv,Hq,Hkv,B,D", STAGED_CASES)
def test_prefill_bool_mask_staged(orc, yt, dtype, kind, Sq, Skv, Hq, Hkv, B, D):
    """Bool masks with 16-byte aligned rows take the staged MFMA path (mask tile
    per key block in LDS, all-false blocks skipped, all-true blocks unmasked; a
    partial last key block reads its bytes directly): against the oracle's
    flash_attention with the same mask (src/kernel/avx2/flash_attention.inl:
    335-379), fully masked rows zero."""
    rng = np.random.default_rng(Sq + Skv)
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    m = _staged_mask(kind, Sq, Skv, rng)
    assert Skv % 16 == 0  # 16-byte aligned mask rows
    scale = 1.0 / math.sqrt(D)
    r = np.zeros((B, Hq, Sq, D), np.float32)
    for b in range(B):
        for h in range(Hq):
            kh = h // (Hq // Hkv)
            r[b, h] = orc.flash_attention(Qh[b, h], Kh[b, kh], Vh[b, kh], scale, m, None)
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask=torch.from_numpy(m).cuda()))
    empty = ~m.any(axis=1)
    assert np.all(g[:, :, empty] == 0.0)
    check16(orc, g, r, dtype, True, f"staged mask {kind} B={B} {Hq}/{Hkv} heads {Sq}x{Skv} {dtype}")


def _prefill_abi(yt, q, k, v, o, mask, ws):
    """ythip_attn_prefill (ws None) or ythip_attn_prefill_ws on [B, H, S, D] tensors."""
    from ytensor_amd import _lib
    from ytensor_amd.ops import _stream, i64array
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    code = _lib.BF16 if q.dtype == torch.bfloat16 else _lib.F16
    args = (code, B, Hq, Hkv, Sq, Skv, D, D, q.data_ptr(), i64array(q.stride()), k.data_ptr(),
            i64array(k.stride()), v.data_ptr(), i64array(v.stride()), o.data_ptr(), i64array(o.stride()),
            1.0 / math.sqrt(D), _lib.MASK_BOOL, mask.data_ptr(), mask.stride(0), None, 0, 0)
    if ws is None:
        return _lib.lib().ythip_attn_prefill(*args, _stream())
    return _lib.lib().ythip_attn_prefill_ws(*args, ws.data_ptr(), ws.numel(), _stream())


@pytest.mark.parametrize("Sq,Skv", [(2048, 2048), (2000, 2096)])
def test_prefill_bool_tiles_equal_causal(yt, Sq, Skv):
    """A causal mask given as bytes, through the tile-class list, takes the same
    blocks, masks and order as the causal kind on the ping-pong kernel: the
    outputs agree bit for bit. Without the workspace the staged-mask kernel runs
    (oracle-checked above); it is held to bf16 rounding here, though on these
    masks it has matched bit for bit too."""
    B, Hq, Hkv, D = 4, 16, 8, 128
    g = torch.Generator().manual_seed(Sq + Skv)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(torch.bfloat16).cuda()
    mk = torch.ones(Sq, Skv, dtype=torch.bool).tril(Skv - Sq).cuda()
    ref = yt.scaled_dot_product_attention(q, k, v, 1.0 / math.sqrt(D), "causal")
    got = yt.scaled_dot_product_attention(q, k, v, 1.0 / math.sqrt(D), mk)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    need = int(__import__("ytensor_amd")._lib.lib().ythip_attn_prefill_workspace_size(Sq, Skv))
    assert need == -(-((Sq + 31) // 32) * ((Skv + 63) // 64) // 256) * 256
    m8 = mk.view(torch.uint8)
    o_ws = torch.empty_like(q)
    assert _prefill_abi(yt, q, k, v, o_ws, m8, torch.empty(need, dtype=torch.uint8, device="cuda")) == 0
    o_plain = torch.empty_like(q)
    assert _prefill_abi(yt, q, k, v, o_plain, m8, None) == 0
    torch.cuda.synchronize()
    assert torch.equal(o_ws, ref)
    d = (o_plain.float() - ref.float()).abs()
    print(f"bool tiles {Sq}x{Skv}: staged-kernel max|d| {d.max().item():.3e} mean {d.mean().item():.3e}", flush=True)
    assert d.mean().item() < 1e-3 and d.max().item() < 3e-2
    # one byte short of the tile table: an argument error, nothing launched
    assert _prefill_abi(yt, q, k, v, o_ws, m8, torch.empty(need - 1, dtype=torch.uint8, device="cuda")) != 0


# Two query heads per workgroup without a byte mask (>= 512 paired workgroups):
# the ping-pong kernel, on ragged lengths, a causal offset, d = 64 and fp16.
PINGPONG_CASES = [
    ("bf16", 4, 16, 8, 2048, 2048, 128, "causal"),
    ("bf16", 4, 16, 8, 2000, 2100, 128, "causal"),   # kv longer than q, partial last blocks
    ("bf16", 4, 16, 8, 2048, 1500, 128, "none"),
    ("f16", 4, 16, 8, 2047, 2047, 128, "causal"),
    ("bf16", 4, 16, 4, 2048, 2048, 64, "causal"),    # d = 64, GQA 4:1 (two head pairs per kv head)
]


@pytest.mark.parametrize("dtype,B,Hq,Hkv,Sq,Skv,D,mk", PINGPONG_CASES)
def test_prefill_paired_heads(orc, yt, dtype, B, Hq, Hkv, Sq, Skv, D, mk):
    rng = np.random.default_rng(Sq * 3 + Skv + D)
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    scale = 1.0 / math.sqrt(D)
    r = orc.sdpa_gqa(Qh, Kh, Vh, scale, mk == "causal")
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask="causal" if mk == "causal" else None))
    check16(orc, g, r, dtype, True, f"paired heads B={B} {Hq}/{Hkv} {Sq}x{Skv} d={D} {mk} {dtype}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prefill_key_halves(orc, yt, dtype):
    """Short prompts split each 128-key stage between two wave groups (keys 0-63
    and 64-127 of the stage) and merge their O, l, m at the end. Closed forms,
    exact: a row whose only visible key is k gives V[k], for k in either half and
    in a later stage (one group saw nothing); a row whose two visible keys a, b
    (one per half) have the same K row gives (V[a] + V[b]) / 2 (both groups set,
    equal reference points). Then a causal and a random byte mask over 300 keys
    (three stages, a partial one) against the oracle."""
    rng = np.random.default_rng(21)
    D, Sq, Skv = 128, 40, 200  # a 200-byte mask row is not 16-byte aligned: read per element
    Q = rng.standard_normal((1, 1, Sq, D)).astype(np.float32)
    K = rng.standard_normal((1, 1, Skv, D)).astype(np.float32)
    V = rng.standard_normal((1, 1, Skv, D)).astype(np.float32)
    K[0, 0, 64:128] = K[0, 0, 0:64]  # key 64 + j has the K row of key j
    Qd, _ = make_input(orc, Q, dtype)
    Kd, _ = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    tdt = TORCH_DT[dtype]
    scale = 1.0 / math.sqrt(D)

    keys = np.array([30, 100, 150, 199])[np.arange(Sq) % 4]
    m = np.zeros((Sq, Skv), bool)
    m[np.arange(Sq), keys] = True
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask=torch.from_numpy(m).cuda()))
    assert np.array_equal(g[0, 0], Vh[0, 0][keys]), "single visible key"

    ka = (np.arange(Sq) * 7) % 64
    m = np.zeros((Sq, Skv), bool)
    m[np.arange(Sq), ka] = True
    m[np.arange(Sq), ka + 64] = True
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask=torch.from_numpy(m).cuda()))
    expect = torch.from_numpy((Vh[0, 0][ka] + Vh[0, 0][ka + 64]) * np.float32(0.5)).to(tdt).float().numpy()
    assert np.array_equal(g[0, 0], expect), "two keys with equal scores, one per half"

    B, Hq, Hkv, S = 1, 4, 2, 300
    Q = rng.standard_normal((B, Hq, S, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    r = orc.sdpa_gqa(Qh, Kh, Vh, scale, True)
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask="causal"))
    check16(orc, g, r, dtype, True, f"key halves causal {dtype}")
    mk = rng.random((S, S)) > 0.7
    mk[7] = False
    r = np.stack([np.stack([orc.flash_attention(Qh[0, h], Kh[0, h // 2], Vh[0, h // 2], scale, mk, None)
                            for h in range(Hq)])])
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask=torch.from_numpy(mk).cuda()))
    assert np.all(g[:, :, 7] == 0.0)
    check16(orc, g, r, dtype, True, f"key halves byte mask {dtype}")


def test_prefill_strided_views(orc, yt):
    """q/k/v as [B,S,H,D] memory viewed as [B,H,S,D] (the qwen3 permute views)."""
    rng = np.random.default_rng(4)
    B, Hq, Hkv, S, D = 2, 4, 2, 48, 128
    Qm = rng.standard_normal((B, S, Hq, D)).astype(np.float32)
    Km = rng.standard_normal((B, S, Hkv, D)).astype(np.float32)
    Vm = rng.standard_normal((B, S, Hkv, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Qm, "bf16")
    Kd, Kh = make_input(orc, Km, "bf16")
    Vd, Vh = make_input(orc, Vm, "bf16")
    g = host_f32(yt.scaled_dot_product_attention(Qd.permute(0, 2, 1, 3), Kd.permute(0, 2, 1, 3),
                                                  Vd.permute(0, 2, 1, 3), 0.0, mask="causal"))
    r = orc.sdpa_gqa(Qh.transpose(0, 2, 1, 3), Kh.transpose(0, 2, 1, 3), Vh.transpose(0, 2, 1, 3), 0.0, True)
    check16(orc, g, r, "bf16", True, "strided")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_huge_key_row_stride(orc, yt, dtype):
    """K rows 2^23 + 8 (bf16) / 2^23 + 4 (fp32) elements apart: one stage of K
    spans more than 2^31 bytes, so the MFMA prefill kernels take their DMA
    path with per-stage offsets instead of the fixed 32-bit lane offsets. The
    output must equal the contiguous-K call bit for bit, and the oracle."""
    S = 256 if dtype == "bf16" else 128
    ks2 = (1 << 23) + (8 if dtype == "bf16" else 4)
    rng = np.random.default_rng(23)
    Q = rng.standard_normal((1, 2, S, 128)).astype(np.float32)
    K = rng.standard_normal((1, 1, S, 128)).astype(np.float32)
    V = rng.standard_normal((1, 1, S, 128)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    buf = torch.zeros((S - 1) * ks2 + 128, dtype=Kd.dtype, device=Kd.device)
    Kw = torch.as_strided(buf, (1, 1, S, 128), (0, 0, ks2, 1))
    Kw.copy_(Kd)
    esz = 2 if dtype == "bf16" else 4
    rows = 128 if dtype == "bf16" else 64  # K rows per DMA stage of the kernel this shape runs
    assert rows * ks2 * esz >= 1 << 31
    g_wide = host_f32(yt.scaled_dot_product_attention(Qd, Kw, Vd, 0.0, mask="causal"))
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, 0.0, mask="causal"))
    del Kw, buf
    torch.cuda.empty_cache()
    assert np.array_equal(g_wide, g)
    r = orc.sdpa_gqa(Qh, Kh, Vh, 0.0, True)
    _check(orc, g, r, dtype, f"huge key row stride {dtype}")


def _decode_inputs(orc, B, ctx, seed=2):
    orc.seed(seed)
    K = orc.randn(B, 8, ctx, 128)
    V = orc.randn(B, 8, ctx, 128)
    Q = orc.randn(B, 16, 1, 128)
    return Q, K, V


@pytest.mark.parametrize("B,ctx", [(1, 1024), (1, 8192), (16, 1024), (16, 8192)])
def test_config4_decode_bf16(orc, yt, B, ctx):
    """one query per sequence over a [B,8,ctx,128] cache; K, V, Q ~
    N(0,1) from seed 2 drawn in that order; no mask beyond the cache length."""
    Q, K, V = _decode_inputs(orc, B, ctx)
    Qd, Qh = make_input(orc, Q, "bf16")
    Kd, Kh = make_input(orc, K, "bf16")
    Vd, Vh = make_input(orc, V, "bf16")
    r = orc.sdpa_gqa(Qh, Kh, Vh, 0.0, True)
    g = host_f32(yt.decode_attention(Qd, Kd, Vd))
    check16(orc, g.reshape(r.shape), r, "bf16", True, f"decode B={B} ctx={ctx}")


def _per_head_flash(orc, Qh, Kh, Vh, mask, bias):
    """The reference's flash_attention per (batch, head), q head h on kv head h // G."""
    B, Hq = Qh.shape[:2]
    G = Hq // Kh.shape[1]
    out = np.zeros((B, Hq, Qh.shape[2], Vh.shape[3]), np.float32)
    for b in range(B):
        for h in range(Hq):
            out[b, h] = orc.flash_attention(Qh[b, h], Kh[b, h // G], Vh[b, h // G],
                                            1.0 / math.sqrt(Qh.shape[3]), mask, bias)
    return out


@pytest.mark.parametrize("kind", ["none", "causal", "bool_all", "bool_rand", "bias", "diag"])
@pytest.mark.parametrize("B,ctx", [(1, 1024), (1, 8192), (16, 1024), (16, 8192)])
def test_single_query_sdpa_every_mask_kind(orc, yt, B, ctx, kind):
    """scaled_dot_product_attention with q_len == 1 -- the reference's per-token
    call (flash_attention.inl:469-499 sends every mask kind to its decode path)
    -- at configs[3]'s shapes: against the reference's flash_attention per head,
    and, with every key visible, bit for bit the explicit decode entry point
    (both run the split-K decode kernel with the same splits)."""
    Q, K, V = _decode_inputs(orc, B, ctx)
    Qd, Qh = make_input(orc, Q, "bf16")
    Kd, Kh = make_input(orc, K, "bf16")
    Vd, Vh = make_input(orc, V, "bf16")
    rng = np.random.default_rng(ctx + B)
    mask = bias = None
    mnp = bnp = None
    if kind == "causal":
        mask = "causal"
    elif kind == "bool_all":
        mnp = np.ones((1, ctx), bool)
        mask = torch.from_numpy(mnp).cuda()
    elif kind == "bool_rand":
        mnp = rng.random((1, ctx)) > 0.3
        mask = torch.from_numpy(mnp).cuda()
    elif kind == "bias":
        bnp = rng.standard_normal((1, ctx)).astype(np.float32)
        bias = torch.from_numpy(bnp).cuda()
    elif kind == "diag":
        mask = ("diag", ctx // 3)
        mnp = np.arange(ctx)[None, :] <= ctx // 3
    g = yt.scaled_dot_product_attention(Qd, Kd, Vd, 0.0, mask=mask, bias=bias)
    if mnp is None and bnp is None:
        r = orc.sdpa_gqa(Qh, Kh, Vh, 0.0, False)
        ref_dec = yt.decode_attention(Qd, Kd, Vd)
        assert torch.equal(g.view(torch.int16), ref_dec.view(torch.int16)), "routed != decode entry point bits"
    else:
        r = _per_head_flash(orc, Qh, Kh, Vh, mnp, bnp)
    if kind == "bool_all":
        ref_dec = yt.decode_attention(Qd, Kd, Vd)
        assert torch.equal(g.view(torch.int16), ref_dec.view(torch.int16)), "all-true mask != unmasked bits"
    check16(orc, host_f32(g).reshape(r.shape), r, "bf16", True, f"q_len=1 {kind} B={B} ctx={ctx}")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_single_query_sdpa_strided_v_and_no_workspace(orc, yt, dtype):
    """q_len == 1 with K and V of different layouts (V a [B,S,H,D] view), through
    ythip_attn_prefill without a workspace (one split per kv head, written
    straight to O) and with one; fully masked rows stay zero."""
    B, Hq, Hkv, S, D = 2, 8, 2, 700, 64
    rng = np.random.default_rng(31)
    Q = rng.standard_normal((B, Hq, 1, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    V = rng.standard_normal((B, S, Hkv, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    Vd = Vd.permute(0, 2, 1, 3)
    Vh = np.ascontiguousarray(Vh.transpose(0, 2, 1, 3))
    m = rng.random((1, S)) > 0.5
    r = _per_head_flash(orc, Qh, Kh, Vh, m, None)
    md = torch.from_numpy(m.astype(np.uint8)).cuda()
    g1 = yt.scaled_dot_product_attention(Qd, Kd, Vd, 0.0, mask=md)
    _check(orc, host_f32(g1), r, dtype, f"q_len=1 strided V {dtype}")
    from ytensor_amd import _lib
    from ytensor_amd._lib import i64array
    out = torch.empty_like(g1)
    code = {"f32": _lib.F32, "f16": _lib.F16}[dtype]
    st = _lib.lib().ythip_attn_prefill(code, B, Hq, Hkv, 1, S, D, D, Qd.data_ptr(), i64array(Qd.stride()),
                                       Kd.data_ptr(), i64array(Kd.stride()), Vd.data_ptr(), i64array(Vd.stride()),
                                       out.data_ptr(), i64array(out.stride()), 0.0, _lib.MASK_BOOL, md.data_ptr(), S,
                                       None, 0, 0, torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "ythip_attn_prefill")
    _check(orc, host_f32(out), r, dtype, f"q_len=1 no workspace {dtype}")
    z = yt.scaled_dot_product_attention(Qd, Kd, Vd, 0.0, mask=torch.zeros((1, S), dtype=torch.bool).cuda())
    assert not host_f32(z).any()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_decode_ragged_lengths(orc, yt, dtype):
    """Per-sequence cache lengths (kv_len[b]); keys past the length are invisible."""
    B, Hq, Hkv, ctx, D = 4, 8, 2, 300, 128
    lens = np.array([1, 77, 300, 128], np.int32)
    rng = np.random.default_rng(9)
    Q = rng.standard_normal((B, Hq, 1, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, ctx, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, ctx, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    g = host_f32(yt.decode_attention(Qd, Kd, Vd, kv_len=torch.from_numpy(lens).cuda()))
    r = np.zeros_like(Q)
    for b in range(B):
        L = int(lens[b])
        r[b] = orc.sdpa_gqa(Qh[b:b + 1], np.ascontiguousarray(Kh[b:b + 1, :, :L]),
                            np.ascontiguousarray(Vh[b:b + 1, :, :L]), 0.0, True)[0]
    _check(orc, g.reshape(r.shape), r, dtype, f"ragged {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_decode_group_of_five_vs_oracle(orc, yt, dtype):
    """GQA group 5 (Qwen3-14B's 40 q / 8 kv heads) on the split-K decode kernel,
    ragged per-sequence lengths, against the reference's flash_attention."""
    B, Hq, Hkv, ctx, D = 2, 40, 8, 700, 128
    lens = np.array([700, 333], np.int32)
    rng = np.random.default_rng(55)
    Q = rng.standard_normal((B, Hq, 1, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, ctx, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, ctx, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, dtype)
    Kd, Kh = make_input(orc, K, dtype)
    Vd, Vh = make_input(orc, V, dtype)
    g = host_f32(yt.decode_attention(Qd, Kd, Vd, kv_len=torch.from_numpy(lens).cuda()))
    r = np.zeros_like(Q)
    for b in range(B):
        L = int(lens[b])
        r[b] = orc.sdpa_gqa(Qh[b:b + 1], np.ascontiguousarray(Kh[b:b + 1, :, :L]),
                            np.ascontiguousarray(Vh[b:b + 1, :, :L]), 0.0, True)[0]
    _check(orc, g.reshape(r.shape), r, dtype, f"decode G=5 {dtype}")


def test_decode_equals_last_prefill_row(orc, yt):
    """Decode of the last query == the last row of causal prefill (same inputs)."""
    rng = np.random.default_rng(12)
    B, Hq, Hkv, S, D = 1, 16, 8, 257, 128
    Q = rng.standard_normal((B, Hq, S, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    Qd, _ = make_input(orc, Q, "f32")
    Kd, _ = make_input(orc, K, "f32")
    Vd, _ = make_input(orc, V, "f32")
    pre = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, 0.0, mask="causal"))[:, :, -1]
    dec = host_f32(yt.decode_attention(Qd[:, :, -1:].contiguous(), Kd, Vd)).reshape(pre.shape)
    assert rel_err(dec, pre) <= 1e-5


def test_single_visible_key_and_zero_query(orc, yt):
    """Closed forms: one visible key -> O = that V row; Q = 0 -> mean of visible V rows."""
    rng = np.random.default_rng(13)
    S, D = 40, 128
    K = rng.standard_normal((1, 1, S, D)).astype(np.float32)
    V = rng.standard_normal((1, 1, S, D)).astype(np.float32)
    Q = rng.standard_normal((1, 1, S, D)).astype(np.float32)
    m = np.zeros((S, S), bool)
    m[:, 7] = True
    g = host_f32(yt.scaled_dot_product_attention(dev_f32(Q), dev_f32(K), dev_f32(V), 0.0,
                                                 mask=torch.from_numpy(m).cuda()))
    assert np.allclose(g[0, 0], np.broadcast_to(V[0, 0, 7], (S, D)), rtol=0, atol=1e-6)
    Z = np.zeros_like(Q)
    g = host_f32(yt.scaled_dot_product_attention(dev_f32(Z), dev_f32(K), dev_f32(V), 0.0, mask="causal"))
    expect = np.cumsum(V[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    assert np.allclose(g[0, 0], expect, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Hq,Hkv,d", [(16, 8, 128), (8, 8, 64), (16, 4, 128), (32, 4, 64), (40, 8, 128)])
def test_decode_attention_rope_equals_unfused(orc, yt, dtype, Hq, Hkv, d):
    """ythip_attn_decode_rope == ythip_rmsnorm_rope (S = 1, dev_state) followed
    by ythip_attn_decode (kv_len = the record's KV_LEN): the same bits in the
    output, the cache rows and (O == NULL) the split-K partials, over a run of
    positions (the owner split moves across chunk boundaries), including
    tokens past the ring's end (slot = total % rows, every row visible, RoPE
    row 0 once max_pos is passed, as the reference's KVCache does)."""
    rng = np.random.default_rng(Hq * 7 + d)
    B, max_ctx = 2, 300
    dt = TORCH_DT[dtype]
    width = (Hq + 2 * Hkv) * d
    cos, sin = orc.rope_tables(d, max_ctx, 1e6)
    cos_d, sin_d = dev_f32(cos), dev_f32(sin)
    wq = dev_f32((1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    wk = dev_f32((1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    kc = torch.zeros((B, Hkv, max_ctx, d), dtype=dt, device="cuda")
    vc = torch.zeros_like(kc)
    pre = torch.from_numpy(rng.standard_normal((B, Hkv, 100, d)).astype(np.float32)).to("cuda").to(dt)
    kc[:, :, :100] = pre
    vc[:, :, :100] = pre * 0.5
    kc2, vc2, kc3, vc3 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    ws = torch.empty(yt.ops.decode_workspace_bytes(B, Hq, max_ctx, d), dtype=torch.uint8, device="cuda")
    ws2 = torch.empty_like(ws)
    ws3 = torch.empty_like(ws)
    for pos in (100, 101, 149, 150, 151, 299, 300, 451):
        qkv = torch.from_numpy(rng.standard_normal((B, width)).astype(np.float32)).to("cuda").to(dt)
        p = yt.ops.decode_state(pos, max_ctx, max_ctx)
        o_f = torch.empty((B, Hq, d), dtype=dt, device="cuda")
        yt.ops.decode_attention_rope(qkv, Hq, Hkv, d, wq, wk, 1e-6, cos_d, sin_d, p, kc, vc, o_f, ws)
        qd = torch.empty((B, Hq, 1, d), dtype=dt, device="cuda")
        yt.rms_norm_rope(qkv.view(B, 1, width), Hq, Hkv, d, wq, wk, 1e-6, cos_d, sin_d, q_out=qd, k_out=kc2,
                         v_out=vc2, dev_state=p)
        kvl = torch.full((B,), min(pos + 1, max_ctx), dtype=torch.int32, device="cuda")
        o_u = yt.decode_attention(qd.view(B, Hq, d), kc2, vc2, kv_len=kvl, workspace=ws2)
        torch.cuda.synchronize()
        assert torch.equal(o_f, o_u), (dtype, pos)
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2), (dtype, pos)
        # partials only (O == NULL): the workspace holds the unfused kernel's partials
        yt.ops.decode_attention_rope(qkv, Hq, Hkv, d, wq, wk, 1e-6, cos_d, sin_d, p, kc3, vc3, None, ws3)
        torch.cuda.synchronize()
        nparts = B * Hq * yt.ops.decode_splits(B, Hq, max_ctx) * (d + 2) * 4
        assert torch.equal(ws3[:nparts], ws2[:nparts]), (dtype, pos)
        assert torch.equal(kc3, kc2) and torch.equal(vc3, vc2)


@pytest.mark.parametrize("dtype,out_dtype", [("bf16", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float32)])
@pytest.mark.parametrize("B,Hq,Hkv,d,max_ctx", [(1, 16, 8, 128, 1000), (3, 8, 2, 64, 300), (2, 16, 8, 128, 40)])
def test_gemv_attn_merge_equals_merge_then_gemv(yt, dtype, out_dtype, B, Hq, Hkv, d, max_ctx):
    """The o projection with the split-K merge as its prologue equals the merged
    attention output (decode_attention_rope with O) fed to gemv_fused, bit for
    bit, including positions where some splits hold no key (m = -inf), both
    reading every split and, given the decode-state record, only the splits
    the run-time partition filled."""
    rng = np.random.default_rng(B * 100 + Hq + d + max_ctx)
    dt = TORCH_DT[dtype]
    width = (Hq + 2 * Hkv) * d
    N = 320
    kc = torch.from_numpy(rng.standard_normal((B, Hkv, max_ctx, d)).astype(np.float32)).to("cuda").to(dt)
    vc = torch.from_numpy(rng.standard_normal((B, Hkv, max_ctx, d)).astype(np.float32)).to("cuda").to(dt)
    w = torch.from_numpy(rng.standard_normal((N, Hq * d)).astype(np.float32) * 0.05).to("cuda").to(dt)
    ws = torch.empty(yt.ops.decode_workspace_bytes(B, Hq, max_ctx, d), dtype=torch.uint8, device="cuda")
    splits = yt.ops.decode_splits(B, Hq, max_ctx)
    for pos in sorted({0, 1, max_ctx // 3, max_ctx - 1}):
        qkv = torch.from_numpy(rng.standard_normal((B, width)).astype(np.float32)).to("cuda").to(dt)
        p = yt.ops.decode_state(pos, max_ctx, max_ctx)
        base = torch.from_numpy(rng.standard_normal((B, N)).astype(np.float32)).to("cuda").to(out_dtype)
        attn = torch.empty((B, Hq, d), dtype=dt, device="cuda")
        k1, v1 = kc.clone(), vc.clone()
        yt.ops.decode_attention_rope(qkv, Hq, Hkv, d, None, None, 1e-6, None, None, p, k1, v1, attn, ws)
        want = base.clone()
        yt.gemv_fused(attn.view(B, Hq * d), w, want, alpha=0.5, beta=1.0)
        k2, v2 = kc.clone(), vc.clone()
        yt.ops.decode_attention_rope(qkv, Hq, Hkv, d, None, None, 1e-6, None, None, p, k2, v2, None, ws)
        got = base.clone()
        yt.gemv_attn_merge(ws, B, Hq, d, max_ctx, w, got, alpha=0.5, beta=1.0)
        got_used = base.clone()
        yt.gemv_attn_merge(ws, B, Hq, d, max_ctx, w, got_used, alpha=0.5, beta=1.0, dev_state=p)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (pos, splits)
        assert torch.equal(got_used, want), (pos, splits)
        assert torch.equal(k1, k2) and torch.equal(v1, v2)


def test_gemv_attn_merge_argument_errors(yt):
    w = torch.zeros((32, 2048), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((1, 32), dtype=torch.float32, device="cuda")
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        yt.gemv_attn_merge(ws, 1, 16, 128, 1000, w, out)  # workspace too small
    with pytest.raises(ValueError):
        yt.gemv_attn_merge(ws, 1, 8, 128, 1000, w, out)  # weight width != Hq * d


@pytest.mark.parametrize("layout", ["bshd", "padded_rows"])
@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(4, 16, 8, 2048, 128), (1, 16, 8, 2048, 128), (8, 8, 8, 1000, 64)])
def test_prefill_output_views(yt, layout, B, Hq, Hkv, S, D):
    """The 16-bit prefill kernels store O as whole 128-byte lines through LDS
    when O's base, rows and heads are 16-byte aligned with unit d stride
    ("bshd": [B, S, H, D] memory viewed as [B, H, S, D]), and with fragment
    stores otherwise ("padded_rows": rows of D + 4 elements). Shapes: the
    paired-head ping-pong kernel (B = 4: 512 paired workgroups), the key split
    inside the workgroup (B = 1: 256 query blocks), and one 128-query block per
    4-wave workgroup (no GQA pairing, 512 blocks) with D = 64 and a partial last
    block (S = 1000). Either layout
    gives the bits of the contiguous output, and padding is left untouched."""
    g = torch.Generator(device="cuda").manual_seed(31 + B + D)
    q = torch.randn(B, Hq, S, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
    ref = torch.empty(B, Hq, S, D, device="cuda", dtype=torch.bfloat16)
    yt.scaled_dot_product_attention(q, k, v, 0.0, mask="causal", out=ref)
    if layout == "bshd":
        mem = torch.full((B, S, Hq, D), 3.0, device="cuda", dtype=torch.bfloat16)
        out = mem.permute(0, 2, 1, 3)
    else:
        mem = torch.full((B, Hq, S, D + 4), 3.0, device="cuda", dtype=torch.bfloat16)
        out = mem[..., :D]
    yt.scaled_dot_product_attention(q, k, v, 0.0, mask="causal", out=out)
    torch.cuda.synchronize()
    assert torch.equal(out.contiguous().view(torch.int16), ref.view(torch.int16))
    if layout == "padded_rows":
        assert bool((mem[..., D:] == 3.0).all())


@pytest.mark.parametrize("kind", ["bias", "mask_unaligned"])
def test_prefill_per_element_mask_paired_grid(orc, yt, kind):
    """Per-element masks and biases (a bias, or byte-mask rows that are not
    16-byte aligned) on a grid large enough for paired heads (B = 4, 16 query
    heads over 8, 2048 queries: 512 paired blocks) run the unpaired 128-query
    tiles: against the oracle's flash_attention with the same mask and bias
    (src/kernel/avx2/flash_attention.inl:335-379), fully masked rows zero."""
    B, Hq, Hkv, Sq, Skv, D = 4, 16, 8, 2048, 2090, 128
    rng = np.random.default_rng(7 if kind == "bias" else 8)
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    Qd, Qh = make_input(orc, Q, "bf16")
    Kd, Kh = make_input(orc, K, "bf16")
    Vd, Vh = make_input(orc, V, "bf16")
    scale = 1.0 / math.sqrt(D)
    m = bnp = None
    mask = bias = None
    if kind == "bias":
        bnp = (rng.standard_normal((Sq, Skv)) * 0.5).astype(np.float32)
        bias = torch.from_numpy(bnp).cuda()
    else:
        m = rng.random((Sq, Skv)) > 0.3
        m[5] = False
        mask = torch.from_numpy(m).cuda()   # rows of 2090 bytes: not 16-byte aligned
    r = np.zeros((B, Hq, Sq, D), np.float32)
    for b in range(B):
        for h in range(Hq):
            kh = h // (Hq // Hkv)
            r[b, h] = orc.flash_attention(Qh[b, h], Kh[b, kh], Vh[b, kh], scale, m, bnp)
    g = host_f32(yt.scaled_dot_product_attention(Qd, Kd, Vd, scale, mask=mask, bias=bias))
    if m is not None:
        assert np.all(g[:, :, 5] == 0.0)
    check16(orc, g, r, "bf16", True, f"per-element {kind} B={B} {Hq}/{Hkv} heads {Sq}x{Skv}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("pattern", ["random", "causal_bytes", "blocks"])
@pytest.mark.parametrize("grid", ["split", "whole"])
def test_prefill_fp32_bool_mask_words(orc, yt, pattern, grid, D):
    """fp32 prefill with a byte mask whose rows are 4-byte aligned (Skv a
    multiple of 4, no bias) reads each lane's mask bytes as words and classes
    every 64-key block for each wave's rows: blocks no row sees are skipped,
    blocks every row sees take no per-score test, mixed blocks test each byte.
    Patterns: random bytes with a fully masked row, the causal mask as bytes,
    and 64-key blocks hidden or shown whole per 16-row group. Against the
    reference's fp32 flash_attention (src/kernel/avx2/flash_attention.inl:
    335-379) at rel <= 1e-4, on both grids (key split and whole blocks) and
    both head dims. Skv = 336 has 16-byte mask rows (tile classes and block
    lists from the workspace); Skv = 604 only 4-byte ones (no lists)."""
    if grid == "split":
        B, Hq, Hkv, Sq, Skv = 2, 8, 2, 201, 336
    else:
        B, Hq, Hkv, Sq, Skv = 2, 64, 16, 520, 604
    rng = np.random.default_rng(Skv + len(pattern) + D)
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, Skv, D)).astype(np.float32)
    if pattern == "random":
        m = rng.random((Sq, Skv)) > 0.35
        m[7] = False
    elif pattern == "causal_bytes":
        m = np.arange(Skv)[None, :] <= np.arange(Sq)[:, None] + (Skv - Sq)
    else:
        show = rng.random(((Sq + 15) // 16, (Skv + 63) // 64)) > 0.5
        m = np.repeat(np.repeat(show, 16, axis=0), 64, axis=1)[:Sq, :Skv].copy()
        m[:, 100:103] = True   # a few mixed blocks
    g = host_f32(yt.scaled_dot_product_attention(dev_f32(Q), dev_f32(K), dev_f32(V), 0.0,
                                                 mask=torch.from_numpy(m).cuda()))
    r = np.zeros_like(g)
    for b in range(B):
        for h in range(Hq):
            r[b, h] = orc.flash_attention(Q[b, h], K[b, h // (Hq // Hkv)], V[b, h // (Hq // Hkv)],
                                          1.0 / math.sqrt(D), m, None)
    e = rel_err(g, r)
    print(f"fp32 word mask {pattern} {grid} D={D}: rel={e:.3e}", flush=True)
    assert e <= 1e-4
    empty = ~m.any(axis=1)
    assert np.all(g[:, :, empty] == 0.0)
