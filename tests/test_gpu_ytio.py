"""GPU: .yt checkpoints loaded into device memory and saved from it through
libythip (ythip_yt_load / ythip_yt_save, via the yt::io mirror ytensor_amd.io).

Pins:
* every tensor of the reference-written fixtures lands on the device with the
  bytes the reference's YTensorIO::load returned (tests/golden/yt_expected.npz);
* conversions on the way equal the reference's casts: 16 -> 32 bit through the
  reference's own tables of all 65536 bf16 / fp16 patterns
  (reference_small.npz kat_bf16_to_f32 / kat_f16_to_f32), 32 -> 16 bit through
  the oracle's yt::bfloat16 / yt::float16 rounding (pinned to the reference's
  by test_oracle.py), float64 / int32 -> float as C's static_cast (numpy astype);
* files saved from the device are byte-identical to the reference's
  (yt_plain.yt, yt_zlib.yt, yt_append.yt, yt_rewrite.yt);
* multi-chunk tensors (beyond the 16 MiB staging buffers, raw and zlib) and
  a Qwen3 checkpoint with the example's tensor names give the same model as
  the flat-weight upload.
"""
from __future__ import annotations

import os
import shutil
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
sys.path.insert(0, GOLD)

import make_yt_fixtures as fx  # noqa: E402
from oracle import ytio  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def yio():
    from ytensor_amd import io
    return io


@pytest.fixture(scope="module")
def kat():
    return np.load(os.path.join(GOLD, "reference_small.npz"))


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.reshape(-1).cpu().view(torch.int16).numpy().view(np.uint16)


def _expected_as(orc, kat, tname: str, raw: bytes, want: str) -> np.ndarray:
    """Reference cast of the stored values to want ("f32" | "bf16" | "f16"); 16-bit results as bits."""
    if tname == "bfloat16":
        f = kat["kat_bf16_to_f32"][np.frombuffer(raw, np.uint16)]
        if want == "bf16":
            return np.frombuffer(raw, np.uint16)
    elif tname == "float16":
        f = kat["kat_f16_to_f32"][np.frombuffer(raw, np.uint16)]
        if want == "f16":
            return np.frombuffer(raw, np.uint16)
    elif tname == "float32":
        f = np.frombuffer(raw, np.float32)
    elif tname == "float64":
        f = np.frombuffer(raw, np.float64).astype(np.float32)
    elif tname == "int32":
        f = np.frombuffer(raw, np.int32).astype(np.float32)
    else:
        raise AssertionError(tname)
    if want == "f32":
        return f
    return orc.bf16_round(f) if want == "bf16" else orc.f16_round(f)


@pytest.mark.parametrize("fname", ["yt_plain.yt", "yt_zlib.yt"])
def test_load_raw_matches_reference(yio, fname):
    e = np.load(os.path.join(GOLD, "yt_expected.npz"))
    f = yio.YTensorIO()
    assert f.open(os.path.join(GOLD, fname))
    for name, _, _, _ in fx.tensors():
        t = f.load(name)
        assert t is not None and t.is_cuda, name
        assert list(t.shape) == list(e[f"{name}|shape"]), name
        got = t.contiguous().reshape(-1).cpu().view(torch.uint8).numpy().tobytes() if t.numel() else b""
        assert got == e[f"{name}|bytes"].tobytes(), name
    f.close()


@pytest.mark.parametrize("fname", ["yt_plain.yt", "yt_zlib.yt"])
@pytest.mark.parametrize("want", ["f32", "bf16", "f16"])
def test_load_converts_with_reference_casts(yio, orc, kat, fname, want):
    e = np.load(os.path.join(GOLD, "yt_expected.npz"))
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[want]
    f = yio.YTensorIO()
    assert f.open(os.path.join(GOLD, fname))
    for name, tname, _, _ in fx.tensors():
        if tname not in ("bfloat16", "float16", "float32", "float64", "int32"):
            assert f.load(name, dt) is None  # no float conversion of uint8
            continue
        t = f.load(name, dt)
        ref = _expected_as(orc, kat, tname, e[f"{name}|bytes"].tobytes(), want)
        got = t.cpu().numpy().reshape(-1) if want == "f32" else _u16(t).reshape(-1)
        if want == "f32":
            assert got.view(np.uint32).tolist() == np.asarray(ref, np.float32).view(np.uint32).tolist(), name
        else:
            assert got.tolist() == np.asarray(ref).tolist(), name
    f.close()


def _dev_tensor(tname: str, a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if tname == "bfloat16":
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
    if tname == "float16":
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.float16).cuda()
    return torch.from_numpy(a.copy()).cuda()


@pytest.mark.parametrize("fname,comp", [("yt_plain.yt", ""), ("yt_zlib.yt", "zlib")])
def test_save_from_device_is_byte_identical(yio, tmp_path, fname, comp, monkeypatch):
    monkeypatch.setattr(yio, "compressMethod", comp)
    p = str(tmp_path / "out.yt")
    f = yio.YTensorIO()
    assert f.open(p, yio.Write)
    for name, tname, shape, a in fx.tensors():
        assert f.save(_dev_tensor(tname, a).reshape(shape), name)
    assert f.close()
    assert open(p, "rb").read() == open(os.path.join(GOLD, fname), "rb").read()


@pytest.mark.parametrize("mode,fname", [("append", "yt_append.yt"), ("rewrite", "yt_rewrite.yt")])
def test_save_over_existing_file_matches_reference(yio, tmp_path, mode, fname):
    p = str(tmp_path / "f.yt")
    shutil.copy(os.path.join(GOLD, "yt_base.yt"), p)
    app, rew = fx.update_sets()
    f = yio.YTensorIO()
    assert f.open(p, yio.Append if mode == "append" else yio.Write)
    for name, tname, shape, a in (app if mode == "append" else rew):
        assert f.save(_dev_tensor(tname, a).reshape(shape), name)
    names = f.getTensorNames()
    assert f.close()
    exp = np.load(os.path.join(GOLD, "yt_expected.npz"))["names_" + mode]
    if mode == "append":
        assert names == list(exp)
    assert open(p, "rb").read() == open(os.path.join(GOLD, fname), "rb").read()


@pytest.mark.parametrize("comp", ["", "zlib"])
def test_multichunk_tensors(yio, orc, tmp_path, comp):
    """Tensors of several 16 MiB staging chunks (odd sizes so the last chunk is
    partial): bf16 copied as is, fp32 narrowed to bf16 on the way, bf16 widened."""
    rng = np.random.default_rng(5)
    big_bf = orc.bf16_round(rng.standard_normal(3000 * 4096 + 77).astype(np.float32))
    big_f32 = rng.standard_normal(1500 * 4096 + 5).astype(np.float32)
    p = str(tmp_path / "big.yt")
    ytio.write(p, {"w": big_bf, "x": big_f32}, comp, types={"w": "bfloat16"})
    f = yio.YTensorIO()
    assert f.open(p)
    w = f.load("w")
    assert w.dtype == torch.bfloat16 and np.array_equal(_u16(w), big_bf)
    xb = f.load("x", torch.bfloat16)
    assert np.array_equal(_u16(xb), orc.bf16_round(big_f32))
    wf = f.load("w", torch.float32)
    assert np.array_equal(wf.cpu().numpy(), orc.bf16_to_f32(big_bf))
    # back-to-back loads into views of one buffer, one wait at the end
    buf = torch.empty(2 * big_bf.size, dtype=torch.bfloat16, device="cuda")
    f.load_many([("w", buf[:big_bf.size]), ("w", buf[big_bf.size:])])
    assert np.array_equal(_u16(buf[big_bf.size:]), big_bf)
    f.close()
    # round trip through the device writer
    q = str(tmp_path / "again.yt")
    yio.compressMethod = comp
    try:
        assert yio.saveTensorBase(q, w, "w")
    finally:
        yio.compressMethod = ""
    _, recs = ytio.read(q)
    assert recs[0]["name"] == "w" and np.array_equal(recs[0]["data"], big_bf)


def test_corrupt_zlib_payload_is_rejected(yio, tmp_path):
    b = bytearray(open(os.path.join(GOLD, "yt_zlib.yt"), "rb").read())
    _, recs = ytio.read(os.path.join(GOLD, "yt_zlib.yt"))
    i = b.index(recs[-2]["payload"])  # big_f32's stream
    b[i + 40:i + 60] = bytes(20)
    p = tmp_path / "bad.yt"
    p.write_bytes(bytes(b))
    f = yio.YTensorIO()
    assert f.open(str(p))
    assert f.load("big_f32") is None
    assert f.load("ids") is not None  # the other records stay readable
    f.close()


def test_qwen3_from_yt_equals_flat_upload(tmp_path):
    """A checkpoint with the example's names (Qwen3Model::load) builds the same
    device model as the flat upload: identical logits and greedy tokens; an
    lm_head.weight in the file replaces the tied head."""
    from ytensor_amd.qwen3 import Qwen3, Qwen3Config, hf_names, weight_layout
    import oracle
    cfg = Qwen3Config(hidden=256, layers=2, vocab=1000, inter=512, n_heads=4, n_kv=2, head_dim=64, max_pos=256)
    flat = oracle.qwen3_random_weights(oracle.oracle(), cfg, seed=9)
    orc = oracle.oracle()
    off, parts = 0, {}
    for name, shp in weight_layout(cfg):
        n = int(np.prod(shp))
        parts[name] = flat[off:off + n].reshape(shp)
        off += n
    arrays, types = {}, {}

    def put(key, a, bf16):
        arrays[key] = orc.bf16_round(a) if bf16 else a.astype(np.float32)
        if bf16:
            types[key] = "bfloat16"
    top = hf_names(cfg)
    put(top["embed"], parts["embed"], True)
    for i in range(cfg.layers):
        n = hf_names(cfg, i)
        for k in ("q", "k", "v", "o", "gate", "up", "down"):
            put(n[k], parts[f"{i}.{k}"], True)
        for k in ("q_norm", "k_norm", "norm1", "norm2"):
            put(n[k], parts[f"{i}.{k}"], False)
    put(top["norm"], parts["norm"], False)
    d = tmp_path / "model"
    d.mkdir()
    ytio.write(str(d / "model.yt"), arrays, types=types)
    (d / "config.json").write_text('{"hidden_size": 256, "num_hidden_layers": 2, "vocab_size": 1000, '
                                   '"intermediate_size": 512, "num_attention_heads": 4, "num_key_value_heads": 2, '
                                   '"head_dim": 64, "max_position_embeddings": 256, "rms_norm_eps": 1e-06, '
                                   '"rope_theta": 1000000.0}')
    prompt = (np.arange(17) * 37 % cfg.vocab).astype(np.int32)
    a = Qwen3(cfg, flat, max_ctx=128, max_prompt=32)
    b = Qwen3.from_yt(str(d), max_ctx=128, max_prompt=32)
    assert vars(b.cfg) == vars(cfg)
    ta = a.generate(prompt, 12)
    la = a.logits.clone()
    tb = b.generate(prompt, 12)
    assert np.array_equal(ta, tb)
    assert torch.equal(la, b.logits)
    # the same weights stored as float32 (narrowed to bf16 on the way, exactly: they are bf16 values)
    arrays32 = {k: (orc.bf16_to_f32(v) if k in types else v) for k, v in arrays.items()}
    d32 = tmp_path / "model32.yt"
    ytio.write(str(d32), arrays32)
    b32 = Qwen3.from_yt(str(d32), cfg, max_ctx=128, max_prompt=32)
    assert all(torch.equal(b32.layers[i][k], b.layers[i][k]) for i in range(cfg.layers) for k in b.layers[i])
    assert torch.equal(b32.embed, b.embed)
    # an explicit LM head (here: the embedding reversed) is used instead of the tied one
    arrays[top["lm_head"]] = arrays[top["embed"]][::-1].copy()
    types[top["lm_head"]] = "bfloat16"
    ytio.write(str(d / "model.yt"), arrays, types=types)
    c = Qwen3.from_yt(str(d), max_ctx=128, max_prompt=32)
    assert c.lm_head.data_ptr() != c.embed.data_ptr()
    assert torch.equal(c.lm_head, torch.flip(b.embed, [0]))
    # a checkpoint missing a tensor is refused
    del arrays[hf_names(cfg, 1)["down"]]
    ytio.write(str(d / "model.yt"), arrays, types=types)
    with pytest.raises(KeyError):
        Qwen3.from_yt(str(d), max_ctx=128, max_prompt=32)
