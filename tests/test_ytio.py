""".yt files on the CPU: the oracle's format restatement against the
reference-written fixtures, and the product's host side (libythip's
ythip_yt_* parser and writer, the yt::io mirror in ytensor_amd.io) on them.
Nothing here touches a GPU: parsing and the rewrite of stored payloads are
host-only; device loads and saves are in test_gpu_ytio.py.

Pins: tests/golden/yt_*.yt were written by the reference's own
yt::io::YTensorIO (src/ytensor_io.inl) and yt_expected.npz holds what its
load() returned (tests/golden/make_yt_fixtures.py)."""
from __future__ import annotations

import ctypes
import os
import shutil
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
sys.path.insert(0, GOLD)

import make_yt_fixtures as fx  # noqa: E402
from oracle import ytio  # noqa: E402


def _exp():
    return np.load(os.path.join(GOLD, "yt_expected.npz"))


def _payload(a) -> bytes:
    return np.ascontiguousarray(a).tobytes()


def _items(ts):
    return [(n, t, s, _payload(a)) for n, t, s, a in ts]


# ------------------------------------------------------------------ oracle pins
@pytest.mark.parametrize("fname,comp", [("yt_plain.yt", ""), ("yt_zlib.yt", "zlib")])
def test_oracle_encode_is_byte_identical_to_reference(fname, comp):
    """The restatement writes the reference's bytes (uncompressed and zlib)."""
    want = open(os.path.join(GOLD, fname), "rb").read()
    assert ytio.encode(_items(fx.tensors()), comp) == want


def test_oracle_encode_append_and_rewrite_semantics():
    """Append keeps the old tensors, replaces "c" in place and numbers the
    unnamed one after them; Write drops what was not saved again
    (src/ytensor_io.inl:256-290, 339-344, 712-724)."""
    base = fx.base_set()
    app, rew = fx.update_sets()
    e = _exp()
    appended = [app[0] if n == "c" else (n, t, s, a) for n, t, s, a in base] + [app[1], ("4",) + app[2][1:]]
    assert [x[0] for x in appended] == list(e["names_append"])
    assert ytio.encode(_items(appended)) == open(os.path.join(GOLD, "yt_append.yt"), "rb").read()
    rewritten = [rew[2], rew[0], ("3",) + rew[1][1:]]
    assert [x[0] for x in rewritten] == list(e["names_rewrite"])
    assert ytio.encode(_items(rewritten)) == open(os.path.join(GOLD, "yt_rewrite.yt"), "rb").read()


@pytest.mark.parametrize("fname", ["yt_plain.yt", "yt_zlib.yt"])
def test_oracle_read_matches_reference_load(fname):
    meta, recs = ytio.read(os.path.join(GOLD, fname))
    e = _exp()
    assert meta == ""
    assert [r["name"] for r in recs] == [t[0] for t in fx.tensors()]
    for r in recs:
        n = r["name"]
        assert r["typeName"] == str(e[f"{n}|type"])
        assert r["shape"] == list(e[f"{n}|shape"])
        assert r["data"].tobytes() == e[f"{n}|bytes"].tobytes()


def test_reference_fixture_regenerates(ref, tmp_path):
    """The fixtures are what the reference writes today (only where it is built)."""
    p = str(tmp_path / "x.yt")
    ref.yt_save(p, fx.tensors(), "zlib")
    assert open(p, "rb").read() == open(os.path.join(GOLD, "yt_zlib.yt"), "rb").read()


# ------------------------------------------------------------------ product host side
@pytest.fixture(scope="module")
def L():
    from ytensor_amd import _lib
    return _lib


def _open(L, path):
    h = ctypes.c_void_p()
    st = L.lib().ythip_yt_open(path.encode(), ctypes.byref(h))
    return st, h


@pytest.mark.parametrize("fname", ["yt_plain.yt", "yt_zlib.yt", "yt_append.yt", "yt_rewrite.yt"])
def test_product_parser_matches_oracle(L, fname):
    path = os.path.join(GOLD, fname)
    st, h = _open(L, path)
    assert st == 0, L.lib().ythip_last_error()
    lib = L.lib()
    try:
        meta, recs = ytio.read(path)
        assert lib.ythip_yt_metadata(h) == meta.encode()
        assert lib.ythip_yt_count(h) == len(recs)
        for i, r in enumerate(recs):
            info = L.YtTensorInfo()
            assert lib.ythip_yt_info(h, i, ctypes.byref(info)) == 0
            assert info.name.decode() == r["name"]
            assert info.dtype.decode() == r["typeName"]
            assert info.type_size == r["typeSize"]
            assert info.tensor_type.decode() == "dense"
            assert info.compress.decode() == r["compress"]
            assert [info.shape[d] for d in range(info.ndim)] == r["shape"]
            assert info.compressed_size == len(r["payload"])
            assert info.nbytes == r["typeSize"] * int(np.prod(r["shape"], dtype=np.int64))
            blob = open(path, "rb").read()
            assert blob[info.data_offset:info.data_offset + info.compressed_size] == r["payload"]
            assert lib.ythip_yt_find(h, r["name"].encode()) == i
        assert lib.ythip_yt_find(h, b"") == 0  # getTensorInfo("") = the first tensor
        assert lib.ythip_yt_find(h, b"no such tensor") == L.YTHIP_ENOTFOUND
    finally:
        lib.ythip_yt_close(h)


def test_product_parser_rejects_bad_files(L, tmp_path):
    lib = L.lib()
    st, _ = _open(L, str(tmp_path / "missing.yt"))
    assert st == L.YTHIP_EIO
    junk = tmp_path / "junk.yt"
    junk.write_bytes(b"NOTATENSORFILE" * 4)
    assert _open(L, str(junk))[0] == L.YTHIP_EFORMAT
    good = open(os.path.join(GOLD, "yt_plain.yt"), "rb").read()
    for cut in (5, 20, len(good) // 2, len(good) - 3):
        t = tmp_path / f"cut{cut}.yt"
        t.write_bytes(good[:cut])
        st, h = _open(L, str(t))
        assert st == L.YTHIP_EFORMAT, (cut, st)
    # an index entry pointing past the data area
    bad = bytearray(good)
    bad[-12:-4] = (len(good) + 100).to_bytes(8, "little")
    t = tmp_path / "badoff.yt"
    t.write_bytes(bytes(bad))
    assert _open(L, str(t))[0] == L.YTHIP_EFORMAT
    # a record whose payload size runs past the data area
    st, h = _open(L, os.path.join(GOLD, "yt_base.yt"))
    info = L.YtTensorInfo()
    lib.ythip_yt_info(h, 0, ctypes.byref(info))
    off = info.data_offset
    lib.ythip_yt_close(h)
    base = bytearray(open(os.path.join(GOLD, "yt_base.yt"), "rb").read())
    base[off - 8:off] = (10 ** 6).to_bytes(8, "little")
    t = tmp_path / "badsize.yt"
    t.write_bytes(bytes(base))
    assert _open(L, str(t))[0] == L.YTHIP_EFORMAT


def test_product_load_argument_errors(L):
    """Checked before anything is queued (no device needed)."""
    lib = L.lib()
    st, h = _open(L, os.path.join(GOLD, "yt_plain.yt"))
    try:
        assert lib.ythip_yt_load(h, 99, None, L.F32, 0, None) == L.YTHIP_EINVAL
        i = lib.ythip_yt_find(h, b"big_f32")
        assert lib.ythip_yt_load(h, i, ctypes.c_void_p(16), L.F32, 100, None) == L.YTHIP_EINVAL  # too small
        i = lib.ythip_yt_find(h, b"bytes_u8")
        assert lib.ythip_yt_load(h, i, ctypes.c_void_p(16), L.BF16, 1 << 20, None) == L.YTHIP_EUNSUPPORTED
        assert lib.ythip_yt_load(h, i, ctypes.c_void_p(16), 7, 1 << 20, None) == L.YTHIP_EINVAL
    finally:
        lib.ythip_yt_close(h)


@pytest.mark.parametrize("fname", ["yt_append.yt", "yt_plain.yt", "yt_zlib.yt"])
def test_product_append_without_new_tensors_rewrites_identically(L, tmp_path, fname):
    """Append with nothing new: the reference's close() writes the same bytes back."""
    p = tmp_path / fname
    shutil.copy(os.path.join(GOLD, fname), p)
    st = L.lib().ythip_yt_save(str(p).encode(), 0, None, b"", 1, None)
    assert st == 0, L.lib().ythip_last_error()
    assert p.read_bytes() == open(os.path.join(GOLD, fname), "rb").read()


def test_product_write_without_tensors_drops_everything(L, tmp_path):
    p = tmp_path / "w.yt"
    shutil.copy(os.path.join(GOLD, "yt_base.yt"), p)
    assert L.lib().ythip_yt_save(str(p).encode(), 0, None, b"zlib", 0, None) == 0
    assert p.read_bytes() == ytio.encode([])


def test_io_mirror_read_side(tmp_path):
    from ytensor_amd import io
    f = io.YTensorIO()
    assert not f.open(str(tmp_path / "none.yt"), io.Read)
    assert f.open(os.path.join(GOLD, "yt_append.yt"), io.Read)
    assert f.validateFile()
    assert f.getTensorNames() == list(_exp()["names_append"])
    i = f.getTensorInfo("d")
    assert (i.typeName, i.typeSize, i.shape, i.tensorType, i.compressMethod) == ("float16", 2, [5], "dense", "")
    assert f.getTensorInfo("").name == "a"
    with pytest.raises(RuntimeError, match="Tensor not found"):
        f.getTensorInfo("zz")
    assert f.load("zz") is None
    f.close()
    assert not f.validateFile()
