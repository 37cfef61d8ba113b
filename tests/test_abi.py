"""CPU checks of the C-ABI boundary: libythip.so loads (no GPU needed to dlopen
it) and exports every function include/ythip.h declares; argument errors are
reported without touching the GPU."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ythip.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ythip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    for n in ("ythip_gemm", "ythip_attn_prefill", "ythip_attn_decode", "ythip_rmsnorm_rope", "ythip_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from ytensor_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libythip.so is not built (python -m ytensor_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(_declared()) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_abi_version_and_argument_errors():
    import ytensor_amd
    lib = ytensor_amd.load()
    assert lib.ythip_abi_version() == 3
    # invalid dtype / negative sizes are rejected before any HIP call
    st = lib.ythip_gemm(7, 0, 1, 2, 2, 2, None, 0, 2, 1, None, 0, 2, 1, None, 0, 2, 1, 1.0, 0.0, None)
    assert st == -1 and b"dtype" in lib.ythip_last_error()
    st = lib.ythip_gemm(0, 0, 1, -2, 2, 2, None, 0, 2, 1, None, 0, 2, 1, None, 0, 2, 1, 1.0, 0.0, None)
    assert st == -1
    # m == 0: a no-op that succeeds (src/kernel/avx2/sgemm.inl:594)
    assert lib.ythip_gemm(0, 0, 1, 0, 2, 2, None, 0, 2, 1, None, 0, 2, 1, None, 0, 2, 1, 1.0, 0.0, None) == 0
    st = lib.ythip_rmsnorm_rope(2, 1, 1, 1, 1, 96, None, 0, None, None, 1e-6, None, None, 0, 0, 0,
                                None, None, None, None, None, None, 0, 0, None, None)
    assert st == -2  # head dim 96 unsupported


def test_decode_noalloc_rejects_oversize_without_a_launch():
    """ythip_attn_decode_noalloc refuses a shape whose split-K partials exceed
    its fixed per-GPU array before touching the GPU (the pointers are never
    dereferenced). B=128, Hq=64, d=128 needs 128*64*1*(128+2)*4 bytes > 4 MiB."""
    import ytensor_amd
    from ytensor_amd import _lib
    lib = ytensor_amd.load()
    cap = int(lib.ythip_attn_decode_noalloc_max_bytes())
    assert cap == 4 << 20
    need = int(lib.ythip_attn_decode_workspace_size(128, 64, 16, 128))
    assert need == 128 * 64 * 130 * 4 > cap
    fake = ctypes.c_void_p(256)
    st = lib.ythip_attn_decode_noalloc(_lib.BF16, 128, 64, 8, 128, 16, fake, _lib.i64array([64 * 128, 128]),
                                       fake, fake, _lib.i64array([8 * 16 * 128, 16 * 128, 128]), None,
                                       fake, _lib.i64array([64 * 128, 128]), 0.0, None)
    assert st == _lib.YTHIP_EINVAL
    assert b"fixed array" in lib.ythip_last_error()


def test_cpp_mirror_compiles_and_reports_errors(tmp_path):
    """The C++ host's kernel-level API (yt::kernel::hip in include/yt/ytensor.hpp)
    builds with the host C++ compiler against libythip.so and maps argument
    errors to exceptions."""
    import shutil
    import subprocess
    from ytensor_amd import _lib
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "abi_errors"
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    subprocess.check_call([gxx, "-std=c++20", "-O1", f"-I{os.path.join(ROOT, 'include')}", "-I/opt/rocm/include",
                           "-D__HIP_PLATFORM_AMD__", os.path.join(ROOT, "tests", "cpp", "abi_errors.cpp"),
                           "-o", str(exe), f"-L{lib_dir}", "-lythip", f"-Wl,-rpath,{lib_dir}", "-L/opt/rocm/lib",
                           "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"])
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "ok:" in out.stdout


def test_prefill_workspace_size_and_short_workspace():
    """ythip_attn_prefill_workspace_size: one byte per 32-row x 64-key tile of
    the bool mask, in 256-byte units; a bool-mask call given fewer bytes is an
    argument error before any launch (the pointers are never dereferenced)."""
    import ytensor_amd
    from ytensor_amd import _lib
    lib = ytensor_amd.load()
    assert lib.ythip_attn_prefill_workspace_size(8192, 8192) == 256 * 128
    assert lib.ythip_attn_prefill_workspace_size(33, 65) == 256
    assert lib.ythip_attn_prefill_workspace_size(2000, 2096) == 63 * 33 // 256 * 256 + 256
    assert lib.ythip_attn_prefill_workspace_size(0, 64) == 0
    assert lib.ythip_attn_prefill_workspace_size(64, 0) == 0
    fake = ctypes.c_void_p(256)
    st4 = _lib.i64array([16 * 64 * 128, 64 * 128, 128, 1])
    st = lib.ythip_attn_prefill_ws(_lib.BF16, 1, 16, 8, 64, 64, 128, 128, fake, st4, fake,
                                   _lib.i64array([8 * 64 * 128, 64 * 128, 128, 1]), fake,
                                   _lib.i64array([8 * 64 * 128, 64 * 128, 128, 1]), fake, st4, 0.0,
                                   _lib.MASK_BOOL, fake, 64, None, 0, 0, fake, 255, None)
    assert st == _lib.YTHIP_EINVAL
    assert b"workspace of 256 bytes" in lib.ythip_last_error()


def test_probe_library_loads_and_rejects_bad_shapes():
    """The roofline probe library (libythip_probe.so, measurement support for
    bench.py) loads and refuses shapes it does not take before any launch
    (the pointers are never dereferenced)."""
    from ytensor_amd import probe
    if not os.path.exists(probe.PROBE_LIB_PATH):
        pytest.fail("libythip_probe.so is not built (python -m ytensor_amd.build)")
    lib = probe.load()
    fake = 256
    assert lib.ythip_probe_dma(fake, fake, 300, 256, 128, fake, None) == -1  # M not a multiple of 256
    assert lib.ythip_probe_dma(fake, fake, 256, 256, 64, fake, None) == -1   # fewer than two k steps
    assert lib.ythip_probe_mfma(fake, fake, fake, 0, 1, None) == -1
    assert lib.ythip_probe_mfma(fake, fake, fake, 1, 0, None) == -1
