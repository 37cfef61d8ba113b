"""Build libythip.so (gfx950) in-tree with hipcc.

    python -m ytensor_amd.build            # compile + link
    python -m ytensor_amd.build --resource # also print per-kernel VGPR/LDS/spill usage

Every translation unit under csrc/*.hip is compiled for gfx950 only, with the
packed-fp32 feature disabled (v_pk_*_f32 are never emitted), then linked into
ytensor_amd/libythip.so next to this file. The roofline probes under
csrc/probe/ (measurement support for bench.py, not part of the C ABI) are
linked into ytensor_amd/libythip_probe.so the same way.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libythip.so")
PROBE_LIB = os.path.join(HERE, "libythip_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _compile(src: str, resource: bool) -> tuple[str, str]:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    if resource:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{p.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; drop that note.
    err = "\n".join(l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l)
    return obj, err


ROOT = os.path.dirname(HERE)
BIN = os.path.join(HERE, "bin")
HOST_PROGRAMS = {"yt_host_parity": os.path.join(ROOT, "tests", "cpp", "host_parity.cpp"),
                 "yt_qwen3": os.path.join(ROOT, "tests", "cpp", "qwen3_host.cpp")}


def _build_host(name: str, src: str) -> str:
    exe = os.path.join(BIN, name)
    # -ffp-contract=off: host float expressions (the weight recipe's 1 + x * s)
    # round each operation, as the numpy restatement does
    cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-ffp-contract=off", f"-I{os.path.join(ROOT, 'include')}",
           "-I/opt/rocm/include",
           "-D__HIP_PLATFORM_AMD__", src, "-o", exe + ".tmp", f"-L{HERE}", "-lythip", "-L/opt/rocm/lib",
           "-lamdhip64", "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath,/opt/rocm/lib"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"g++ failed for {src}:\n{p.stderr}")
    os.replace(exe + ".tmp", exe)
    return exe


def build_host_programs() -> list[str]:
    """C++ programs over the host API (include/yt/ytensor.hpp, include/yt/qwen3.hpp)
    linked against libythip.so, built with the host compiler into ytensor_amd/bin/."""
    os.makedirs(BIN, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(HOST_PROGRAMS)) as ex:
        return list(ex.map(lambda kv: _build_host(*kv), HOST_PROGRAMS.items()))


def build(resource: bool = False, verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    probe_srcs = sorted(glob.glob(os.path.join(CSRC, "probe", "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + len(probe_srcs))) as ex:
        results = list(ex.map(lambda s: _compile(s, resource), srcs + probe_srcs))
    for _, err in results:
        if err.strip() and (verbose or resource):
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    for lib, lib_objs, extra in ((LIB, objs[:len(srcs)], ["-lz"]), (PROBE_LIB, objs[len(srcs):], [])):
        tmp = lib + ".tmp"
        subprocess.check_call([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *lib_objs, *extra])
        os.replace(tmp, lib)
    build_host_programs()
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--resource", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(resource=args.resource, verbose=args.verbose))


if __name__ == "__main__":
    main()
