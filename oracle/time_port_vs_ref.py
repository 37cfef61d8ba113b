"""Time the oracle restatement against the compiled reference on the same
inputs -- TEST INFRASTRUCTURE. Runs only where oracle/_ref/libytref.so was
built (this needs /root/reference); the GPU box times the restatement alone
(bench.py's cpu_baseline, kind "port") and reports beside it the ratio this
script measured, read from profiles/cpu_port_vs_reference.md.

    python oracle/time_port_vs_ref.py   # writes profiles/cpu_port_vs_reference.md

Workloads (single thread for the GEMM, the reference default g_num_threads = 0;
the attention and normalisation loops with their OpenMP defaults), one per
bench.py cpu_baseline row:
  sgemm 4096^3 fp32 on bf16-rounded inputs   (the bench headline's CPU leg)
  causal GQA prefill S=2048, 16 q / 8 kv heads, D=128
  decode B=16, ctx=8192
  rmsNorm_ + rope S=8192, 24 heads
  scaledDotProductAttention(MATH), causal predicate, 16 heads, S=2048
  masked_matmul 2048^3, causal predicate
  YTensorIO::load of a 256 MiB bf16 tensor
The ratio is port time / reference time (median of the runs): > 1 means the
restatement is slower than the reference on the same host. Each row's ratio is
also written as a line `ratio <bench row>: <value>` for bench.py.
"""
from __future__ import annotations

import datetime
import math
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

OUT = os.path.join(ROOT, "profiles", "cpu_port_vs_reference.md")


def med(fn, n):
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def main() -> None:
    port, ref = oracle.oracle(), oracle.reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libytref.so is not built (make -C oracle ref)")
    rng = np.random.default_rng(0)

    def bf(*shape, scale=1.0):
        x = rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)
        return port.bf16_to_f32(port.bf16_round(x))

    rows = []
    A, B = bf(4096, 4096), bf(4096, 4096, scale=0.02)
    for p in (port, ref):
        p.set_num_threads(1)
    tp = med(lambda: port.sgemm(A, B), 3)
    tr = med(lambda: ref.sgemm(A, B), 3)
    rows.append(("sgemm 4096^3 fp32, 1 thread", tp, tr))
    del A, B
    omp = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    S = 2048
    q, k, v = bf(1, 16, S, 128), bf(1, 8, S, 128), bf(1, 8, S, 128)
    tp = med(lambda: port.sdpa_gqa(q, k, v, 1 / math.sqrt(128), True), 3)
    tr = med(lambda: ref.sdpa_gqa(q, k, v, 1 / math.sqrt(128), True), 3)
    rows.append((f"causal GQA prefill S=2048 (OpenMP {omp} threads)", tp, tr))
    ctx = 8192
    q, k, v = bf(16, 16, 1, 128), bf(16, 8, ctx, 128), bf(16, 8, ctx, 128)
    tp = med(lambda: port.sdpa_gqa(q, k, v, 1 / math.sqrt(128), False), 3)
    tr = med(lambda: ref.sdpa_gqa(q, k, v, 1 / math.sqrt(128), False), 3)
    rows.append((f"decode B=16 ctx=8192 (OpenMP {omp} threads)", tp, tr))
    del q, k, v
    S = 8192
    qk = bf(1, 24, S, 128)
    w = bf(128, scale=0.02)
    cp, sp = port.rope_tables(128, S, 1e6)
    cr, sr = ref.rope_tables(128, S, 1e6)
    tp = med(lambda: port.rope(port.rms_norm(qk, w, 1e-6), cp, sp), 3)
    tr = med(lambda: ref.rope(ref.rms_norm(qk, w, 1e-6), cr, sr), 3)
    rows.append(("rmsNorm_ + rope S=8192, 24 heads", tp, tr))
    del qk
    S = 2048
    q, k = bf(16, S, 128), bf(16, S, 128)
    tp = med(lambda: port.sdpa_math(q, k, k, 0.0, diag=0), 2)
    tr = med(lambda: ref.sdpa_math(q, k, k, 0.0, diag=0), 2)
    rows.append((f"scaledDotProductAttention(MATH) causal S=2048, 16 heads (OpenMP {omp} threads)", tp, tr))
    del q, k
    a = bf(2048, 2048)
    tp = med(lambda: port.masked_matmul(a, a, diag=0, value=-1e9), 2)
    tr = med(lambda: ref.masked_matmul(a, a, diag=0, value=-1e9), 2)
    rows.append(("masked_matmul 2048^3, causal predicate", tp, tr))
    del a
    import shutil
    import tempfile
    from oracle import ytio
    tmp = tempfile.mkdtemp(prefix="ythip_ratio_")
    try:
        pth = os.path.join(tmp, "w.yt")
        wv = np.arange(128 << 20, dtype=np.uint16)
        ytio.write(pth, {"w": wv}, types={"w": "bfloat16"})
        ytio.read(pth)
        tp = med(lambda: ytio.read(pth), 3)
        tr = med(lambda: ref.yt_load(pth, "w", cap=wv.nbytes), 3)
        rows.append(("YTensorIO::load 256 MiB bf16 (page cache)", tp, tr))
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    keys = ["gemm_4096_fp32_1thread", "attn_prefill_causal_S2048", "attn_decode_B16_ctx8192", "rmsnorm_rope_S8192",
            "attn_math_S2048", "masked_matmul_2048_causal", "yt_load_256MiB_bf16"]
    head = rows[0]
    with open(OUT, "w") as f:
        f.write("# CPU baseline: the oracle restatement (\"port\") against the compiled reference\n\n")
        f.write("Command: `python oracle/time_port_vs_ref.py` (this container; the GPU box times only the port).\n\n")
        f.write(f"Host: {platform.processor() or platform.machine()}, {os.cpu_count()} logical CPUs, "
                f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}; "
                f"{datetime.date.today().isoformat()}.\n\n")
        f.write("| workload | port s | reference s | port / reference |\n|---|---|---|---|\n")
        for name, tp, tr in rows:
            f.write(f"| {name} | {tp:.4f} | {tr:.4f} | {tp / tr:.3f} |\n")
        f.write(f"\nport_over_reference_time: {head[1] / head[2]:.4f}\n\n")
        f.write("Per bench.py cpu_baseline row (port time / reference time):\n\n")
        for key, (_, tp, tr) in zip(keys, rows):
            f.write(f"    ratio {key}: {tp / tr:.4f}\n")
    print(open(OUT).read())


if __name__ == "__main__":
    main()
