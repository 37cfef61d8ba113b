#!/usr/bin/env python3
"""Benchmark of the MI355X hot path (libythip.so) on one GPU.

Headline (`value`): bf16 GEMM C[M,N] = A[M,K] . B[K,N] at M=N=K=4096 with fp32
accumulation and bf16 output (its MFMA-bound shape),
in TFLOP/s of algorithmic work (2*M*N*K per step). One step = one GEMM launch
through the C ABI (ythip_gemm); inputs are resident in HBM before timing.

Also reported in the same JSON line (each timed with HIP events on the stream
the kernels are launched on):
  gemm_4096_ceilings  the headline kernel's MFMA stream alone (register
                  operands) and its global -> LDS operand stream alone, same grid
  gemm_sweep      the other configs[1] shapes (NN and the W^T "linear" layout)
  gemm_fp32       configs[0] (fp32 1024^3), and the same kernel at 4096^3
  attn_prefill    configs[2] causal flash prefill S = 512/2048/8192 (TFLOP/s), the
                  causal mask as bytes, and fp32 (the reference flash backend's dtype)
  attn_decode     configs[3] decode attention (GB/s of K/V read)
  rmsnorm_rope    fused RMSNorm+RoPE on configs[2] shapes at S=8192 (GB/s)
  attn_math       the MATH attention backend (materialised scores) at S=2048, and
                  a causal masked matmul at 4096^3
  qwen3_0p6b      configs[4] shape: 512-token prefill + greedy decode tok/s (a KV
                  ring sized to the run, and the reference's max_position_embeddings
                  ring; bf16 and fp16; the C++ host)
  yt_checkpoint   .yt checkpoint of the Qwen3-0.6B shape loaded to the device (GB/s)
  roofline        the headline kernel against MI355X dense bf16 MFMA peak
  cpu_baseline    YTensor's own CPU sgemm (compiled reference when present,
                  else the oracle restatement) on the host cores, same shape;
                  its "rows" time the same CPU path on the prefill, decode and
                  RMSNorm+RoPE shapes (single thread, bounded samples)
Synthetic data: torch.randn with fixed seeds, N(0,1) activations and
N(0,0.02) weights (the configs' distributions). The parity tests use YTensor's
own seeded generator; the benchmark only needs the shapes and magnitudes.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_bf16_4096_nn_traffic.md")


def read_traffic(path: str):
    """HBM bytes per launch of the headline kernel, from the committed rocprofv3
    PMC summary (a line `hbm_bytes_per_launch: <int>`), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("hbm_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1].strip().strip("`")))
    except OSError:
        pass
    return None


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only (no sweep, no CPU baseline)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma list of sections to run "
                                               "(gemm,ceiling,sweep,fp32,prefill,decode,norm,math,qwen3,ytload)")
    ap.add_argument("--calib", action="store_true",
                    help="first run a plain conversion-copy kernel of known size (HBM counter calibration)")
    return ap.parse_args()


def time_launches(fn, steps: int, warmup: int, torch, graph: bool = True) -> float:
    """Average milliseconds per launch of fn(), HIP events on the current stream.

    With graph=True the `steps` launches are captured once into a HIP graph
    (the C-ABI launches go to torch's current stream, which is the capture
    stream) and the timed region replays the graph: the host-side Python and
    ctypes cost of issuing each launch is then outside the measurement, so
    microsecond-scale kernels are timed back to back on the GPU."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if graph:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for _ in range(steps):
                    fn()
        torch.cuda.current_stream().wait_stream(side)
        # Capturing keeps the GPU idle for tens of milliseconds; the clocks then
        # boost, overshoot the power limit and settle over ~50 ms of load (a
        # kernel trace shows the same GEMM at 118 -> 142 -> 105 us per launch in
        # that window). Replay until 0.2 s of load have passed, as the headline
        # region's 0.5 s settle does, so every section is timed at steady clocks.
        t_end = time.perf_counter() + 0.2
        while time.perf_counter() < t_end:
            g.replay()
            torch.cuda.synchronize()
        s.record()
        g.replay()
        e.record()
        torch.cuda.synchronize()
        del g
        return s.elapsed_time(e) / steps
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def rotating(n_bufs: int, make):
    bufs = [make(i) for i in range(n_bufs)]
    state = {"i": 0}

    def nxt():
        b = bufs[state["i"] % n_bufs]
        state["i"] += 1
        return b
    return nxt


def host_info() -> dict:
    info = {"host_cpu": platform.processor() or "", "logical_cpus": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Thread(s) per core", "Core(s) per socket", "Socket(s)"):
                info[k.strip()] = v.strip()
    except Exception:
        pass
    return info


PORT_RATIO_FILE = os.path.join(ROOT, "profiles", "cpu_port_vs_reference.md")


def read_port_ratio(path: str):
    """port / reference time for the 4096^3 sgemm, measured where the compiled
    reference exists (oracle/time_port_vs_ref.py), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("port_over_reference_time:"):
                    return float(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def read_row_ratios(path: str) -> dict:
    """{cpu row: port / reference time} from the `ratio <row>: <value>` lines
    oracle/time_port_vs_ref.py writes."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                t = line.strip()
                if t.startswith("ratio ") and ":" in t:
                    k, v = t[len("ratio "):].split(":", 1)
                    out[k.strip()] = float(v)
    except (OSError, ValueError):
        pass
    return out


def cpu_baseline(M: int, N: int, K: int, budget_s: float = 12.0) -> dict:
    """YTensor's CPU path for the headline shape: the bf16 inputs are up-converted
    and multiplied by the fp32 sgemm (src/ytensor_base_math.inl:689-700), with
    the reference default of a single-threaded GEMM (g_num_threads = 0,
    include/kernel/avx2/gemm_utils.hpp:64). Timed here is the oracle's
    restatement (kind "port": the compiled reference never travels to the GPU
    box); beside it the port / reference time ratio that
    oracle/time_port_vs_ref.py measured where the reference is built. The sample
    is whole 4096^3 calls repeated for about `budget_s` seconds (median
    reported), then a shorter run with the GEMM's OpenMP threads on all cores of
    this process's CPU share (the reference's set_num_threads(n), reported
    beside)."""
    import numpy as np
    import oracle
    path = oracle.oracle()
    kind = "port"
    rng = np.random.default_rng(0)
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = (rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    A = oracle.oracle().bf16_to_f32(oracle.oracle().bf16_round(A))
    B = oracle.oracle().bf16_to_f32(oracle.oracle().bf16_round(B))

    def timed(threads: int, budget: float, min_runs: int) -> tuple[float, int]:
        path.set_num_threads(threads)
        times = []
        t_end = time.perf_counter() + budget
        while len(times) < min_runs or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            path.sgemm(A, B)
            times.append(time.perf_counter() - t0)
        return sorted(times)[len(times) // 2], len(times)

    flops = 2.0 * M * N * K
    t1, n1 = timed(1, budget_s, 2)
    try:
        ncores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "1024")))
    except (AttributeError, ValueError):
        ncores = os.cpu_count() or 1
    tn, nn = timed(ncores, budget_s / 3, 2)
    path.set_num_threads(1)
    ratio = read_port_ratio(PORT_RATIO_FILE)
    return {"value": round(flops / t1 / 1e12, 4), "unit": "TFLOP/s", "cores": 1, "kind": kind,
            "sample": f"{n1} whole {M}x{N}x{K} fp32 sgemm calls on bf16-rounded inputs (about {budget_s:.0f} s), "
                      f"median {t1:.2f} s per call, single thread (reference default g_num_threads=0)",
            "port_over_reference_time": ratio,
            "reference_equivalent_value": round(flops / t1 / 1e12 * ratio, 4) if ratio else None,
            "ratio_note": "the port's time / the compiled reference's time for the same call, measured on the "
                          "build container's host (profiles/cpu_port_vs_reference.md); the reference itself is "
                          "not run on the GPU box",
            "all_cores": {"value": round(flops / tn / 1e12, 4), "threads": ncores, "calls": nn,
                          "median_s": round(tn, 3)},
            "host": host_info()}


def cpu_rows(path, kind: str) -> dict:
    """The reference's CPU path timed beside the other GPU rows, with its own
    threading defaults (the GEMM's thread count left at 1; the attention and
    normalisation loops' OpenMP pools sized by OMP_NUM_THREADS), on bounded
    samples of the same shapes (a few seconds in all):
      prefill   yt::function::scaledDotProductAttention (FLASH_AVX2) causal GQA,
                16 q / 8 kv heads, D=128, S=2048 (src/function/ops.inl:109-234,
                src/kernel/avx2/flash_attention.inl:274-443)
      decode    the same with one query row per batch entry, B=16, ctx=8192
                (flash_attention.inl:202-272)
      norm_rope rmsNorm_ of the q and k heads + RoPE of both, S=8192
                (src/function/normalization.inl:256-277, example/qwen3/src/qwen3.cpp:522-559)
      math      scaledDotProductAttention(MATH), causal, S=2048 (src/function/ops.inl:388-418)
      masked    YTensor::masked_matmul 2048^3 with a causal predicate (src/ytensor_math.inl:372-410)
      yt_load   YTensorIO::load of a 256 MiB bf16 tensor (src/ytensor_io.inl:785-830)
    Inputs are N(0,1) (weights N(0,0.02)) rounded to bf16, as on the GPU.
    Every row carries port_over_reference_time (the port's time / the compiled
    reference's on the same call, measured where the reference is built:
    profiles/cpu_port_vs_reference.md) and the reference-equivalent rate."""
    import numpy as np
    import oracle
    o = oracle.oracle()
    path.set_num_threads(1)
    rng = np.random.default_rng(1)

    def bf(*shape, scale=1.0):
        x = rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)
        return o.bf16_to_f32(o.bf16_round(x))

    def med(fn, n):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    rows = {"kind": kind, "threads": "reference defaults: GEMM 1 thread, OpenMP loops OMP_NUM_THREADS="
                                      + os.environ.get("OMP_NUM_THREADS", "unset (all cores)")}
    S = 2048
    q, k, v = bf(1, 16, S, 128), bf(1, 8, S, 128), bf(1, 8, S, 128)
    t = med(lambda: path.sdpa_gqa(q, k, v, 1 / math.sqrt(128), True), 3)
    rows["attn_prefill_causal_S2048"] = {"s_per_call": round(t, 4),
                                         "tflops": round(4.0 * 16 * 128 * S * (S + 1) / 2 / t / 1e12, 4)}
    ctx = 8192
    q, k, v = bf(16, 16, 1, 128), bf(16, 8, ctx, 128), bf(16, 8, ctx, 128)
    t = med(lambda: path.sdpa_gqa(q, k, v, 1 / math.sqrt(128), False), 2)
    rows["attn_decode_B16_ctx8192"] = {"s_per_call": round(t, 4),
                                       "gbs_bf16_kv": round(2.0 * 16 * 8 * ctx * 128 * 2 / t / 1e9, 3)}
    del q, k, v
    S = 8192
    qk = bf(1, 24, S, 128)
    w = bf(128, scale=0.02)
    cos, sin = path.rope_tables(128, S, 1e6)

    def nr():
        path.rope(path.rms_norm(qk, w, 1e-6), cos, sin)
    t = med(nr, 3)
    byts = 2.0 * 32 * 128 * S * 2 + 2.0 * S * 128 * 4
    rows["rmsnorm_rope_S8192"] = {"s_per_call": round(t, 4), "gbs_bf16_equiv": round(byts / t / 1e9, 3)}
    del qk
    # scaledDotProductAttention(MATH), causal predicate, 16 heads, S=2048, fp32
    S = 2048
    q, k = bf(16, S, 128), bf(16, S, 128)
    t = med(lambda: path.sdpa_math(q, k, k, 0.0, diag=0), 2)
    rows["attn_math_S2048"] = {"s_per_call": round(t, 4),
                               "tflops_full_square": round(4.0 * 16 * 128 * S * S / t / 1e12, 4)}
    del q, k
    a = bf(2048, 2048)
    t = med(lambda: path.masked_matmul(a, a, diag=0, value=-1e9), 2)
    rows["masked_matmul_2048_causal"] = {"s_per_call": round(t, 4), "tflops_full": round(2.0 * 2048 ** 3 / t / 1e12, 4)}
    del a
    # YTensorIO::load of one 256 MiB bf16 tensor from a page-cache file (the
    # restatement's reader, oracle/ytio.py)
    import shutil
    import tempfile
    from oracle import ytio
    tmp = tempfile.mkdtemp(prefix="ythip_cpu_")
    try:
        p = os.path.join(tmp, "w.yt")
        w = np.arange(128 << 20, dtype=np.uint16)
        ytio.write(p, {"w": w}, types={"w": "bfloat16"})
        ytio.read(p)
        t = med(lambda: ytio.read(p), 3)
        rows["yt_load_256MiB_bf16"] = {"s_per_call": round(t, 4), "gbs": round(w.nbytes / t / 1e9, 3)}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    ratios = read_row_ratios(PORT_RATIO_FILE)
    for key, row in rows.items():
        if not isinstance(row, dict):
            continue
        r = ratios.get(key)
        row["port_over_reference_time"] = r
        if r:
            row["reference_equivalent_s_per_call"] = round(row["s_per_call"] / r, 4)
            rate = next((k for k in row if k not in ("s_per_call", "port_over_reference_time",
                                                     "reference_equivalent_s_per_call")), None)
            if rate:
                row["reference_equivalent_" + rate] = round(row[rate] * r, 4)
    return rows


def bench_qwen3(torch, dev, prompt_len: int = 512, n_tokens: int = 256, dtype=None, ring: str = "fit") -> dict:
    """configs[4] shape: random-init Qwen3-0.6B (synthetic N(0, 0.02) weights,
    bf16 (or `dtype`) matrices, fp32 norms), 512-token prompt, then greedy
    decode with each step replayed from one captured HIP graph. tok/s counts the
    decode steps. ring "fit": a KV ring of prompt + tokens + 64 rows; "default":
    max_position_embeddings rows, the size the reference's KVCache::init gives
    it (example/qwen3/src/qwen3.cpp:415-421)."""
    import numpy as np
    from ytensor_amd.qwen3 import Qwen3, Qwen3Config, weight_layout
    cfg = Qwen3Config()
    total = sum(int(np.prod(s)) for _, s in weight_layout(cfg))
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    W = torch.randn(total, device=dev, generator=g) * 0.02
    max_ctx = prompt_len + n_tokens + 64 if ring == "fit" else None
    m = Qwen3(cfg, W, max_ctx=max_ctx, max_prompt=prompt_len, dtype=dtype or torch.bfloat16)
    del W
    torch.cuda.empty_cache()
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, cfg.vocab, prompt_len).astype(np.int32)
    m.prefill(prompt)  # warm-up (kernels, allocator)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    m.prefill(prompt)
    e.record()
    torch.cuda.synchronize()
    prefill_eager_ms = s.elapsed_time(e)
    m.prefill(prompt, use_graph=True)  # capture (per prompt length) + first replay
    torch.cuda.synchronize()
    s.record()
    m.prefill(prompt, use_graph=True)
    e.record()
    torch.cuda.synchronize()
    prefill_ms = s.elapsed_time(e)
    m.capture()
    steps = n_tokens - 1
    s.record()
    for _ in range(steps):
        m.graph.replay()
    e.record()
    torch.cuda.synchronize()
    dec_ms = s.elapsed_time(e)
    toks = m.history[:n_tokens].cpu().numpy()
    per_tok_ms = dec_ms / steps
    # HBM bytes per decode token: every bf16 weight matrix once (tied LM head
    # included) + the K/V rows attended (mean context over the run).
    w_bytes = 2.0 * sum(int(np.prod(s)) for n, s in weight_layout(cfg) if "norm" not in n)
    mean_ctx = prompt_len + n_tokens / 2.0
    kv_bytes = cfg.layers * 2 * cfg.n_kv * cfg.head_dim * 2 * mean_ctx
    gbs = (w_bytes + kv_bytes) / (per_tok_ms * 1e-3) / 1e9
    return {"decode_tok_s": round(1e3 / per_tok_ms, 1), "ms_per_token": round(per_tok_ms, 4),
            "prefill_ms_512": round(prefill_ms, 3), "prefill_tok_s": round(prompt_len / prefill_ms * 1e3, 1),
            "prefill_ms_512_eager": round(prefill_eager_ms, 3),
            "prefill_note": "prefill_ms_512: the prompt's launches replayed as one HIP graph (captured once per "
                            "prompt length); _eager: the same launches issued one by one from Python",
            "bytes_per_token": w_bytes + kv_bytes, "hbm_gbs": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "tokens_generated": int(n_tokens), "kv_ring_rows": m.max_ctx,
            "distinct_tokens": int(len(set(toks.tolist()))),
            "note": "batch 1, greedy, decode step = one HIP graph replay of 143 kernels (5 per layer: "
                    "RMSNorm fused into the GEMV prologues, SwiGLU into the gate_up GEMV epilogue, q/k norm + "
                    "RoPE + cache append into the split-K attention kernel, the split merge into the o "
                    "projection's prologue)"}


def bench_qwen3_cpp(prompt_len: int = 512, n_tokens: int = 256) -> dict:
    """configs[4] through the C++ host (include/yt/qwen3.hpp, the example's
    Qwen3ForCausalLM over libythip.so; tests/cpp/qwen3_host.cpp built into
    ytensor_amd/bin/yt_qwen3): seed-3 randn * 0.02 weights drawn by YTensor's
    own RNG, the same 512-token prompt, the prompt as one graph replay, then
    n_tokens - 2 timed replays of the captured decode step (HIP events). Run as
    a child process; its JSON line is returned."""
    import subprocess
    import tempfile

    import numpy as np
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ytensor_amd", "bin", "yt_qwen3")
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 151936, prompt_len).astype(np.int32)
    with tempfile.TemporaryDirectory() as d:
        pf = os.path.join(d, "prompt.i32")
        prompt.tofile(pf)
        p = subprocess.run([exe, "bench", pf, str(n_tokens)], capture_output=True, text=True, timeout=300)
    if p.returncode != 0:
        return {"error": p.stderr.strip()[-400:]}
    return json.loads(p.stdout.strip().splitlines()[-1])


def bench_yt_load(torch, dev, reps: int = 3) -> dict:
    """.yt checkpoint to device: a Qwen3-0.6B-shaped checkpoint (the example's
    tensor names, bf16 matrices, fp32 norms, random device weights) written by
    ythip_yt_save to a temporary file, then loaded back into preallocated
    device buffers (ythip_yt_load through YTensorIO.load_many, one wait at the
    end) with the file in the page cache. GB/s of payload bytes; beside it a
    pinned host-to-device copy of 256 MiB, the PCIe ceiling the loader feeds."""
    import shutil
    import tempfile
    import numpy as np
    from ytensor_amd import io as yio
    from ytensor_amd.qwen3 import Qwen3Config, hf_names
    cfg = Qwen3Config()
    H, I, hd, nh, nkv = cfg.hidden, cfg.inter, cfg.head_dim, cfg.n_heads, cfg.n_kv
    shapes = {hf_names(cfg)["embed"]: (cfg.vocab, H), hf_names(cfg)["norm"]: (H,)}
    for i in range(cfg.layers):
        n = hf_names(cfg, i)
        shapes.update({n["q"]: (nh * hd, H), n["k"]: (nkv * hd, H), n["v"]: (nkv * hd, H), n["o"]: (H, nh * hd),
                       n["q_norm"]: (hd,), n["k_norm"]: (hd,), n["gate"]: (I, H), n["up"]: (I, H),
                       n["down"]: (H, I), n["norm1"]: (H,), n["norm2"]: (H,)})
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    src = {k: (torch.randn(s, device=dev, generator=g) * 0.02).to(torch.float32 if len(s) == 1 else torch.bfloat16)
           for k, s in shapes.items()}
    payload = sum(t.numel() * t.element_size() for t in src.values())
    tmp = tempfile.mkdtemp(prefix="ythip_bench_")
    path = os.path.join(tmp, "model.yt")
    try:
        f = yio.YTensorIO()
        t0 = time.perf_counter()
        f.open(path, yio.Write)
        for k, t in src.items():
            f.save(t, k)
        if not f.close():
            return {"error": "writing the checkpoint failed"}
        t_write = time.perf_counter() - t0
        dst = [(k, torch.empty_like(t)) for k, t in src.items()]
        f = yio.YTensorIO()
        f.open(path, yio.Read)
        f.load_many(dst)  # warm: page cache, pinned staging
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            f.load_many(dst)
            times.append(time.perf_counter() - t0)
        f.close()
        ok = all(torch.equal(src[k], d) for k, d in dst)
        best = min(times)
        # PCIe ceiling: one pinned 256 MiB host buffer copied to the device
        h = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
        dd = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        dd.copy_(h, non_blocking=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(4):
            dd.copy_(h, non_blocking=True)
        e.record()
        torch.cuda.synchronize()
        h2d = 4 * (256 << 20) / (s.elapsed_time(e) * 1e-3) / 1e9
        return {"payload_bytes": payload, "file_bytes": os.path.getsize(path), "tensors": len(src),
                "load_s": round(best, 4), "load_gbs": round(payload / best / 1e9, 2),
                "load_s_all": [round(t, 4) for t in times], "write_s": round(t_write, 3),
                "pinned_h2d_gbs": round(h2d, 2), "frac_of_pinned_h2d": round(payload / best / 1e9 / h2d, 3),
                "bit_exact": bool(ok),
                "note": "page-cache resident file; bf16 stored = bf16 on device (no conversion)"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU; --gpus > 1 is not supported (the multi-GPU "
                                   "sharding is a design in this build, not code)", "n_gpus": args.gpus}))
        return 2
    import torch
    import ytensor_amd as yt
    from ytensor_amd import ops
    yt.load()
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    only = set(filter(None, args.only.split(",")))

    def want(x):
        return (not only) or (x in only)

    out: dict = {}
    sections: dict = {}

    if args.calib:
        # 256 Mi fp32 elements read (1 GiB), written as bf16 (512 MiB): one elementwise kernel.
        src = torch.randn(256 * 1024 * 1024, device=dev)
        dst = torch.empty(src.shape, device=dev, dtype=torch.bfloat16)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()

    # ---- headline: bf16 GEMM 4096^3, NN (A [M,K] activations, B [K,N] weights) ----
    M = N = K = 4096
    A = torch.randn(M, K, device=dev).to(torch.bfloat16)
    B = (torch.randn(K, N, device=dev) * 0.02).to(torch.bfloat16)
    C = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    flops = 2.0 * M * N * K
    # An idle MI355X needs a few hundred milliseconds of load before its clocks
    # settle; without this the first section would be timed on a cold GPU.
    t_end = time.perf_counter() + 0.5
    while time.perf_counter() < t_end:
        for _ in range(20):
            ops.gemm(A, B, C)
        torch.cuda.synchronize()

    if want("gemm") and not args.quick:
        Wt = (torch.randn(N, K, device=dev) * 0.02).to(torch.bfloat16)
        ms_nn = time_launches(lambda: ops.gemm(A, B, C), args.steps, args.warmup, torch)
        ms_nt = time_launches(lambda: ops.gemm(A, Wt.t(), C), args.steps, args.warmup, torch)
        ms_torch = time_launches(lambda: torch.matmul(A, B, out=C), args.steps, args.warmup, torch)
        A16, B16, C16 = A.to(torch.float16), B.to(torch.float16), torch.empty_like(C, dtype=torch.float16)
        ms_f16 = time_launches(lambda: ops.gemm(A16, B16, C16), args.steps, args.warmup, torch)
        del A16, B16, C16
        sections["gemm_4096_bf16"] = {"NN_tflops": round(flops / ms_nn / 1e9, 2), "NT_tflops": round(flops / ms_nt / 1e9, 2),
                                      "torch_hipblaslt_NN_tflops": round(flops / ms_torch / 1e9, 2),
                                      "NN_fp16_tflops": round(flops / ms_f16 / 1e9, 2)}
        del Wt

    if want("ceiling") and not args.quick:
        # The headline GEMM's two resources, each alone, with its grid (256
        # workgroups of 8 waves, one per CU) and per-CU work (64 k steps): the
        # MFMA stream on register operands (the same 137.4 GFLOP and 32 MiB bf16
        # epilogue) and the global -> LDS operand stream (64 KiB per CU per k
        # step, 1.07 GB per launch, no MFMA). libythip_probe.so, built from
        # ytensor_amd/csrc/probe/ceiling.hip.
        from ytensor_amd import probe
        wg, ksteps = (M // 256) * (N // 256), K // 64
        pa = torch.randn(8 * wg, 128, 64, device=dev).to(torch.bfloat16)
        pb = torch.randn(8 * wg, 64, 64, device=dev).to(torch.bfloat16)
        po = torch.empty(8 * wg, 128, 64, device=dev, dtype=torch.bfloat16)
        ms_mfma = time_launches(lambda: probe.mfma_ceiling(pa, pb, po, wg, ksteps), args.steps, args.warmup, torch)
        psum = torch.empty(wg, 512, 16, dtype=torch.uint8, device=dev)
        ms_dma = time_launches(lambda: probe.dma_ceiling(A, B, psum), args.steps, args.warmup, torch)
        dma_bytes = wg * ksteps * 65536
        sections["gemm_4096_ceilings"] = {
            "mfma_register_operands": {"ms": round(ms_mfma, 5), "tflops": round(flops / ms_mfma / 1e9, 2),
                                       "frac_bf16_peak": round(flops / ms_mfma / 1e9 / PEAK_BF16_TFLOPS, 4)},
            "dma_operand_stream": {"ms": round(ms_dma, 5), "bytes_l2_to_lds": dma_bytes,
                                   "gbs": round(dma_bytes / ms_dma / 1e6, 1)},
            "note": "the headline kernel's MFMA work alone (operands in registers) and its operand DMA alone "
                    "(same grid, tile order and schedule, no LDS reads or MFMA)"}
        del pa, pb, po, psum

    if want("sweep") and not args.quick:
        sweep = []
        for (m, n, k) in [(1, 3072, 1024), (128, 3072, 1024), (2048, 151936, 1024)]:
            for layout in ("NN", "NT"):
                fl = 2.0 * m * n * k
                byts = 2.0 * (m * k + k * n + m * n)
                nb = 1 if byts > 600e6 else max(2, int(math.ceil(600e6 / byts)))  # rotate past the 256 MB MALL
                nb = min(nb, 64)
                mk = lambda i: (torch.randn(m, k, device=dev).to(torch.bfloat16),
                                (torch.randn(k, n, device=dev) * 0.02).to(torch.bfloat16) if layout == "NN"
                                else (torch.randn(n, k, device=dev) * 0.02).to(torch.bfloat16).t(),
                                torch.empty(m, n, device=dev, dtype=torch.bfloat16))
                nxt = rotating(nb, mk)

                def run():
                    a_, b_, c_ = nxt()
                    ops.gemm(a_, b_, c_)
                st = max(args.steps, 20)
                t = time_launches(run, st, args.warmup, torch)
                sweep.append({"M": m, "N": n, "K": k, "layout": layout, "ms": round(t, 5),
                              "tflops": round(fl / t / 1e9, 2), "gbs": round(byts / t / 1e6, 1),
                              "rotating_buffers": nb})
                del nxt
                torch.cuda.empty_cache()
        sections["gemm_sweep_bf16"] = sweep

    if want("fp32") and not args.quick:
        a32 = torch.randn(1024, 1024, device=dev)
        b32 = torch.randn(1024, 1024, device=dev)
        c32 = torch.empty(1024, 1024, device=dev)
        t = time_launches(lambda: ops.gemm(a32, b32, c32), args.steps, args.warmup, torch)
        fl = 2.0 * 1024 ** 3
        sections["gemm_fp32_1024"] = {"ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                                      "frac_fp32_peak": round(fl / t / 1e9 / PEAK_FP32_TFLOPS, 4)}
        del a32, b32, c32
        # the same fp32 kernel at 4096^3 (enough tiles to fill the CUs several times)
        a32 = torch.randn(4096, 4096, device=dev)
        b32 = torch.randn(4096, 4096, device=dev)
        c32 = torch.empty(4096, 4096, device=dev)
        t = time_launches(lambda: ops.gemm(a32, b32, c32), max(args.steps // 4, 5), min(args.warmup, 3), torch)
        fl = 2.0 * 4096 ** 3
        sections["gemm_fp32_4096"] = {"ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                                      "frac_fp32_peak": round(fl / t / 1e9 / PEAK_FP32_TFLOPS, 4)}
        del a32, b32, c32

    if want("prefill") and not args.quick:
        pre = []
        for S in (512, 2048, 8192):
            q = torch.randn(1, 16, S, 128, device=dev).to(torch.bfloat16)
            k = torch.randn(1, 8, S, 128, device=dev).to(torch.bfloat16)
            v = torch.randn(1, 8, S, 128, device=dev).to(torch.bfloat16)
            o = torch.empty_like(q)
            fl = 4.0 * 1 * 16 * 128 * S * (S + 1) / 2
            t = time_launches(lambda: ops.scaled_dot_product_attention(q, k, v, 1 / math.sqrt(128), "causal", out=o),
                              max(args.steps // 2, 10), args.warmup, torch)
            pre.append({"S": S, "ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                        "frac_bf16_peak": round(fl / t / 1e9 / PEAK_BF16_TFLOPS, 4)})
        sections["attn_prefill_causal_bf16"] = pre
        # the reference Qwen3's call form: the causal mask as a bool tensor
        # (KVCache::get_mask, example/qwen3/src/qwen3.cpp:104-126), staged per
        # key block; flops count the visible half, as for the causal rows
        pre_b = []
        for S in (2048, 8192):
            q = torch.randn(1, 16, S, 128, device=dev).to(torch.bfloat16)
            k = torch.randn(1, 8, S, 128, device=dev).to(torch.bfloat16)
            v = torch.randn(1, 8, S, 128, device=dev).to(torch.bfloat16)
            o = torch.empty_like(q)
            mk = torch.ones(S, S, device=dev, dtype=torch.bool).tril()
            fl = 4.0 * 1 * 16 * 128 * S * (S + 1) / 2
            t = time_launches(lambda: ops.scaled_dot_product_attention(q, k, v, 1 / math.sqrt(128), mk, out=o),
                              max(args.steps // 2, 10), args.warmup, torch)
            pre_b.append({"S": S, "ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                          "frac_bf16_peak": round(fl / t / 1e9 / PEAK_BF16_TFLOPS, 4)})
            del q, k, v, o, mk
        sections["attn_prefill_bool_mask_bf16"] = pre_b
        # fp32, the dtype of the reference's flash backend (src/function/ops.inl:
        # 119-121), on v_mfma_f32_16x16x4_f32; fraction of the fp32 MFMA peak
        pre32 = []
        for S in (2048, 8192):
            q = torch.randn(1, 16, S, 128, device=dev)
            k = torch.randn(1, 8, S, 128, device=dev)
            v = torch.randn(1, 8, S, 128, device=dev)
            o = torch.empty_like(q)
            fl = 4.0 * 1 * 16 * 128 * S * (S + 1) / 2
            t = time_launches(lambda: ops.scaled_dot_product_attention(q, k, v, 1 / math.sqrt(128), "causal", out=o),
                              max(args.steps // 4, 5), min(args.warmup, 3), torch)
            pre32.append({"S": S, "ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                          "frac_fp32_peak": round(fl / t / 1e9 / PEAK_FP32_TFLOPS, 4)})
            del q, k, v, o
        sections["attn_prefill_causal_fp32"] = pre32
        # fp32 with the causal mask given as bytes: the reference Qwen3's call form
        # on its own flash backend (fp32-only; get_mask's bool tensor)
        pre32b = []
        for S in (2048, 8192):
            q = torch.randn(1, 16, S, 128, device=dev)
            k = torch.randn(1, 8, S, 128, device=dev)
            v = torch.randn(1, 8, S, 128, device=dev)
            o = torch.empty_like(q)
            mk = torch.ones(S, S, device=dev, dtype=torch.bool).tril()
            ws = torch.empty(int(yt._lib.lib().ythip_attn_sdpa_workspace_size(1, 16, S, S, 128)), dtype=torch.uint8,
                             device=dev)
            fl = 4.0 * 1 * 16 * 128 * S * (S + 1) / 2
            t = time_launches(lambda: ops.scaled_dot_product_attention(q, k, v, 1 / math.sqrt(128), mk, out=o,
                                                                       workspace=ws),
                              max(args.steps // 4, 5), min(args.warmup, 3), torch)
            pre32b.append({"S": S, "ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                           "frac_fp32_peak": round(fl / t / 1e9 / PEAK_FP32_TFLOPS, 4)})
            del q, k, v, o, mk, ws
        sections["attn_prefill_bool_mask_fp32"] = pre32b

    if want("decode") and not args.quick:
        dec = []
        for (Bq, ctx) in [(1, 1024), (1, 8192), (16, 1024), (16, 8192)]:
            byts = 2.0 * Bq * 8 * ctx * 128 * 2
            nb = min(64, max(1, int(math.ceil(600e6 / byts))))
            mk = lambda i: (torch.randn(Bq, 16, 128, device=dev).to(torch.bfloat16),
                            torch.randn(Bq, 8, ctx, 128, device=dev).to(torch.bfloat16),
                            torch.randn(Bq, 8, ctx, 128, device=dev).to(torch.bfloat16),
                            torch.empty(Bq, 16, 128, device=dev, dtype=torch.bfloat16))
            nxt = rotating(nb, mk)
            ws = torch.empty(ops.decode_workspace_bytes(Bq, 16, ctx, 128), dtype=torch.uint8, device=dev)

            def run():
                q_, k_, v_, o_ = nxt()
                ops.decode_attention(q_, k_, v_, out=o_, workspace=ws)
            t = time_launches(run, max(args.steps, 20), args.warmup, torch)
            dec.append({"B": Bq, "ctx": ctx, "ms": round(t, 5), "gbs": round(byts / t / 1e6, 1),
                        "frac_hbm": round(byts / t / 1e6 / PEAK_HBM_GBS, 4), "rotating_buffers": nb})
            del nxt
            torch.cuda.empty_cache()
        sections["attn_decode_bf16"] = dec
        # The reference Qwen3's per-token call form (qwen3.cpp:250-264):
        # scaledDotProductAttention with q_len == 1 and KVCache::get_mask's bool
        # mask [1, ctx], which the library sends to the same split-K kernel
        # (flash_attention.inl:469-499 routes every q_len == 1 call to decode).
        dec_m = []
        for (Bq, ctx) in [(1, 1024), (1, 8192), (16, 1024), (16, 8192)]:
            byts = 2.0 * Bq * 8 * ctx * 128 * 2
            nb = min(64, max(1, int(math.ceil(600e6 / byts))))
            mk = lambda i: (torch.randn(Bq, 16, 1, 128, device=dev).to(torch.bfloat16),
                            torch.randn(Bq, 8, ctx, 128, device=dev).to(torch.bfloat16),
                            torch.randn(Bq, 8, ctx, 128, device=dev).to(torch.bfloat16),
                            torch.empty(Bq, 16, 1, 128, device=dev, dtype=torch.bfloat16))
            nxt = rotating(nb, mk)
            mask = torch.ones(1, ctx, device=dev, dtype=torch.bool)
            ws = torch.empty(int(yt.lib().ythip_attn_sdpa_workspace_size(Bq, 16, 1, ctx, 128)), dtype=torch.uint8,
                             device=dev)

            def run():
                q_, k_, v_, o_ = nxt()
                ops.scaled_dot_product_attention(q_, k_, v_, 0.0, mask, out=o_, workspace=ws)
            t = time_launches(run, max(args.steps, 20), args.warmup, torch)
            dec_m.append({"B": Bq, "ctx": ctx, "ms": round(t, 5), "gbs": round(byts / t / 1e6, 1),
                          "frac_hbm": round(byts / t / 1e6 / PEAK_HBM_GBS, 4), "rotating_buffers": nb})
            del nxt
            torch.cuda.empty_cache()
        sections["attn_decode_sdpa_bool_mask_bf16"] = dec_m

    if want("norm") and not args.quick:
        S = 8192
        qkv = torch.randn(1, S, 32 * 128, device=dev).to(torch.bfloat16)
        wq = torch.randn(128, device=dev) * 0.02
        wk = torch.randn(128, device=dev) * 0.02
        ang = torch.arange(S, device=dev)[:, None] * torch.rand(1, 128, device=dev)
        cos, sin = torch.cos(ang).contiguous(), torch.sin(ang).contiguous()
        qo = torch.empty(1, 16, S, 128, device=dev, dtype=torch.bfloat16)
        ko = torch.empty(1, 8, S, 128, device=dev, dtype=torch.bfloat16)
        vo = torch.empty(1, 8, S, 128, device=dev, dtype=torch.bfloat16)
        byts = 2.0 * 32 * 128 * S * 2 + 2.0 * S * 128 * 4
        t = time_launches(lambda: ops.rms_norm_rope(qkv, 16, 8, 128, wq, wk, 1e-6, cos, sin, 0, qo, ko, vo),
                          args.steps, args.warmup, torch)
        sections["rmsnorm_rope_bf16_S8192"] = {"ms": round(t, 5), "gbs": round(byts / t / 1e6, 1),
                                               "frac_hbm": round(byts / t / 1e6 / PEAK_HBM_GBS, 4)}

    if want("math") and not args.quick:
        # MATH backend (materialised scores) and masked matmul: the whole S x S
        # product is computed, so flops count the full square; bytes are the
        # fp32 scores written + read and the bf16 weights written + read.
        S = 2048
        q = torch.randn(1, 16, S, 128, device=dev).to(torch.bfloat16)
        k = torch.randn(1, 8, S, 128, device=dev).to(torch.bfloat16)
        v = torch.randn(1, 8, S, 128, device=dev).to(torch.bfloat16)
        o = torch.empty_like(q)
        ws = torch.empty(int(yt.lib().ythip_attn_math_workspace_size(2, 1, 16, S, S)), dtype=torch.uint8,
                         device=dev)
        t = time_launches(lambda: ops.scaled_dot_product_attention(q, k, v, 0.0, "causal", out=o, backend="math",
                                                                   workspace=ws), max(args.steps // 2, 10),
                          args.warmup, torch)
        fl = 4.0 * 16 * 128 * S * S
        byts = 16.0 * S * S * (4 + 4 + 2 + 2)
        M2 = 4096
        a2 = torch.randn(M2, M2, device=dev).to(torch.bfloat16)
        b2 = (torch.randn(M2, M2, device=dev) * 0.02).to(torch.bfloat16)
        c2 = torch.empty(M2, M2, device=dev, dtype=torch.bfloat16)
        w2 = torch.empty(ops.masked_gemm_workspace_bytes(1, M2, M2), dtype=torch.uint8, device=dev)
        t2 = time_launches(lambda: ops.gemm_masked(a2, b2, c2, "causal", fill=-1e9, workspace=w2),
                           max(args.steps // 2, 10), args.warmup, torch)
        sections["attn_math_bf16_S2048"] = {
            "ms": round(t, 5), "tflops_full_square": round(fl / t / 1e9, 2),
            "gbs_scores": round(byts / t / 1e6, 1), "frac_hbm": round(byts / t / 1e6 / PEAK_HBM_GBS, 4),
            "note": "causal, 16 q / 8 kv heads, D=128; scores fp32 + weights bf16 materialised (HBM-bound)"}
        sections["masked_matmul_bf16_4096_causal"] = {
            "ms": round(t2, 5), "tflops_full": round(2.0 * M2 ** 3 / t2 / 1e9, 2),
            "note": "fill -1e9 above the diagonal; the product is computed whole, then masked"}
        del q, k, v, o, ws, a2, b2, c2, w2
        torch.cuda.empty_cache()

    if want("qwen3") and not args.quick:
        sections["qwen3_0p6b_decode"] = bench_qwen3(torch, dev)
        torch.cuda.empty_cache()
        sections["qwen3_0p6b_decode_default_ring"] = bench_qwen3(torch, dev, ring="default")
        torch.cuda.empty_cache()
        sections["qwen3_0p6b_decode_cpp_host"] = bench_qwen3_cpp()
        sections["qwen3_0p6b_decode_fp16"] = bench_qwen3(torch, dev, dtype=torch.float16)
        torch.cuda.empty_cache()

    if want("ytload") and not args.quick:
        try:
            sections["yt_checkpoint_load"] = bench_yt_load(torch, dev)
        except Exception as exc:  # reported, never required
            sections["yt_checkpoint_load"] = {"error": repr(exc)}
        torch.cuda.empty_cache()

    # ---- the timed headline region: exactly K steps, synchronised both sides ----
    # The sections above end with host-side work (checkpoint I/O, CPU timing),
    # during which the GPU idles and its clocks drop: settle them again with
    # 0.5 s of the same GEMM (untimed), as before the kernel measurement.
    t_end = time.perf_counter() + 0.5
    while time.perf_counter() < t_end:
        for _ in range(20):
            ops.gemm(A, B, C)
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        ops.gemm(A, B, C)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()  # torch's current stream: the stream the C-ABI launches on
    for _ in range(args.steps):
        ops.gemm(A, B, C)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    value = flops / (ms_step * 1e-3) / 1e12

    # Roofline of the headline kernel over the same timed region: HIP events
    # on the launch stream bracket the K launches (back to back, the host runs
    # ahead of the GPU), so their average is the kernel's launch duration.
    ms = ev0.elapsed_time(ev1) / args.steps
    tflops = flops / (ms * 1e-3) / 1e12
    traffic = read_traffic(TRAFFIC_FILE)
    roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "kernel": "gemm_pingpong_kernel<BF16,BF16,NN=true> (256x256 tile, 8 waves, ping-pong)",
                "algorithmic_flops_per_launch": flops, "avg_launch_ms": round(ms, 5)}

    cpu = None
    if not args.quick and not args.no_cpu:
        try:
            cpu = cpu_baseline(M, N, K)
        except Exception as exc:  # the baseline is reported, never required
            cpu = {"error": repr(exc)}
        if not only and "error" not in cpu:
            try:
                import oracle
                cpu["rows"] = cpu_rows(oracle.oracle(), cpu["kind"])
            except Exception as exc:
                cpu["rows"] = {"error": repr(exc)}

    out = {
        "metric": "bf16 GEMM & flash-attn TFLOP/s (% MFMA peak); decode tok/s at Qwen3-0.6B shape",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch.randn, seed 0: A ~ N(0,1), B ~ N(0,0.02), bf16)",
        "config": {"workload": "bf16 GEMM M=N=K=4096, A [M,K] x B [K,N] row-major, fp32 accumulate, bf16 out "
                               "(configs[1])", "M": M, "N": N, "K": K, "layout": "NN",
                   "untimed_clock_settle_s": 0.5},
        "roofline": roofline,
        "cpu_baseline": cpu,
        **sections,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
