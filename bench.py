"""Benchmark of the fused linear + bias + GELU kernel on one MI355X.

Default workload (the one the headline metric is quoted on): a single fused
addmm + bias + exact-erf GELU, fp32, M = N = K = 4096, A row-major and
B = W^T of a contiguous nn.Linear weight W[N,K] (strided operand), on the
IEEE fp32 MFMA path.  A "step" is one fused kernel launch over that problem
with the inputs already resident in HBM.

Prints ONE JSON line with the throughput (TFLOP/s from 2*M*N*K), the
roofline of the kernel (HIP-event launch durations on the launch stream
against MI355X's dense MFMA peak) and the reference's CPU path (torch addmm
+ GELU on the host cores) as a reported baseline.  Additional workloads are
reported under "extra" unless --no-extra is given.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

PEAK_TFLOPS = {torch.float32: 157.3, torch.bfloat16: 2516.6, torch.float16: 2516.6}
HBM_GBPS = 8000.0
COPY_BYTES = 256 * 1024 * 1024  # --calibrate-copy: bytes read and bytes written by the copy
DTYPE_NAMES = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _inputs(m, n, k, dtype, dev, seed, *, bias=True, w_std=None, a_std=None):
    g = torch.Generator().manual_seed(seed)
    a_std = k ** -0.25 if a_std is None else a_std
    w_std = k ** -0.25 if w_std is None else w_std
    a = (torch.randn(m, k, generator=g) * a_std).to(dtype).to(dev)
    w = (torch.randn(n, k, generator=g) * w_std).to(dtype).to(dev)
    b = ((torch.rand(n, generator=g) * 0.2 - 0.1).to(dtype).to(dev)) if bias else None
    return a, w.t(), b


def _time_launches(launch, steps: int, warmup: int):
    """The timed region: `warmup` untimed launches, then `steps` back-to-back
    launches bracketed by synchronisation, with a HIP event recorded on the
    launch stream on each side.  Returns (wall-clock ms per step, GPU ms per
    launch over the region from those events, each launch's ms from a separate
    pass with an event between launches).  The events between launches leave
    a gap of a few µs and slow a long kernel by a few percent (its next launch
    no longer starts on CUs the previous one has just freed), so the region's
    own events give the launch duration."""
    from forgeml_amd.measurement import event_times

    per_launch = event_times(launch, iters=steps, warmup=warmup, stream=torch.cuda.current_stream())
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        launch()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        launch()
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return wall_ms, start.elapsed_time(end) / steps, per_launch


def _row_sample(m: int, count: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(m)
    picked = torch.randperm(m, generator=g)[: max(0, count - 2)]
    return torch.cat([torch.tensor([0, m - 1]), picked]).unique().sort().values


def _gate_gemm(out, a, b, bias, act, rows=64):
    """The correctness gate before timing (src/forgeml/benchmarks.py:84-87): the
    kernel's output on sampled rows against the reference's CPU path at the
    parity tolerance; 16-bit outputs also against the epilogue contract."""
    from oracle.fused_linear import contract_ulp_check, reference_cpu, tolerance

    idx = _row_sample(a.shape[0], rows)
    a_rows = a[idx.to(a.device)].cpu()
    b_cpu = b.cpu()
    bias_cpu = None if bias is None else bias.cpu()
    activation = "gelu" if act == "gelu" else "none"
    got = out[idx.to(out.device)].cpu()
    expected = reference_cpu(a_rows, b_cpu, bias_cpu, activation)
    rtol, atol = tolerance(out.dtype, a.shape[1])
    err = (got.double() - expected.double()).abs()
    ok = bool(torch.isfinite(got).all()) and bool((err <= atol + rtol * expected.double().abs()).all())
    record = {"passed": ok, "rows_checked": int(idx.numel()), "rtol": rtol, "atol": atol,
              "max_abs_err": float(err.max())}
    if out.dtype != torch.float32:
        report = contract_ulp_check(got, a_rows, b_cpu, bias_cpu, activation, "none")
        record["contract"] = report
        record["passed"] = ok and report["bad"] == 0 and report["exact_frac"] >= 0.99
    return record


def gemm_workload(name, m, n, k, dtype, *, steps, warmup, act="gelu", bias=True, a_std=None, w_std=None,
                  config=None, vendor=False):
    """One GEMM workload through this library's kernel, or with `vendor` through torch's
    library GEMM (hipBLASLt: `torch.matmul(A, W^T, out=)`, no bias or activation) on the
    same operands, as a reference point for the counters."""
    from forgeml_amd import kernels

    dev = torch.device("cuda", 0)
    a, b, bvec = _inputs(m, n, k, dtype, dev, seed=0, bias=bias, a_std=a_std, w_std=w_std)
    out = torch.empty(m, n, dtype=dtype, device=dev)
    cfg = config or kernels.DEFAULT_CONFIG
    resolved = kernels.resolve_config(m, n, k, dtype, cfg)

    if vendor:
        def launch():
            torch.matmul(a, b, out=out)
    else:
        def launch():
            kernels.matmul(a, b, bvec, activation=act, out=out, config=cfg)

    gate = None
    if not vendor:
        launch()
        torch.cuda.synchronize()
        gate = _gate_gemm(out, a, b, bvec, act)
    wall_ms, avg_ms, per_launch = _time_launches(launch, steps, warmup)
    flop = 2 * m * n * k
    esz = a.element_size()
    algo_bytes = (m * k + k * n + m * n + (n if bias else 0)) * esz
    return {
        "workload": name,
        "shape": [m, n, k],
        "dtype": DTYPE_NAMES[dtype],
        "kernel": "torch.matmul (vendor library GEMM, no epilogue)" if vendor else "forgeml_hip fused GEMM",
        "activation": "none" if vendor else act,
        "bias": bias and not vendor,
        "tile": None if vendor else [resolved.block_m, resolved.block_n, resolved.block_k, resolved.num_waves],
        "ms_per_step": wall_ms,
        "kernel_ms_avg": avg_ms,
        "kernel_ms_per_launch_events_median": statistics.median(per_launch),
        "tflops": flop / (wall_ms * 1e-3) / 1e12,
        "kernel_tflops": flop / (avg_ms * 1e-3) / 1e12,
        "pct_peak": 100.0 * flop / (avg_ms * 1e-3) / 1e12 / PEAK_TFLOPS[dtype],
        "algorithmic_bytes": algo_bytes,
        "flop": flop,
        "gate": gate,
    }


def _graph_per_call_us(calls, replays: int = 10) -> float:
    """Capture `calls` (a list of launch closures) into one HIP graph and return the
    mean GPU time per captured call over `replays` replays (HIP events)."""
    for fn in calls[:3]:
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in calls[:2]:
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in calls:
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (replays * len(calls))


SKINNY_POOL_BYTES = 320 << 20  # weights rotate through more than the 256 MB Infinity Cache


def skinny_workload(m, n, k, dtype):
    """HBM-bound skinny GEMM (C = GELU(A W^T + bias), M tiny): GPU time per call inside a
    HIP graph, the weight read from a rotating pool larger than the Infinity Cache."""
    from forgeml_amd import kernels

    dev = torch.device("cuda", 0)
    esz = torch.tensor([], dtype=dtype).element_size()
    nbuf = max(2, -(-SKINNY_POOL_BYTES // (n * k * esz)))
    g = torch.Generator(device=dev).manual_seed(0)
    a = (torch.randn(m, k, generator=g, device=dev) * k ** -0.25).to(dtype)
    weights = [(torch.randn(n, k, generator=g, device=dev) * k ** -0.25).to(dtype) for _ in range(nbuf)]
    bias = (torch.rand(n, generator=g, device=dev) * 0.2 - 0.1).to(dtype)
    out = torch.empty(m, n, dtype=dtype, device=dev)
    plan = kernels.plan(a, weights[0].t())
    ws = torch.empty(plan["workspace_bytes"], dtype=torch.uint8, device=dev) if plan["workspace_bytes"] else None
    act = kernels._act_code("gelu", "none")
    calls = [lambda w=w: kernels.launch(a, w.t(), bias, out, act=act, config_id=-1, workspace=ws) for w in weights]
    calls[0]()
    torch.cuda.synchronize()
    gate = _gate_gemm(out, a, weights[0].t(), bias, "gelu", rows=m)
    us = _graph_per_call_us(calls)
    algo_bytes = (m * k + k * n + m * n + n) * esz
    cfg = plan["config"]
    del weights
    return {
        "workload": f"skinny_{DTYPE_NAMES[dtype]}_{m}x{n}x{k}_bias_gelu",
        "shape": [m, n, k],
        "dtype": DTYPE_NAMES[dtype],
        "us_per_call_in_graph": round(us, 2),
        "algorithmic_bytes": algo_bytes,
        "GB_per_s": round(algo_bytes / us / 1e3, 1),
        "hbm_frac": round(algo_bytes / us / 1e3 / HBM_GBPS, 4),
        "kernel": plan["kernel"],
        "tile": [cfg.block_m, cfg.block_n],
        "k_splits": plan["k_splits"],
        "gate": gate,
    }


SKINNY_SHAPES = [(m, n, k, dt) for dt in (torch.float32, torch.bfloat16) for m in (1, 33)
                 for n, k in ((3072, 1024), (3000, 1531))]


# Before a latency measurement on the GPU, its variants run back to back for
# this long: the GPU leaves its idle clocks over tens of milliseconds (a
# transformer block measured 623 us per call over its first 20 synchronized
# calls, then 545), and the CPU baseline before it leaves the GPU idle.
GPU_WARMUP_S = 0.3


@torch.inference_mode()
def _gpu_warm(fns) -> None:
    fns = list(fns)
    t_end = time.perf_counter() + GPU_WARMUP_S
    while time.perf_counter() < t_end:
        for fn in fns:
            fn()
        torch.cuda.synchronize()


def compiled_workload(name, make_model, make_input, *, steps, warmup, cpu_budget_s=20.0):
    """CompiledModel forward latency (synchronized host wall clock, as the reference
    times it): eager hip backend, the same captured in a HIP graph, and the
    reference's CPU path (the model compiled with the torch backend, on the host)."""
    import forgeml_amd
    from forgeml_amd.measurement import measure_variants

    dev = torch.device("cuda", 0)
    model_cpu, x_cpu = make_model(), make_input()
    compiled_cpu = forgeml_amd.compile(model_cpu, (x_cpu,), backend="torch")
    cpu = []
    t_end = time.perf_counter() + cpu_budget_s
    with torch.inference_mode():
        compiled_cpu(x_cpu)
        while len(cpu) < 10 and (len(cpu) < 3 or time.perf_counter() < t_end):
            t0 = time.perf_counter()
            compiled_cpu(x_cpu)
            cpu.append((time.perf_counter() - t0) * 1e3)
    with torch.inference_mode():
        expected = compiled_cpu(x_cpu).clone()
    model = make_model().to(dev).eval()
    x = x_cpu.to(dev)
    compiled = forgeml_amd.compile(model, (x,), backend="hip")
    graphed = compiled.capture_graph(x)
    # The gate before timing: the hip compile and its graph against the CPU
    # compile at the fp32 parity tolerance with K of the widest GEMM.
    from oracle.fused_linear import tolerance

    specs = compiled.graph.specs()
    widest_k = max(specs[n.inputs[0]].shape[-1] for n in compiled.graph.nodes
                   if n.op in ("linear", "fused_linear_gelu", "matmul"))
    rtol, atol = tolerance(torch.float32, widest_k)
    gate = {"rtol": rtol, "atol": atol}
    for label, fn in (("hip", lambda: compiled(x)), ("hip_graph", lambda: graphed(x))):
        got = fn().cpu()
        err = (got.double() - expected.double()).abs()
        gate[label] = bool(torch.isfinite(got).all()) and bool((err <= atol + rtol * expected.double().abs()).all())
        gate[f"{label}_max_abs_err"] = float(err.max())
    gate["passed"] = gate["hip"] and gate["hip_graph"]
    variants = {"hip": lambda: compiled(x), "hip_graph": lambda: graphed(x), "torch_eager_gpu": lambda: model(x)}
    _gpu_warm(variants.values())
    timings = measure_variants(variants, device=dev, warmup=warmup, repeats=max(steps, 2))
    # The reference's numerically gated autotuner (CompiledModel.autotune), then a new graph.
    compiled.autotune(x, warmup=2, repeats=5)
    tuned_graph = compiled.capture_graph(x)
    _gpu_warm([lambda: tuned_graph(x)])
    tuned = measure_variants({"hip_tuned_graph": lambda: tuned_graph(x)}, device=dev, warmup=warmup,
                             repeats=max(steps, 2))["hip_tuned_graph"]
    cpu_ms = statistics.median(cpu)
    return {
        "workload": name,
        "kernel_plan": sorted(set(compiled.kernel_plan.values())),
        "hip_median_us": round(timings["hip"]["median_ms"] * 1e3, 1),
        "hip_p95_us": round(timings["hip"]["p95_ms"] * 1e3, 1),
        "hip_graph_median_us": round(timings["hip_graph"]["median_ms"] * 1e3, 1),
        "hip_graph_p95_us": round(timings["hip_graph"]["p95_ms"] * 1e3, 1),
        "hip_tuned_graph_median_us": round(tuned["median_ms"] * 1e3, 1),
        "hip_tuned_graph_p95_us": round(tuned["p95_ms"] * 1e3, 1),
        "torch_eager_gpu_median_us": round(timings["torch_eager_gpu"]["median_ms"] * 1e3, 1),
        "torch_eager_gpu_p95_us": round(timings["torch_eager_gpu"]["p95_ms"] * 1e3, 1),
        "gate": gate,
        "tuned_configs": {node: f"{c.block_m}x{c.block_n}x{c.num_waves}" for node, c in compiled.kernel_configs.items()},
        "fused_residual_adds": len(compiled.fused_residuals),
        "gpu_warmup_s": GPU_WARMUP_S,
        "cpu_reference_median_us": round(cpu_ms * 1e3, 1),
        "cpu_reference_threads": torch.get_num_threads(),
        "cpu_reference_samples": len(cpu),
        "speedup_vs_cpu_tuned_graph": round(cpu_ms / tuned["median_ms"], 1),
    }


def _cpu_run(a, w, bias, threads: int, budget_s: float, max_reps: int):
    from oracle.fused_linear import reference_cpu

    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        reference_cpu(a, w.t(), bias, "gelu")
        samples = []
        t_end = time.perf_counter() + budget_s
        while len(samples) < max_reps and (len(samples) < 3 or time.perf_counter() < t_end):
            t0 = time.perf_counter()
            reference_cpu(a, w.t(), bias, "gelu")
            samples.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(previous)
    return samples


def cpu_baseline(m, n, k, *, budget_s: float = 10.0, max_reps: int = 30):
    """The reference's CPU path (torch addmm + erf GELU, fp32) on the host's
    physical cores, and on one thread as the reference's captures ran
    (src/forgeml/benchmarks.py:159,184), on the same seeded operands.  The
    one-thread run takes a 512-row sample of A (the rate per row is the same,
    and the full problem would take minutes on one core)."""
    from forgeml_amd.measurement import cpu_description, percentile

    host = cpu_description()
    cores = host.get("physical_cores") or os.cpu_count() or 1
    cores = min(cores, host.get("usable_cpus", cores))
    g = torch.Generator().manual_seed(0)
    a = torch.randn(m, k, generator=g) * k ** -0.25
    w = torch.randn(n, k, generator=g) * k ** -0.25
    bias = torch.rand(n, generator=g) * 0.2 - 0.1
    full = _cpu_run(a, w, bias, cores, budget_s, max_reps)
    rows1 = 512
    one = _cpu_run(a[:rows1].contiguous(), w, bias, 1, budget_s, 5)
    med, med1 = statistics.median(full), statistics.median(one)
    return {
        "value": 2 * m * n * k / med / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"torch.addmm(bias, A, W^T) + F.gelu on the CPU, fp32, M=N=K=4096 (full problem) on {cores} "
                  f"threads (one per physical core): median of {len(full)} runs, {med * 1e3:.1f} ms each",
        "p95_ms": round(percentile(full, 0.95) * 1e3, 2),
        "one_thread": {
            "value": 2 * rows1 * n * k / med1 / 1e12,
            "unit": "TFLOP/s",
            "sample": f"the same path on 1 thread over a {rows1}-row sample of A ({rows1}x{n}x{k}), "
                      f"median of {len(one)} runs, {med1 * 1e3:.1f} ms each",
        },
        "host": host,
    }


# Extra GEMM workloads: (M, N, K, dtype) and their options.
EXTRA_GEMMS = {
    "decoder_mlp_up_bf16_8192x14336x4096_gelu": (8192, 14336, 4096, torch.bfloat16),
    "decoder_mlp_down_bf16_8192x4096x14336_bias": (8192, 4096, 14336, torch.bfloat16),
    "fused_addmm_bias_gelu_bf16_4096": (4096, 4096, 4096, torch.bfloat16),
}
EXTRA_KW = {
    "decoder_mlp_up_bf16_8192x14336x4096_gelu": dict(bias=False, a_std=1.0, w_std=0.02),
    "decoder_mlp_down_bf16_8192x4096x14336_bias": dict(act="none", a_std=0.5, w_std=0.02),
    "fused_addmm_bias_gelu_bf16_4096": dict(),
}


def _measured_traffic(key: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE runs, if
    they were taken for this exact kernel tile; None otherwise."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    try:
        table = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = table.get(key)
    return None if entry is None else entry["traffic_bytes"]


LN_SHAPES = [(4096, 768, torch.float32), (4096, 4096, torch.float32), (4096, 8192, torch.float32),
             (2048, 12288, torch.bfloat16), (4096, 16384, torch.bfloat16), (1024, 65536, torch.float32),
             (512, 200000, torch.float32)]
ATTN_CASES = [(8, 12, 512, 64, True), (8, 12, 512, 128, True), (4, 32, 1024, 128, True), (4, 32, 1024, 128, False)]


def block_op_workloads(steps: int, warmup: int):
    """The transformer block's LayerNorm and attention kernels against torch's
    GPU kernels for the same ops, one record per case.  ``us`` is the GPU time
    per launch over ``steps`` back-to-back launches (HIP events around the
    block, after at least 10 warmup launches: the first launches of a long
    kernel run while the clock ramps); ``us_per_launch_median`` the median of
    events recorded between the launches (each adds a few µs of gap).  Ours
    and torch's are timed the same way.  LayerNorm also reports its HBM floor
    (read x, write y at 8 TB/s)."""
    import torch.nn.functional as F

    from forgeml_amd import kernels
    from forgeml_amd.measurement import event_times

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)

    def med_us(fn):
        """(block mean, per-launch median) in µs."""
        per = event_times(fn, iters=steps, warmup=max(warmup, 10))
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        stream.synchronize()
        return round(start.elapsed_time(end) * 1e3 / steps, 2), round(statistics.median(per) * 1e3, 2)

    for rows, cols, dt in LN_SHAPES:
        x = torch.randn(rows, cols, device=dev, generator=g).to(dt)
        w = torch.randn(cols, device=dev, generator=g).to(dt)
        b = torch.randn(cols, device=dev, generator=g).to(dt)
        got = kernels.layer_norm(x, (cols,), w, b, 1e-5).float().cpu()
        want = F.layer_norm(x.float().cpu(), (cols,), w.float().cpu(), b.float().cpu(), 1e-5)
        tol = 1e-4 if dt == torch.float32 else 2.0 ** -7
        gate = {"passed": bool(((got - want).abs() <= tol * (1 + want.abs())).all()),
                "max_abs_err": float((got - want).abs().max())}
        ours, ours_med = med_us(lambda: kernels.layer_norm(x, (cols,), w, b, 1e-5))
        ref, ref_med = med_us(lambda: F.layer_norm(x, (cols,), w, b, 1e-5))
        floor = 2 * x.numel() * x.element_size() / (HBM_GBPS * 1e3)
        yield {"workload": f"layer_norm_{DTYPE_NAMES[dt]}_{rows}x{cols}", "us": ours, "torch_gpu_us": ref,
               "us_per_launch_median": ours_med, "torch_gpu_us_per_launch_median": ref_med,
               "hbm_floor_us": round(floor, 2), "hbm_frac": round(floor / ours, 3), "gate": gate}
        del x, w, b
    for bsz, heads, seq, dim, causal in ATTN_CASES:
        q, k, v = (torch.randn(bsz, heads, seq, dim, device=dev, generator=g) for _ in range(3))
        got = kernels.attention(q, k, v, is_causal=causal).cpu()
        want = F.scaled_dot_product_attention(q.cpu(), k.cpu(), v.cpu(), is_causal=causal)
        gate = {"passed": bool(((got - want).abs() <= 1e-5 + 1e-4 * want.abs()).all()),
                "max_abs_err": float((got - want).abs().max())}
        ours, ours_med = med_us(lambda: kernels.attention(q, k, v, is_causal=causal))
        ref, ref_med = med_us(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal))
        flop = 4 * bsz * heads * seq * seq * dim * (0.5 if causal else 1.0)
        yield {"workload": f"attention_fp32_{bsz}x{heads}x{seq}x{dim}_{'causal' if causal else 'full'}", "us": ours,
               "torch_gpu_us": ref, "us_per_launch_median": ours_med, "torch_gpu_us_per_launch_median": ref_med,
               "tflops": round(flop / ours / 1e6, 1), "gate": gate}
        del q, k, v


# The transformer block's GEMMs (d = 768, 8 x 512 tokens, FFN 3072) on the
# tiles its autotuner picks, QKV also on 128x128, and the fp32 headline.
BLOCK_GEMMS = [("qkv_4096x2304x768", 4096, 2304, 768, "none", (64, 64, 4)),
               ("qkv_4096x2304x768", 4096, 2304, 768, "none", (128, 128, 4)),
               ("ffn_up_4096x3072x768_gelu", 4096, 3072, 768, "gelu", (128, 128, 4)),
               ("ffn_down_4096x768x3072", 4096, 768, 3072, "none", (64, 64, 4)),
               ("out_proj_4096x768x768", 4096, 768, 768, "none", (64, 64, 4)),
               ("headline_4096x4096x4096_gelu", 4096, 4096, 4096, "gelu", (256, 256, 8))]


def block_gemm_launches(steps: int):
    """Each BLOCK_GEMMS case gated on sampled rows, then launched ``steps`` times
    back to back (fp32, B = W^T, bias, the activation shown): a fixed sequence
    of dispatches for counter runs, one record per case."""
    from forgeml_amd import kernels

    dev = torch.device("cuda", 0)
    for name, m, n, k, act, tile in BLOCK_GEMMS:
        a, b, bias = _inputs(m, n, k, torch.float32, dev, seed=m + n + k)
        cfg = next(c for c in kernels.candidates(torch.float32) if (c.block_m, c.block_n, c.num_waves) == tile)
        out = kernels.matmul(a, b, bias, activation=act, config=cfg)
        torch.cuda.synchronize()
        gate = _gate_gemm(out, a, b, bias, act)
        cid = kernels.config_id(cfg, torch.float32)
        plan = kernels.plan(a, b, cfg)
        ws = torch.empty(plan["workspace_bytes"], dtype=torch.uint8, device=dev) if plan["workspace_bytes"] else None
        code = kernels._act_code(act, "none")
        for _ in range(steps):
            kernels.launch(a, b, bias, out, act=code, config_id=cid, workspace=ws)
        torch.cuda.synchronize()
        yield {"workload": name, "shape": [m, n, k], "tile": list(tile), "kernel": plan["kernel"],
               "k_splits": plan["k_splits"], "launches": steps, "gate": gate}
        del a, b, bias, out


def _calibration_copy() -> None:
    """One plain 256 MiB device copy: a dispatch of known bytes read and written,
    against which HBM byte counters of the other dispatches are scaled."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=sorted(EXTRA_GEMMS), default=None,
                    help="run one extra GEMM workload only (for profiling) and print its record")
    ap.add_argument("--tile", default=None, metavar="BMxBNxWAVES",
                    help="with --only: force this tile configuration instead of the shape heuristic")
    ap.add_argument("--vendor", action="store_true",
                    help="with --only: time torch's library GEMM (hipBLASLt) on the same operands instead")
    ap.add_argument("--block-ops", action="store_true",
                    help="time the LayerNorm and attention kernels against torch's GPU kernels instead")
    ap.add_argument("--skinny", action="store_true",
                    help="run only the skinny (HBM-bound) GEMM records, one JSON line each (for counter runs)")
    ap.add_argument("--block-gemms", action="store_true",
                    help="launch the transformer block's four fp32 GEMM shapes (and the headline) --steps times each "
                         "on fixed tiles, one JSON line each (for counter runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one plain 256 MiB device copy (reference point for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the kernel is single-GPU; see the sharding notes in DESIGN.md)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.block_ops:
        for rec in block_op_workloads(args.steps, args.warmup):
            print(json.dumps(rec), flush=True)
        return 0
    if args.only:
        config = None
        if args.tile:
            from forgeml_amd import kernels

            bm, bn, waves = (int(v) for v in args.tile.lower().split("x"))
            matches = [c for c in kernels.candidates(EXTRA_GEMMS[args.only][3])
                       if (c.block_m, c.block_n, c.num_waves) == (bm, bn, waves)]
            if not matches:
                print(f"no built tile {args.tile} for this dtype", file=sys.stderr)
                return 2
            config = matches[0]
        print(json.dumps(gemm_workload(args.only, *EXTRA_GEMMS[args.only], steps=args.steps, warmup=args.warmup,
                                       config=config, vendor=args.vendor, **EXTRA_KW[args.only])), flush=True)
        return 0
    if args.block_gemms:
        if args.calibrate_copy:
            _calibration_copy()
        ok = True
        for rec in block_gemm_launches(args.steps):
            ok = ok and rec["gate"]["passed"]
            print(json.dumps(rec), flush=True)
        return 0 if ok else 1
    if args.skinny:
        if args.calibrate_copy:
            _calibration_copy()
        ok = True
        for shape in SKINNY_SHAPES:
            rec = skinny_workload(*shape)
            ok = ok and rec["gate"]["passed"]
            print(json.dumps(rec), flush=True)
        return 0 if ok else 1
    if args.calibrate_copy:
        _calibration_copy()
    m = n = k = 4096
    head = gemm_workload("fused_addmm_bias_gelu_erf_fp32_4096", m, n, k, torch.float32,
                         steps=args.steps, warmup=args.warmup)
    traffic_key = (f"fp32 {m}x{n}x{k} B=W^T tile={head['tile'][0]}x{head['tile'][1]}x"
                   f"{head['tile'][2]} waves={head['tile'][3]}")
    traffic = _measured_traffic(traffic_key)
    result = {
        "metric": "fused linear+bias+GELU TFLOP/s (fp32 M=N=K=4096, B=W^T, erf GELU)",
        "value": round(head["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0, K**-0.5) operands, U(-0.1,0.1) bias)",
        "config": {"workload": "fused addmm+bias+GELU(erf), fp32, M=N=K=4096, A row-major, B=W^T strided",
                   "M": m, "N": n, "K": k, "tile": head["tile"]},
        "roofline": {
            "bound": "mfma",
            "achieved": round(head["kernel_tflops"], 3),
            "peak": PEAK_TFLOPS[torch.float32],
            "unit": "TFLOP/s",
            "frac": round(head["kernel_tflops"] / PEAK_TFLOPS[torch.float32], 4),
            "traffic": traffic,
            "traffic_source": ("committed rocprofv3 FETCH_SIZE/WRITE_SIZE runs of this kernel tile "
                               "(profiles/hbm_traffic.json), not measured in this run") if traffic is not None
                              else f"no committed counter run for {traffic_key}",
            "kernel_us_avg": round(head["kernel_ms_avg"] * 1e3, 2),
        },
        "gate": head["gate"],
    }
    from forgeml_amd.measurement import environment

    result["environment"] = environment(torch.device("cuda", 0))
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(m, n, k)
    if not args.no_extra:
        extra = [gemm_workload(name, *EXTRA_GEMMS[name], steps=10, warmup=3, **EXTRA_KW[name])
                 for name in EXTRA_GEMMS]
        from forgeml_amd.neural import TransformerBlock, make_mlp

        def mlp():
            torch.manual_seed(0)
            return make_mlp(512, 2048, 512).eval()

        def mlp_input():
            torch.manual_seed(1)
            return torch.randn(64, 512)

        def block():
            torch.manual_seed(0)
            return TransformerBlock(768, 12, 3072).eval()

        def block_input():
            torch.manual_seed(1)
            return torch.randn(8, 512, 768)

        extra.append(compiled_workload("compiled_mlp_64x512x2048_fp32", mlp, mlp_input, steps=50, warmup=5))
        extra.append(compiled_workload("compiled_transformer_block_8x512x768_fp32", block, block_input,
                                       steps=10, warmup=3))
        result["skinny"] = [skinny_workload(*shape) for shape in SKINNY_SHAPES]
        result["extra"] = extra
    gates = [result["gate"]] + [r["gate"] for r in result.get("extra", []) + result.get("skinny", [])]
    result["all_gates_passed"] = all(g["passed"] for g in gates)
    print(json.dumps(result), flush=True)
    return 0 if result["all_gates_passed"] else 1


if __name__ == "__main__":
    sys.exit(main())
