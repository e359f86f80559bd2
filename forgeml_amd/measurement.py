"""Timing and correctness-gate contract shared by the autotuner and benchmarks.

Keeps ForgeML's measurement rules (src/forgeml/measurement.py):

* raw samples are kept; median, p95 (linear interpolation at (n-1)*q), min
  and max are derived from them (measurement.py:19-41);
* ``measure_variants`` runs warmups, then rotates the variant order every
  repeat and brackets each sample with device synchronisation
  (measurement.py:52-78);
* ``check_output`` refuses non-finite values and applies per-dtype
  tolerances before any timing counts (measurement.py:81-107).

GPU-side timing of single kernels uses HIP events on the launch stream
(``time_on_stream``), which excludes host launch overhead.
"""

from __future__ import annotations

import json
import math
import os
import platform
import statistics
import subprocess
import tempfile
import time
from collections.abc import Callable, Mapping, Sequence
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch


def percentile(samples: Sequence[float], q: float) -> float:
    if not samples or not 0 <= q <= 1:
        raise ValueError("percentile requires samples and q in [0, 1]")
    values = sorted(samples)
    if not all(math.isfinite(v) for v in values):
        raise ValueError("samples must be finite")
    pos = (len(values) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    return values[lo] + (values[hi] - values[lo]) * (pos - lo)


def summarize(samples_ms: Sequence[float]) -> dict[str, Any]:
    if not samples_ms or any(not math.isfinite(v) or v <= 0 for v in samples_ms):
        raise ValueError("latencies must be finite and positive")
    return {
        "samples_ms": list(samples_ms),
        "count": len(samples_ms),
        "median_ms": statistics.median(samples_ms),
        "p95_ms": percentile(samples_ms, 0.95),
        "min_ms": min(samples_ms),
        "max_ms": max(samples_ms),
    }


def synchronize(device: torch.device | str) -> None:
    device = torch.device(device)
    if device.type == "cuda":
        torch.cuda.synchronize(device)
    elif device.type != "cpu":
        raise ValueError("measurement supports CPU or GPU (cuda) devices only")


@torch.inference_mode()
def measure_variants(
    variants: Mapping[str, Callable[[], Any]],
    *,
    device: torch.device | str,
    warmup: int = 5,
    repeats: int = 25,
) -> dict[str, dict[str, Any]]:
    if not variants or warmup < 0 or repeats < 2:
        raise ValueError("provide variants, warmup >= 0 and repeats >= 2")
    names = list(variants)
    for name in names:
        for _ in range(warmup):
            variants[name]()
    synchronize(device)
    samples: dict[str, list[float]] = {name: [] for name in names}
    for rep in range(repeats):
        shift = rep % len(names)
        for name in names[shift:] + names[:shift]:
            synchronize(device)
            t0 = time.perf_counter_ns()
            result = variants[name]()
            synchronize(device)
            samples[name].append((time.perf_counter_ns() - t0) / 1_000_000)
            del result
    return {name: summarize(v) for name, v in samples.items()}


def time_on_stream(fn: Callable[[], Any], *, iters: int, warmup: int = 2) -> list[float]:
    """Per-call milliseconds of ``fn`` measured with events on the current stream.

    ``fn`` must launch its work on ``torch.cuda.current_stream()``; one event
    pair brackets each call so launch gaps between calls are excluded only
    when the queue stays full.
    """
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    stream.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for start, end in events:
        start.record(stream)
        fn()
        end.record(stream)
    stream.synchronize()
    return [s.elapsed_time(e) for s, e in events]


def tolerances(dtype: torch.dtype) -> tuple[float, float]:
    if dtype == torch.float16:
        return 1e-2, 1e-2
    if dtype == torch.bfloat16:
        return 5e-2, 5e-2
    if dtype == torch.float32:
        return 1e-4, 1e-4
    if dtype == torch.float64:
        return 1e-7, 1e-8
    return 0.0, 0.0


@torch.inference_mode()
def check_output(actual: torch.Tensor, expected: torch.Tensor, *, rtol: float | None = None,
                 atol: float | None = None) -> dict[str, float | bool]:
    """Correctness gate: finite values and allclose under the dtype's tolerance."""
    if not isinstance(actual, torch.Tensor) or not isinstance(expected, torch.Tensor):
        raise TypeError("benchmark outputs must be tensors")
    d_rtol, d_atol = tolerances(expected.dtype)
    rtol = d_rtol if rtol is None else rtol
    atol = d_atol if atol is None else atol
    if not torch.isfinite(actual).all() or not torch.isfinite(expected).all():
        raise AssertionError("non-finite output cannot pass a benchmark correctness gate")
    torch.testing.assert_close(actual, expected, rtol=rtol, atol=atol)
    delta = (actual.to(torch.float64) - expected.to(torch.float64)).abs()
    return {
        "passed": True,
        "rtol": rtol,
        "atol": atol,
        "max_absolute_error": delta.max().item() if delta.numel() else 0.0,
    }


def environment(device: torch.device | str) -> dict[str, Any]:
    device = torch.device(device)
    synchronize(device)
    meta: dict[str, Any] = {
        "captured_at_utc": datetime.now(timezone.utc).isoformat(),
        "python": platform.python_version(),
        "platform": platform.platform(),
        "machine": platform.machine(),
        "processor": platform.processor(),
        "torch": torch.__version__,
        "torch_threads": torch.get_num_threads(),
        "cpu_count": os.cpu_count(),
        "device": str(device),
        "hip_runtime": torch.version.hip,
        "timing": "synchronized_host_wall_clock",
        "percentile_method": "linear_interpolation_at_(n-1)*q",
    }
    root = Path(__file__).resolve().parents[1]
    try:
        meta["git_commit"] = subprocess.check_output(
            ["git", "rev-parse", "HEAD"], cwd=root, text=True, stderr=subprocess.DEVNULL
        ).strip()
        meta["git_dirty"] = bool(
            subprocess.check_output(["git", "status", "--porcelain"], cwd=root, text=True,
                                    stderr=subprocess.DEVNULL).strip()
        )
    except (OSError, subprocess.CalledProcessError):
        meta["git_commit"] = None
        meta["git_dirty"] = None
    if device.type == "cuda":
        props = torch.cuda.get_device_properties(device)
        meta.update(
            gpu_name=props.name,
            gpu_arch=getattr(props, "gcnArchName", None),
            gpu_memory_bytes=props.total_memory,
            gpu_compute_units=props.multi_processor_count,
            gpu_device_count=torch.cuda.device_count(),
        )
    return meta


def write_report(report: dict[str, Any], path: str | Path) -> None:
    """Atomically write ``report`` as JSON; NaN/inf are refused."""
    dest = Path(path)
    dest.parent.mkdir(parents=True, exist_ok=True)
    text = json.dumps(report, indent=2, sort_keys=True, allow_nan=False) + "\n"
    tmp = None
    try:
        with tempfile.NamedTemporaryFile("w", encoding="utf-8", dir=dest.parent, delete=False) as fh:
            tmp = Path(fh.name)
            fh.write(text)
        os.replace(tmp, dest)
    finally:
        if tmp is not None and tmp.exists():
            tmp.unlink()
