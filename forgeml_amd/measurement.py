"""Latency measurement, the correctness gate and run provenance.

The rules are ForgeML's (src/forgeml/measurement.py:19-147), because the
autotuner and the benchmark reports are compared against the reference's:

* every raw sample is kept; a summary reports the median, the p95 by linear
  interpolation at (n - 1) q, the minimum and the maximum, under the keys
  ``samples_ms``, ``count``, ``median_ms``, ``p95_ms``, ``min_ms``,
  ``max_ms`` (measurement.py:19-41);
* variants are timed in rounds after their warmups, each round starting one
  variant later than the previous one, each sample bracketed by device
  synchronisation on the host wall clock (measurement.py:52-78);
* the gate refuses non-finite values and then applies the dtype's
  rtol/atol before a variant may be timed (measurement.py:81-107).

How it is built here: a sample schedule is generated up front (so the
rotation is a value that can be inspected), the clock is a parameter, and
the gate reports the worst element.  ``event_times`` is the GPU-side timer
(HIP events on the launch stream) that the benchmark uses for kernel time.
"""

from __future__ import annotations

import json
import math
import os
import platform
import re
import subprocess
import time
from collections.abc import Callable, Iterator, Mapping, Sequence
from dataclasses import dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import numpy as np
import torch

# The gate's (rtol, atol) per dtype (src/forgeml/measurement.py:81-91).
_TOLERANCES = {
    torch.float16: (1e-2, 1e-2),
    torch.bfloat16: (5e-2, 5e-2),
    torch.float32: (1e-4, 1e-4),
    torch.float64: (1e-7, 1e-8),
}


def percentile(samples: Sequence[float], q: float) -> float:
    """The q-quantile of ``samples`` by linear interpolation at (n - 1) q."""
    if len(samples) == 0 or not 0.0 <= q <= 1.0:
        raise ValueError("percentile requires samples and q in [0, 1]")
    data = np.asarray(samples, dtype=np.float64)
    if not np.isfinite(data).all():
        raise ValueError("samples must be finite")
    return float(np.quantile(data, q, method="linear"))


@dataclass(frozen=True)
class LatencySummary:
    samples_ms: tuple[float, ...]

    def __post_init__(self):
        if not self.samples_ms or not all(math.isfinite(s) and s > 0 for s in self.samples_ms):
            raise ValueError("latencies must be finite and positive")

    def as_dict(self) -> dict[str, Any]:
        ordered = sorted(self.samples_ms)
        n = len(ordered)
        middle = ordered[n // 2] if n % 2 else 0.5 * (ordered[n // 2 - 1] + ordered[n // 2])
        return {
            "samples_ms": list(self.samples_ms),
            "count": n,
            "median_ms": middle,
            "p95_ms": percentile(ordered, 0.95),
            "min_ms": ordered[0],
            "max_ms": ordered[-1],
        }


def summarize(samples_ms: Sequence[float]) -> dict[str, Any]:
    """Summary of raw latencies in milliseconds (finite and positive)."""
    return LatencySummary(tuple(float(s) for s in samples_ms)).as_dict()


def synchronize(device: torch.device | str) -> None:
    kind = torch.device(device).type
    if kind == "cuda":
        torch.cuda.synchronize(device)
    elif kind != "cpu":
        raise ValueError("measurement supports CPU or GPU (cuda) devices only")


def rotation_schedule(names: Sequence[str], repeats: int) -> Iterator[str]:
    """Sample order: ``repeats`` rounds over ``names``, round r starting at name r mod n."""
    n = len(names)
    for r in range(repeats):
        for j in range(n):
            yield names[(r + j) % n]


@torch.inference_mode()
def measure_variants(
    variants: Mapping[str, Callable[[], Any]],
    *,
    device: torch.device | str,
    warmup: int = 5,
    repeats: int = 25,
    clock: Callable[[], int] = time.perf_counter_ns,
) -> dict[str, dict[str, Any]]:
    """Host wall-clock latency of each zero-argument callable, in rotating rounds.

    Each variant first runs ``warmup`` untimed calls; the timed calls follow
    ``rotation_schedule``.  ``clock`` returns nanoseconds.
    """
    if not variants or warmup < 0 or repeats < 2:
        raise ValueError("provide variants, warmup >= 0 and repeats >= 2")
    names = list(variants)
    for name in names:
        fn = variants[name]
        for _ in range(warmup):
            fn()
    synchronize(device)
    samples: dict[str, list[float]] = {name: [] for name in names}
    for name in rotation_schedule(names, repeats):
        fn = variants[name]
        synchronize(device)
        start = clock()
        result = fn()
        synchronize(device)
        samples[name].append((clock() - start) * 1e-6)
        del result
    return {name: summarize(values) for name, values in samples.items()}


def event_times(fn: Callable[[], Any], *, iters: int, warmup: int = 2,
                stream: torch.cuda.Stream | None = None) -> list[float]:
    """Milliseconds of each of ``iters`` back-to-back calls of ``fn``, from HIP
    events recorded on ``stream`` (default: the current stream), which must
    be the stream ``fn`` launches on.  Host launch gaps are excluded as long
    as the queue stays ahead of the GPU."""
    stream = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    stream.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
    marks[0].record(stream)
    for i in range(iters):
        fn()
        marks[i + 1].record(stream)
    stream.synchronize()
    return [marks[i].elapsed_time(marks[i + 1]) for i in range(iters)]


def tolerances(dtype: torch.dtype) -> tuple[float, float]:
    """The gate's (rtol, atol) for outputs of ``dtype``; exact for other dtypes."""
    return _TOLERANCES.get(dtype, (0.0, 0.0))


@torch.inference_mode()
def check_output(actual: torch.Tensor, expected: torch.Tensor, *, rtol: float | None = None,
                 atol: float | None = None) -> dict[str, float | bool]:
    """The correctness gate: both tensors finite, same shape and dtype, and
    |actual - expected| <= atol + rtol |expected| everywhere (the dtype's
    tolerances unless given).  Raises AssertionError otherwise; returns the
    tolerances used and the largest absolute error."""
    if not isinstance(actual, torch.Tensor) or not isinstance(expected, torch.Tensor):
        raise TypeError("benchmark outputs must be tensors")
    default_rtol, default_atol = tolerances(expected.dtype)
    rtol = default_rtol if rtol is None else rtol
    atol = default_atol if atol is None else atol
    got = actual.detach().to(expected.device, torch.float64)
    want = expected.detach().to(torch.float64)
    if not (torch.isfinite(got).all() and torch.isfinite(want).all()):
        raise AssertionError("non-finite output cannot pass a benchmark correctness gate")
    if actual.shape != expected.shape or actual.dtype != expected.dtype:
        raise AssertionError(f"output {tuple(actual.shape)} {actual.dtype} does not match the expected "
                             f"{tuple(expected.shape)} {expected.dtype}")
    err = (got - want).abs()
    excess = err - (atol + rtol * want.abs())
    if excess.numel() and bool((excess > 0).any()):
        worst = int(excess.argmax())
        raise AssertionError(
            f"{int((excess > 0).sum())} of {excess.numel()} elements exceed rtol={rtol} atol={atol}; worst at "
            f"flat index {worst}: got {got.flatten()[worst].item()!r}, expected {want.flatten()[worst].item()!r}")
    return {
        "passed": True,
        "rtol": rtol,
        "atol": atol,
        "max_absolute_error": float(err.max()) if err.numel() else 0.0,
    }


# -- provenance ------------------------------------------------------------------

def cpu_description() -> dict[str, Any]:
    """CPU model and core counts of this host, read from /proc/cpuinfo."""
    info: dict[str, Any] = {"cpu_model": platform.processor() or None, "logical_cpus": os.cpu_count()}
    try:
        text = Path("/proc/cpuinfo").read_text()
    except OSError:
        return info
    cores = set()
    for block in text.split("\n\n"):
        fields = dict(
            (m.group(1).strip(), m.group(2).strip())
            for m in re.finditer(r"^([^:\n]+):(.*)$", block, flags=re.M)
        )
        if "model name" in fields:
            info["cpu_model"] = fields["model name"]
        if "core id" in fields:
            cores.add((fields.get("physical id", "0"), fields["core id"]))
    if cores:
        info["physical_cores"] = len(cores)
    try:
        info["usable_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    return info


def _git_state(root: Path) -> dict[str, Any]:
    def git(*args: str) -> str:
        return subprocess.check_output(["git", *args], cwd=root, text=True, stderr=subprocess.DEVNULL).strip()

    try:
        return {"git_commit": git("rev-parse", "HEAD"), "git_dirty": bool(git("status", "--porcelain"))}
    except (OSError, subprocess.CalledProcessError):
        return {"git_commit": None, "git_dirty": None}


def environment(device: torch.device | str) -> dict[str, Any]:
    """Provenance of a measurement: time, host, CPU, library versions, commit, GPU."""
    device = torch.device(device)
    synchronize(device)
    meta: dict[str, Any] = {
        "captured_at_utc": datetime.now(timezone.utc).isoformat(),
        "python": platform.python_version(),
        "platform": platform.platform(),
        "machine": platform.machine(),
        "torch": torch.__version__,
        "torch_threads": torch.get_num_threads(),
        "hip_runtime": torch.version.hip,
        "device": str(device),
        "timing": "synchronized_host_wall_clock",
        "percentile_method": "linear_interpolation_at_(n-1)*q",
    }
    meta.update(cpu_description())
    meta.update(_git_state(Path(__file__).resolve().parents[1]))
    try:  # the kernel library's own record of what it was built from
        built = json.loads((Path(__file__).resolve().parent / "_build_info.json").read_text())
        meta["library_build"] = {k: built.get(k) for k in ("git_commit", "git_dirty", "sources_sha256")}
        if meta.get("git_commit") is None:
            meta["git_commit"] = built.get("git_commit")
    except (OSError, ValueError):
        meta["library_build"] = None
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
    """Write ``report`` as JSON, replacing ``path`` atomically; NaN and inf
    are refused before anything is written."""
    text = json.dumps(report, indent=2, sort_keys=True, allow_nan=False) + "\n"
    dest = Path(path)
    dest.parent.mkdir(parents=True, exist_ok=True)
    staging = dest.with_name(f".{dest.name}.{os.getpid()}.partial")
    try:
        staging.write_text(text, encoding="utf-8")
        os.replace(staging, dest)
    finally:
        staging.unlink(missing_ok=True)
