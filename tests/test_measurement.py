"""The measurement rules and the autotuner's gate-then-time contract, on the CPU.

Percentiles are checked against closed forms; the timing loop runs with an
injected clock and recording callables; the autotuner runs on a compiled
model whose GEMM nodes are planned for the GPU kernel, with
``kernels.matmul`` replaced by a fake whose behaviour per tile is scripted
(src/forgeml/autotune.py:16-103 is the contract).
"""

from __future__ import annotations

import json
import math

import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

import forgeml_amd
from forgeml_amd import autotune, kernels, measurement

# -- summaries -------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 2, 5, 20, 101])
@pytest.mark.parametrize("q", [0.0, 0.25, 0.5, 0.95, 1.0])
def test_percentile_of_an_arithmetic_sequence(n, q):
    # For the values 1..n the linear interpolation at (n-1) q is 1 + (n-1) q exactly.
    samples = [float(v) for v in range(n, 0, -1)]  # order must not matter
    assert measurement.percentile(samples, q) == pytest.approx(1 + (n - 1) * q)


@settings(max_examples=60, derandomize=True, deadline=None)
@given(st.lists(st.floats(0.001, 1e3), min_size=1, max_size=40), st.floats(0, 1))
def test_percentile_is_bounded_and_monotone(samples, q):
    p = measurement.percentile(samples, q)
    assert min(samples) <= p <= max(samples)
    assert measurement.percentile(samples, min(1.0, q + 0.1)) >= p


@pytest.mark.parametrize("bad", [[], [1.0, math.nan]])
def test_percentile_rejects_bad_input(bad):
    with pytest.raises(ValueError):
        measurement.percentile(bad, 0.5)
    with pytest.raises(ValueError):
        measurement.percentile([1.0], 1.5)


def test_summary_fields():
    s = measurement.summarize([5.0, 1.0, 2.0, 4.0, 3.0])
    assert s["samples_ms"] == [5.0, 1.0, 2.0, 4.0, 3.0]  # raw order kept
    assert (s["count"], s["median_ms"], s["min_ms"], s["max_ms"]) == (5, 3.0, 1.0, 5.0)
    assert s["p95_ms"] == pytest.approx(1 + 4 * 0.95)
    assert measurement.summarize([2.0, 1.0])["median_ms"] == 1.5


@pytest.mark.parametrize("samples", [[], [math.inf], [0.0], [-2.0], [1.0, math.nan]])
def test_summary_rejects_non_latencies(samples):
    with pytest.raises(ValueError):
        measurement.summarize(samples)


# -- the timing loop ---------------------------------------------------------------


def test_rotation_schedule_starts_each_round_one_later():
    order = list(measurement.rotation_schedule(["x", "y", "z"], 4))
    assert order == ["x", "y", "z", "y", "z", "x", "z", "x", "y", "x", "y", "z"]


def test_warmups_untimed_and_samples_from_the_clock():
    calls = []
    now = [0]

    def clock():
        now[0] += 7_000  # each reading 7 us after the previous one
        return now[0]

    variants = {name: (lambda name=name: calls.append(name)) for name in ("p", "q")}
    report = measurement.measure_variants(variants, device="cpu", warmup=2, repeats=3, clock=clock)
    # two warmups each, then three rotating rounds
    assert calls == ["p", "p", "q", "q", "p", "q", "q", "p", "p", "q"]
    for name in variants:
        assert report[name]["samples_ms"] == pytest.approx([0.007] * 3)
    with pytest.raises(ValueError):
        measurement.measure_variants(variants, device="cpu", repeats=1)
    with pytest.raises(ValueError):
        measurement.measure_variants({}, device="cpu")


# -- the correctness gate ------------------------------------------------------------


def test_gate_tolerances_per_dtype():
    assert measurement.tolerances(torch.float32) == (1e-4, 1e-4)
    assert measurement.tolerances(torch.bfloat16) == (5e-2, 5e-2)
    assert measurement.tolerances(torch.float16) == (1e-2, 1e-2)
    assert measurement.tolerances(torch.int32) == (0.0, 0.0)


def test_gate_passes_within_and_fails_outside():
    want = torch.linspace(-2, 2, 9)
    inside = want + 0.9e-4 * (1 + want.abs())
    report = measurement.check_output(inside, want)
    assert report["passed"] and report["max_absolute_error"] > 0
    with pytest.raises(AssertionError, match="exceed"):
        measurement.check_output(want + 3e-4, want)
    # explicit tolerances override the dtype's
    measurement.check_output(want + 3e-4, want, atol=1e-3)


@pytest.mark.parametrize("poison", [math.nan, math.inf])
def test_gate_refuses_non_finite_on_either_side(poison):
    good = torch.ones(3)
    bad = torch.tensor([1.0, poison, 1.0])
    with pytest.raises(AssertionError, match="non-finite"):
        measurement.check_output(bad, good)
    with pytest.raises(AssertionError, match="non-finite"):
        measurement.check_output(good, bad)


def test_gate_refuses_shape_or_dtype_change():
    with pytest.raises(AssertionError):
        measurement.check_output(torch.ones(2, 3), torch.ones(3, 2))
    with pytest.raises(AssertionError):
        measurement.check_output(torch.ones(3, dtype=torch.float64), torch.ones(3))
    with pytest.raises(TypeError):
        measurement.check_output([1.0], torch.ones(1))


# -- reports and provenance ------------------------------------------------------------


def test_report_is_replaced_whole_and_refuses_nan(tmp_path):
    dest = tmp_path / "deep" / "run.json"
    measurement.write_report({"b": 2, "a": [1.5]}, dest)
    assert json.loads(dest.read_text()) == {"a": [1.5], "b": 2}
    with pytest.raises(ValueError):
        measurement.write_report({"a": math.inf}, dest)
    assert json.loads(dest.read_text()) == {"a": [1.5], "b": 2}
    assert [p.name for p in dest.parent.iterdir()] == ["run.json"]  # no partial file left


def test_environment_names_host_and_versions():
    env = measurement.environment("cpu")
    for key in ("captured_at_utc", "torch", "torch_threads", "logical_cpus", "cpu_model", "git_commit"):
        assert key in env
    assert env["logical_cpus"] >= 1
    assert env.get("physical_cores", 1) >= 1


# -- the autotuner with scripted fake kernels -------------------------------------------


class _ScriptedKernel:
    """Stands in for kernels.matmul: correct, except for tiles told to be wrong or to fail."""

    def __init__(self, wrong=(), failing=()):
        self.wrong, self.failing = set(wrong), set(failing)
        self.calls = []

    def __call__(self, a, b, bias=None, *, activation="none", approximate="none", config=None, out=None,
                 residual=None):
        self.calls.append(config)
        if config in self.failing:
            raise RuntimeError("scripted launch failure")
        value = a @ b if bias is None else torch.addmm(bias, a, b)
        if activation == "gelu":
            value = torch.nn.functional.gelu(value, approximate=approximate)
        if config in self.wrong:
            value = value * 1.01
        return value if out is None else out.copy_(value)


def _hip_planned(model, x, optimize=True):
    compiled = forgeml_amd.compile(model, (x,), optimize=optimize)
    compiled.kernel_plan = {n.name: "hip" for n in compiled.graph.nodes}
    return compiled


def _flat_timings(median_of):
    def fake(variants, **_):
        return {name: measurement.summarize([median_of(name)] * 2) for name in variants}
    return fake


TILES = kernels.candidates(torch.float32)


def test_wrong_tile_is_rejected_before_timing(monkeypatch):
    model = torch.nn.Sequential(torch.nn.Linear(6, 5), torch.nn.GELU(approximate="tanh")).eval()
    x = torch.randn(3, 6)
    compiled = _hip_planned(model, x)
    fake = _ScriptedKernel(wrong={TILES[0]})
    timed = []
    monkeypatch.setattr(kernels, "matmul", fake)
    monkeypatch.setattr(autotune, "measure_variants",
                        lambda variants, **kw: timed.extend(variants) or _flat_timings(lambda n: 1.0)(variants))
    report = autotune.tune_graph(compiled, (x,), warmup=0, repeats=2)
    (name, node), = report["nodes"].items()
    assert "candidate_0" in node["rejected"] and "candidate_0" not in timed
    assert node["winner"] == "candidate_1" and node["activation"] == "gelu" and node["approximate"] == "tanh"
    assert compiled.kernel_configs == {name: TILES[1]}
    assert node["input_shapes"][0] == [3, 6] and node["dtype"] == "torch.float32"
    assert all(c["correctness"]["passed"] for c in node["candidates"].values())


def test_lowest_median_wins_and_ties_keep_table_order(monkeypatch):
    model = torch.nn.Linear(4, 4).eval()
    x = torch.randn(2, 4)
    compiled = _hip_planned(model, x, optimize=False)
    monkeypatch.setattr(kernels, "matmul", _ScriptedKernel())
    last = f"candidate_{len(TILES) - 1}"
    monkeypatch.setattr(autotune, "measure_variants", _flat_timings(lambda n: 0.5 if n == last else 2.0))
    assert next(iter(autotune.tune_graph(compiled, (x,), repeats=2)["nodes"].values()))["winner"] == last
    monkeypatch.setattr(autotune, "measure_variants", _flat_timings(lambda n: 1.0))
    assert next(iter(autotune.tune_graph(compiled, (x,), repeats=2)["nodes"].values()))["winner"] == "candidate_0"


def test_launch_failure_rejects_and_each_candidate_launches_once(monkeypatch):
    model = torch.nn.Linear(4, 8, bias=False).eval()
    x = torch.randn(2, 4)
    compiled = _hip_planned(model, x, optimize=False)
    fake = _ScriptedKernel(failing={TILES[-1]})
    monkeypatch.setattr(kernels, "matmul", fake)
    monkeypatch.setattr(autotune, "measure_variants", _flat_timings(lambda n: 1.0))
    report = autotune.tune_graph(compiled, (x,), warmup=0, repeats=2)
    node = next(iter(report["nodes"].values()))
    assert "scripted launch failure" in node["rejected"][f"candidate_{len(TILES) - 1}"]
    # one call through the compiled model, then one gate launch per candidate
    assert len(fake.calls) == 1 + len(TILES)
    assert report["scope"] == "this_compiled_model_instance_only" and report["repeats"] == 2


def test_no_valid_candidate_raises(monkeypatch):
    model = torch.nn.Linear(4, 8).eval()
    x = torch.randn(2, 4)
    compiled = _hip_planned(model, x, optimize=False)
    fake = _ScriptedKernel(wrong=set(TILES))
    monkeypatch.setattr(kernels, "matmul", lambda *a, **kw: fake(*a, **kw) if kw.get("out") is None
                        else _ScriptedKernel()(*a, **kw))
    with pytest.raises(RuntimeError, match="no numerically valid"):
        autotune.tune_graph(compiled, (x,), warmup=0, repeats=2)


def test_cpu_plan_tunes_nothing():
    model = torch.nn.Sequential(torch.nn.Linear(4, 8), torch.nn.GELU()).eval()
    x = torch.randn(2, 4)
    compiled = forgeml_amd.compile(model, (x,))
    assert compiled.autotune(x, warmup=0, repeats=2)["nodes"] == {}
    assert compiled.kernel_configs == {}
    with pytest.raises(ValueError):
        compiled.autotune(x, repeats=1)
