"""Timing contract and the autotuner's correctness gate (src/forgeml/measurement.py,
src/forgeml/autotune.py), exercised with fake kernels on the CPU
(the reference's strategy, tests/test_measurement.py:58-149)."""

import json

import pytest
import torch

import forgeml_amd
from forgeml_amd import autotune, kernels, measurement


def test_summary_percentile():
    r = measurement.summarize([4.0, 1.0, 3.0, 2.0])
    assert r["samples_ms"] == [4.0, 1.0, 3.0, 2.0]
    assert r["median_ms"] == 2.5 and r["p95_ms"] == pytest.approx(3.85)
    assert (r["count"], r["min_ms"], r["max_ms"]) == (4, 1.0, 4.0)


@pytest.mark.parametrize("samples", [[], [float("nan")], [float("inf")], [0.0], [-1.0]])
def test_invalid_latencies_rejected(samples):
    with pytest.raises(ValueError):
        measurement.summarize(samples)


def test_rotation_and_warmup_exclusion(monkeypatch):
    calls = []
    ticks = iter(range(0, 100_000_000, 1_000_000))
    monkeypatch.setattr(measurement.time, "perf_counter_ns", lambda: next(ticks))
    report = measurement.measure_variants(
        {"a": lambda: calls.append("a"), "b": lambda: calls.append("b")}, device="cpu", warmup=1, repeats=3
    )
    assert calls == ["a", "b", "a", "b", "b", "a", "a", "b"]
    assert report["a"]["samples_ms"] == [1.0, 1.0, 1.0]


def test_gate_rejects_wrong_and_nonfinite():
    expected = torch.ones(4)
    assert measurement.check_output(expected.clone(), expected)["max_absolute_error"] == 0.0
    with pytest.raises(AssertionError):
        measurement.check_output(torch.zeros(4), expected)
    with pytest.raises(AssertionError, match="non-finite"):
        measurement.check_output(torch.full((4,), float("nan")), expected)


def test_report_roundtrip_and_no_nan(tmp_path):
    path = tmp_path / "r" / "report.json"
    measurement.write_report({"samples": [1.0, 2.0]}, path)
    assert json.loads(path.read_text()) == {"samples": [1.0, 2.0]}
    with pytest.raises(ValueError):
        measurement.write_report({"bad": float("nan")}, path)
    assert json.loads(path.read_text()) == {"samples": [1.0, 2.0]}


def _compiled(model, x, optimize=True):
    c = forgeml_amd.compile(model, (x,), optimize=optimize)
    c.kernel_plan = {n.name: "hip" for n in c.graph.nodes}
    return c


def test_autotune_on_cpu_reports_nothing():
    model = torch.nn.Sequential(torch.nn.Linear(4, 8), torch.nn.GELU()).eval()
    x = torch.randn(2, 4)
    c = forgeml_amd.compile(model, (x,))
    assert c.autotune(x, warmup=0, repeats=2)["nodes"] == {}
    assert c.kernel_configs == {}


def test_autotune_rejects_incorrect_candidate(monkeypatch):
    model = torch.nn.Sequential(torch.nn.Linear(4, 8), torch.nn.GELU()).eval()
    x = torch.randn(2, 4)
    c = _compiled(model, x)
    wrong = kernels.candidates(torch.float32)[0]

    def fake(a, b, bias=None, *, activation="none", approximate="none", config=None, out=None):
        value = a @ b + bias
        if activation == "gelu":
            value = torch.nn.functional.gelu(value, approximate=approximate)
        return value + 10 if config == wrong else value

    monkeypatch.setattr(kernels, "matmul", fake)
    monkeypatch.setattr(autotune, "measure_variants",
                        lambda variants, **kw: {n: measurement.summarize([2.0, 2.0]) for n in variants})
    report = autotune.tune_graph(c, (x,), warmup=0, repeats=2)
    node = next(iter(report["nodes"].values()))
    assert "candidate_0" in node["rejected"] and "candidate_0" not in node["candidates"]
    assert node["winner"] == "candidate_1"
    assert list(c.kernel_configs.values()) == [kernels.candidates(torch.float32)[1]]


def test_autotune_launch_failure_is_a_rejection(monkeypatch):
    model = torch.nn.Linear(4, 8, bias=False).eval()
    x = torch.randn(2, 4)
    c = _compiled(model, x, optimize=False)
    failing = kernels.candidates(torch.float32)[0]
    seen_bias = []

    def fake(a, b, bias=None, *, activation="none", approximate="none", config=None, out=None):
        seen_bias.append(bias is not None)
        if config == failing:
            raise RuntimeError("simulated launch failure")
        value = a @ b
        return value if out is None else out.copy_(value)

    monkeypatch.setattr(kernels, "matmul", fake)
    monkeypatch.setattr(autotune, "measure_variants",
                        lambda variants, **kw: {n: measurement.summarize([1.0, 1.0]) for n in variants})
    report = autotune.tune_graph(c, (x,), warmup=0, repeats=2)
    node = next(iter(report["nodes"].values()))
    assert "candidate_0" in node["rejected"] and node["winner"] in node["candidates"]
    # one warm call through the executor, then one launch per candidate
    assert seen_bias == [False] * (len(kernels.candidates(torch.float32)) + 1)


def test_autotune_all_candidates_wrong_raises(monkeypatch):
    model = torch.nn.Linear(4, 8).eval()
    x = torch.randn(2, 4)
    c = _compiled(model, x, optimize=False)
    monkeypatch.setattr(kernels, "matmul",
                        lambda a, b, bias=None, **kw: (a @ b + bias + 1) if kw.get("out") is None else kw["out"].copy_(a @ b + bias))
    with pytest.raises(RuntimeError, match="no numerically valid"):
        autotune.tune_graph(c, (x,), warmup=0, repeats=2)
