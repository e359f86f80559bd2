"""Compiled graphs, memory plans, pass records and cost analysis must match
the reference's own published captures (tests/golden/forgeml_captures.json,
extracted from ForgeML's benchmarks/results/*.json)."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

import forgeml_amd
from forgeml_amd.neural import ResidualMLP, TransformerBlock

CAPTURES = json.loads((Path(__file__).resolve().parent / "golden" / "forgeml_captures.json").read_text())


def _model(w):
    if w["suite"] == "transformer_block":
        batch, seq, hidden = w["input_shape"]
        heads, ffn = 8, 256  # README.md:498: hidden 128, 8 heads, FFN 256
        return TransformerBlock(hidden, heads, ffn).eval(), torch.randn(batch, seq, hidden)
    if w["residual"]:
        return ResidualMLP(w["width"], w["hidden"]).eval(), torch.randn(w["batch"], w["width"])
    model = torch.nn.Sequential(
        torch.nn.Linear(w["width"], w["hidden"]), torch.nn.GELU(approximate="tanh"),
        torch.nn.Linear(w["hidden"], w["output"]),
    ).eval()
    return model, torch.randn(w["batch"], w["width"])


@pytest.mark.parametrize("variant", ["unoptimized", "optimized"])
@pytest.mark.parametrize("w", CAPTURES["workloads"], ids=lambda w: w["name"])
def test_compile_reproduces_reference_capture(w, variant):
    model, x = _model(w)
    compiled = forgeml_amd.compile(model, (x,), optimize=variant == "optimized")
    got = json.loads(json.dumps(compiled.explain()))
    ref = w[variant]
    for key in ("graph", "memory_plan", "passes", "kernel_plan", "optimized_nodes", "original_nodes",
                "optimization_delta"):
        assert got[key] == ref[key], key
    for part in ("analysis", "original_analysis"):
        for key, value in ref[part].items():
            assert got[part][key] == value, f"{part}.{key}"
    torch.testing.assert_close(compiled(x), model(x))
