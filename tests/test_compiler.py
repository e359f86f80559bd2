"""Executor behaviour (src/forgeml/compiler.py) on the CPU, including the GPU
dispatch path driven through a fake kernel (the reference's strategy,
tests/test_compiler.py:180-214)."""

import json

import pytest
import torch
from torch import nn

import forgeml_amd
from forgeml_amd import kernels
from forgeml_amd.frontend import from_torch
from forgeml_amd.ir import GraphBuilder, GraphError, TensorSpec


def make_mlp():
    torch.manual_seed(0)
    return nn.Sequential(nn.Linear(8, 16), nn.GELU(approximate="tanh"), nn.Linear(16, 4)).eval()


def spec(*shape):
    return TensorSpec(tuple(shape), torch.float32, "cpu")


def test_mlp_parity_and_fusion():
    m = make_mlp()
    x = torch.randn(4, 8)
    c = forgeml_amd.compile(m, (x,))
    assert [n.op for n in c.graph.nodes] == ["fused_linear_gelu", "linear"]
    torch.testing.assert_close(c(x), m(x))


def test_backend_rejection_and_hip_requires_gpu():
    with pytest.raises(GraphError, match="backend"):
        forgeml_amd.compile(make_mlp(), (torch.randn(4, 8),), backend="triton")
    if not kernels.available():
        with pytest.raises(GraphError, match="hip"):
            forgeml_amd.compile(make_mlp(), (torch.randn(4, 8),), backend="hip")
        c = forgeml_amd.compile(make_mlp(), (torch.randn(4, 8),), backend="auto")
        assert set(c.kernel_plan.values()) == {"torch"}


def test_outputs_independent_across_calls():
    m = make_mlp()
    x = torch.randn(4, 8)
    c = forgeml_amd.compile(m, (x,))
    out1 = c(x)
    keep = out1.clone()
    out2 = c(x + 1.0)
    torch.testing.assert_close(out1, keep)
    assert out1.data_ptr() != out2.data_ptr()


def test_explain_is_json_and_consistent():
    c = forgeml_amd.compile(make_mlp(), (torch.randn(4, 8),))
    e = c.explain()
    assert "fused_linear_gelu" in json.dumps(e)
    assert e["optimized_nodes"] <= e["original_nodes"]
    assert e["memory_plan"]["planned_bytes"] <= e["memory_plan"]["naive_bytes"]
    assert e["optimization_delta"]["nodes"] == e["original_nodes"] - e["optimized_nodes"]


def test_internal_linear_writes_into_its_slot():
    m = nn.Sequential(nn.Linear(8, 16), nn.ReLU(), nn.Linear(16, 4, bias=False)).eval()
    x = torch.randn(4, 8)
    c = forgeml_amd.compile(m, (x,), optimize=False)
    first = c.graph.nodes[0].name
    assert first in c.memory_plan.allocations
    torch.testing.assert_close(c(x), m(x))


def test_view_and_output_alias_rules():
    b = GraphBuilder({"x": spec(4)})
    b.add("a", "relu", ("x",))
    b.add("b", "reshape", ("a",), shape=(2, 2))
    b.add("c", "relu", ("a",))
    b.constant("two", torch.full((4,), 2.0))
    b.add("d", "mul", ("c", "two"))
    b.add("out", "relu", ("d",))
    c = forgeml_amd.compile(b.finish(("b", "out")), optimize=False)
    assert c.memory_plan.allocations["d"].slot == c.memory_plan.allocations["a"].slot
    x = torch.randn(4)
    out_b, out_d = c(x)
    torch.testing.assert_close(out_b, torch.relu(x).reshape(2, 2))
    torch.testing.assert_close(out_d, torch.relu(torch.relu(x) * 2))


def test_constants_are_snapshotted():
    b = GraphBuilder({"x": spec(2)})
    b.constant("c", torch.ones(2))
    b.add("y", "add", ("x", "c"))
    g = b.finish(("y",))
    c = forgeml_amd.compile(g, optimize=False)
    g.constants["c"].fill_(99.0)
    torch.testing.assert_close(c(torch.zeros(2)), torch.ones(2))


def test_input_guards():
    c = forgeml_amd.compile(make_mlp(), (torch.randn(4, 8),))
    with pytest.raises(GraphError, match="shape"):
        c(torch.randn(5, 8))
    with pytest.raises(GraphError, match="dtype"):
        c(torch.randn(4, 8, dtype=torch.float64))
    with pytest.raises(GraphError, match="expected 1 inputs"):
        c()


def _fake_matmul(seen):
    def fake(a, b, bias=None, *, activation="none", approximate="none", config=None, out=None):
        seen.append((activation, approximate, bias is not None, out is not None))
        value = a @ b + (bias if bias is not None else 0)
        if activation == "gelu":
            value = torch.nn.functional.gelu(value, approximate=approximate)
        elif activation == "relu":
            value = torch.clamp_min(value, 0)
        return value if out is None else out.copy_(value)
    return fake


def test_gpu_dispatch_path_with_fake_kernel(monkeypatch):
    seen = []
    monkeypatch.setattr(kernels, "matmul", _fake_matmul(seen))
    model = make_mlp()
    x = torch.randn(4, 8)
    c = forgeml_amd.compile(model, (x,))
    c.kernel_plan = {n.name: "hip" for n in c.graph.nodes}  # rebuilds the step closures
    torch.testing.assert_close(c(x), model(x))
    # the internal fused node writes into its slot (out given), the output gets a fresh tensor
    assert seen == [("gelu", "tanh", True, True), ("none", "none", True, False)]


def _fake_matmul_residual(seen):
    def fake(a, b, bias=None, *, activation="none", approximate="none", config=None, out=None, residual=None):
        seen.append(residual is not None)
        value = a @ b + (bias if bias is not None else 0)
        if activation == "gelu":
            value = torch.nn.functional.gelu(value, approximate=approximate)
        if residual is not None:
            value = value + residual
        return value if out is None else out.copy_(value)
    return fake


def test_gemm_and_residual_add_fuse_on_hip_plan(monkeypatch):
    from forgeml_amd.neural import TransformerBlock

    torch.manual_seed(0)
    block = TransformerBlock(64, 4, 128).eval()
    x = torch.randn(2, 8, 64)
    c = forgeml_amd.compile(block, (x,))
    expected = c(x)
    assert c.fused_residuals == {}  # torch backend: the reference's two kernels
    seen = []
    monkeypatch.setattr(kernels, "matmul", _fake_matmul_residual(seen))
    c.kernel_plan = {n.name: ("hip" if n.op in kernels.GEMM_OPS else "torch") for n in c.graph.nodes}
    # out-proj -> reshape -> add(x, .) and FFN down -> reshape -> add(h, .), the
    # second writing the graph output.
    assert sorted((g, add) for g, (add, _v, _r, _c) in c.fused_residuals.items()) == [("down", "add_1"), ("o", "add")]
    torch.testing.assert_close(c(x), expected, rtol=1e-5, atol=1e-5)
    assert seen.count(True) == 2 and len(seen) == 4
    # Outputs stay fresh per call; calls are repeatable.
    first = c(x)
    second = c(x)
    assert first.data_ptr() != second.data_ptr()
    torch.testing.assert_close(first, second, rtol=0, atol=0)


def test_residual_fusion_needs_adjacency_and_exclusive_use():
    b = GraphBuilder({"x": spec(4, 8), "r": spec(4, 16)})
    w = b.constant("w", torch.randn(8, 16))
    b.add("y", "linear", ("x", w))
    b.add("z", "relu", ("r",))  # between the GEMM and its add: no fusion
    b.add("s", "add", ("y", "z"))
    c = forgeml_amd.compile(b.finish(("s",)), optimize=False)
    object.__setattr__(c, "kernel_plan", {"y": "hip", "z": "torch", "s": "torch"})
    assert c._plan_residual_fusions() == {}
    b = GraphBuilder({"x": spec(4, 8), "r": spec(4, 16)})
    w = b.constant("w", torch.randn(8, 16))
    b.add("y", "linear", ("x", w))
    b.add("s", "add", ("y", "r"))
    b.add("t", "add", ("s", "y"))  # y has a second consumer: no fusion
    c = forgeml_amd.compile(b.finish(("t",)), optimize=False)
    object.__setattr__(c, "kernel_plan", {"y": "hip", "s": "torch", "t": "torch"})
    assert c._plan_residual_fusions() == {}


def test_hip_plan_stores_weights_k_contiguous(monkeypatch):
    monkeypatch.setattr(kernels, "matmul", _fake_matmul([]))
    model = make_mlp()
    x = torch.randn(4, 8)
    c = forgeml_amd.compile(model, (x,))
    before = {k: v.clone() for k, v in c.graph.constants.items()}
    c.kernel_plan = {n.name: "hip" for n in c.graph.nodes}
    for node in c.graph.nodes:
        w = c.graph.constants[node.inputs[1]]
        k, n = w.shape
        # Same logical [K, N] values, stored as nn.Linear stores its weight.
        assert w.stride() == (1, k) and torch.equal(w, before[node.inputs[1]])
    torch.testing.assert_close(c(x), model(x))


def test_graph_capture_requires_gpu_inputs():
    model = make_mlp()
    x = torch.randn(4, 8)
    c = forgeml_amd.compile(model, (x,))
    with pytest.raises(GraphError, match="one GPU"):
        c.capture_graph(x)


def test_hip_plan_on_view_op_is_rejected():
    b = GraphBuilder({"x": spec(2, 4)})
    b.add("r", "reshape", ("x",), shape=(8,))
    c = forgeml_amd.compile(b.finish(("r",)), optimize=False)
    with pytest.raises(GraphError, match="no hip kernel"):
        c.kernel_plan = {"r": "hip"}


def test_explicit_graph_compiles():
    m = make_mlp()
    x = torch.randn(4, 8)
    torch.testing.assert_close(forgeml_amd.compile(from_torch(m, (x,)))(x), m(x))
