"""IR semantics (specs, builder, validation) kept from src/forgeml/ir.py."""

import pytest
import torch

from forgeml_amd.ir import Graph, GraphBuilder, GraphError, Node, TensorSpec, infer_spec


def spec(*shape, device="cpu", dtype=torch.float32):
    return TensorSpec(tuple(shape), dtype, device)


def test_tensorspec_validation_and_nbytes():
    with pytest.raises(GraphError):
        spec(0, 3)
    with pytest.raises(GraphError):
        TensorSpec((2,), torch.complex64, "cpu")
    with pytest.raises(GraphError):
        TensorSpec((2,), torch.float32, "not-a-device")
    assert spec(2, 3).nbytes == 24
    assert TensorSpec((2,), torch.float32, "cuda").device == "cuda:0"


def test_builder_rejects_duplicates_missing_inputs_and_unknown_ops():
    b = GraphBuilder({"x": spec(2, 4)})
    b.constant("w", torch.randn(4, 8))
    with pytest.raises(GraphError, match="duplicate"):
        b.constant("w", torch.randn(4, 8))
    with pytest.raises(GraphError, match="not defined"):
        b.add("y", "matmul", ("x", "nope"))
    with pytest.raises(GraphError, match="unsupported op"):
        b.add("y", "sin", ("x",))
    with pytest.raises(GraphError, match="shape mismatch"):
        b.constant("w2", torch.randn(5, 8))
        b.add("y", "matmul", ("x", "w2"))


def test_linear_and_fused_specs():
    b = GraphBuilder({"x": spec(2, 4)})
    b.constant("w", torch.randn(4, 8))
    b.constant("bias", torch.randn(8))
    b.add("lin", "linear", ("x", "w", "bias"))
    b.add("f", "fused_linear_gelu", ("x", "w"), approximate="tanh")
    g = b.finish(("lin", "f"))
    assert g.nodes[0].spec.shape == (2, 8) and g.nodes[1].spec.shape == (2, 8)
    assert g.output_is_tuple
    with pytest.raises(GraphError, match="bias"):
        b2 = GraphBuilder({"x": spec(2, 4)})
        b2.constant("w", torch.randn(4, 8))
        b2.constant("bias", torch.randn(7))
        b2.add("lin", "linear", ("x", "w", "bias"))
    with pytest.raises(GraphError, match="approximate"):
        b3 = GraphBuilder({"x": spec(2, 4)})
        b3.constant("w", torch.randn(4, 8))
        b3.add("f", "fused_linear_gelu", ("x", "w"), approximate="fast")


def test_graph_validate_rejects_wrong_spec_and_empty_outputs():
    node = Node("y", "relu", ("x",), {}, spec(3))
    g = Graph({"x": spec(2)}, {}, [node], ("y",))
    with pytest.raises(GraphError, match="spec mismatch"):
        g.validate()
    with pytest.raises(GraphError, match="non-empty"):
        Graph({"x": spec(2)}, {}, [], ()).validate()


def test_device_mismatch_and_cpu_scalar():
    with pytest.raises(GraphError, match="device mismatch"):
        infer_spec("add", [spec(2), spec(2, device="cuda:0")], {})
    out = infer_spec("add", [TensorSpec((), torch.float32, "cpu"), spec(2, device="cuda:0")], {})
    assert out.device == "cuda:0"


def test_float_only_ops_and_required_attrs():
    with pytest.raises(GraphError, match="floating-point"):
        infer_spec("gelu", [spec(2, dtype=torch.int32)], {})
    with pytest.raises(GraphError, match="requires attrs"):
        infer_spec("reshape", [spec(2)], {})


def test_clone_and_to_dict_and_mermaid():
    b = GraphBuilder({"x": spec(2, 4)})
    b.constant("w", torch.ones(4, 8))
    b.add("y", "matmul", ("x", "w"))
    g = b.finish(("y",))
    c = g.clone()
    c.constants["w"].fill_(3.0)
    assert g.constants["w"].max().item() == 1.0
    d = g.to_dict()
    assert d["nodes"][0]["op"] == "matmul" and d["outputs"] == ["y"]
    assert "graph TD" in g.to_mermaid()
