"""Graph rewrites that produce the GEMM nodes (src/forgeml/passes.py)."""

import pytest
import torch

from forgeml_amd.ir import GraphBuilder, TensorSpec
from forgeml_amd.passes import (
    canonicalize_linear,
    common_subexpression_elimination,
    eliminate_dead_nodes,
    fold_constants,
    fuse_linear_gelu,
    fuse_shared_projections,
    optimize,
    schedule,
    simplify_algebra,
)


def spec(*shape):
    return TensorSpec(tuple(shape), torch.float32, "cpu")


def _mm_bias_gelu(outputs=("y",), share=False):
    b = GraphBuilder({"x": spec(2, 4)})
    b.constant("w", torch.randn(4, 8))
    b.constant("bias", torch.randn(8))
    b.add("mm", "matmul", ("x", "w"))
    b.add("lin", "add", ("mm", "bias"))
    b.add("y", "gelu", ("lin",), approximate="tanh")
    if share:
        b.add("z", "relu", ("lin",))
        outputs = ("y", "z")
    return b.finish(outputs)


def test_dce_and_fold():
    b = GraphBuilder({"x": spec(2, 3)})
    b.constant("dead_w", torch.ones(3, 3))
    b.constant("a", torch.ones(3))
    b.constant("c", torch.full((3,), 3.0))
    b.add("dead", "matmul", ("x", "dead_w"))
    b.add("ac", "add", ("a", "c"))
    b.add("y", "mul", ("x", "ac"))
    g = eliminate_dead_nodes(b.finish(("y",)))
    assert [n.name for n in g.nodes] == ["ac", "y"] and "dead_w" not in g.constants
    f = fold_constants(g)
    assert [n.name for n in f.nodes] == ["y"]
    torch.testing.assert_close(f.constants["ac"], torch.full((3,), 4.0))


def test_fold_respects_size_cap(monkeypatch):
    import forgeml_amd.passes as passes

    monkeypatch.setattr(passes, "FOLD_LIMIT_BYTES", 8)
    b = GraphBuilder({"x": spec(4)})
    b.constant("a", torch.ones(4))
    b.add("aa", "add", ("a", "a"))
    b.add("y", "mul", ("x", "aa"))
    f = passes.fold_constants(b.finish(("y",)))
    assert [n.name for n in f.nodes] == ["aa", "y"]


def test_matmul_bias_gelu_fuses_to_one_node():
    out = fuse_linear_gelu(_mm_bias_gelu())
    assert len(out.nodes) == 1
    node = out.nodes[0]
    assert (node.op, node.name, node.attrs["approximate"]) == ("fused_linear_gelu", "y", "tanh")
    assert node.inputs == ("x", "w", "bias")


def test_fusion_skipped_when_intermediate_is_shared_or_output():
    assert [n.op for n in fuse_linear_gelu(_mm_bias_gelu(share=True)).nodes] == ["matmul", "add", "gelu", "relu"]
    g = _mm_bias_gelu(outputs=("y", "lin"))
    assert "fused_linear_gelu" not in [n.op for n in fuse_linear_gelu(g).nodes]


def test_canonicalize_linear_either_operand_order():
    b = GraphBuilder({"x": spec(2, 4)})
    b.constant("w", torch.randn(4, 8))
    b.constant("bias", torch.randn(8))
    b.add("mm", "matmul", ("x", "w"))
    b.add("y", "add", ("bias", "mm"))
    out = canonicalize_linear(b.finish(("y",)))
    assert [(n.op, n.name, n.inputs) for n in out.nodes] == [("linear", "y", ("x", "w", "bias"))]


def test_fused_linear_gelu_from_linear_and_bare_matmul():
    for op, inputs in (("linear", ("x", "w", "bias")), ("matmul", ("x", "w"))):
        b = GraphBuilder({"x": spec(2, 4)})
        b.constant("w", torch.randn(4, 8))
        b.constant("bias", torch.randn(8))
        b.add("p", op, inputs)
        b.add("y", "gelu", ("p",))
        out = fuse_linear_gelu(b.finish(("y",)))
        assert [(n.op, n.inputs) for n in out.nodes] == [("fused_linear_gelu", inputs)]


def test_shared_projections_become_one_wide_gemm():
    b = GraphBuilder({"x": spec(3, 4)})
    for name in ("q", "k", "v"):
        b.constant(f"{name}_w", torch.randn(4, 4))
        b.constant(f"{name}_b", torch.randn(4))
        b.add(name, "linear", ("x", f"{name}_w", f"{name}_b"))
    b.add("qk", "add", ("q", "k"))
    b.add("y", "add", ("qk", "v"))
    g = b.finish(("y",))
    out = fuse_shared_projections(g)
    ops = [(n.op, n.name) for n in out.nodes]
    assert ops[0] == ("linear", "q_shared_3") and ops[1:4] == [("narrow", "q"), ("narrow", "k"), ("narrow", "v")]
    assert out.nodes[0].spec.shape == (3, 12)
    x = torch.randn(3, 4)
    from forgeml_amd import compile as fcompile

    torch.testing.assert_close(fcompile(out, optimize=False)(x), fcompile(g, optimize=False)(x))


def test_simplify_and_cse():
    b = GraphBuilder({"x": spec(2, 3)})
    b.add("t1", "transpose", ("x",), dim0=0, dim1=1)
    b.add("t2", "transpose", ("t1",), dim0=1, dim1=0)
    b.add("r", "reshape", ("t2",), shape=(2, 3))
    b.add("a", "relu", ("r",))
    b.add("b", "relu", ("r",))
    b.add("y", "add", ("a", "b"))
    g = common_subexpression_elimination(simplify_algebra(b.finish(("y",))))
    assert [n.op for n in g.nodes] == ["relu", "add"]
    assert g.nodes[1].inputs == ("a", "a")


def test_schedule_is_valid_and_deterministic():
    g = _mm_bias_gelu()
    s1, s2 = schedule(g), schedule(g)
    assert [n.name for n in s1.nodes] == [n.name for n in s2.nodes]
    seen = set(g.inputs) | set(g.constants)
    for n in s1.nodes:
        assert all(i in seen for i in n.inputs)
        seen.add(n.name)


def test_optimize_records_every_pass_and_keeps_input_graph():
    g = _mm_bias_gelu()
    before = [n.name for n in g.nodes]
    out, records = optimize(g)
    assert [r.name for r in records][-1] == "schedule" and len(records) == 10
    assert [n.name for n in g.nodes] == before
    assert [n.op for n in out.nodes] == ["fused_linear_gelu"]


@pytest.mark.parametrize("bad_bias_shape", [(1, 8), (7,)])
def test_fusion_requires_1d_output_width_bias(bad_bias_shape):
    b = GraphBuilder({"x": spec(2, 4)})
    b.constant("w", torch.randn(4, 8))
    b.constant("bias", torch.randn(*bad_bias_shape))
    b.add("mm", "matmul", ("x", "w"))
    if bad_bias_shape == (7,):
        return  # not even a valid add; nothing to fuse
    b.add("lin", "add", ("mm", "bias"))
    b.add("y", "gelu", ("lin",))
    assert "fused_linear_gelu" not in [n.op for n in fuse_linear_gelu(b.finish(("y",))).nodes]
