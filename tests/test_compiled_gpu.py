"""CompiledModel on the GPU: GEMM nodes run on the gfx950 kernels, results
match the reference's CPU path (the same model compiled with the torch
backend on the CPU) on the same seeded inputs."""

from __future__ import annotations

import pytest
import torch
from torch import nn

import forgeml_amd
from forgeml_amd import kernels
from forgeml_amd.neural import TransformerBlock, make_mlp
from oracle.fused_linear import reference_cpu, tolerance

pytestmark = pytest.mark.gpu


def _say(*parts):
    print("case:", *parts, flush=True)


def _cpu_reference(model: nn.Module, x: torch.Tensor) -> torch.Tensor:
    compiled = forgeml_amd.compile(model, (x,), backend="torch")
    with torch.inference_mode():
        return compiled(x)


def _compiled_mlp(gpu, approximate="none"):
    torch.manual_seed(0)
    model = make_mlp(512, 2048, 512, approximate=approximate)
    torch.manual_seed(1)
    x = torch.randn(64, 512)
    return model, x


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_compiled_mlp_matches_cpu_path(gpu, approximate):
    """Linear(512->2048)+bias+GELU -> Linear(2048->512)+bias, batch 64, fp32."""
    model, x = _compiled_mlp(gpu, approximate)
    expected = _cpu_reference(model, x)
    model_gpu = model.to(gpu)
    xg = x.to(gpu)
    compiled = forgeml_amd.compile(model_gpu, (xg,), backend="hip")
    assert [n.op for n in compiled.graph.nodes] == ["fused_linear_gelu", "linear"]
    assert set(compiled.kernel_plan.values()) == {"hip"}
    _say("compiled MLP", approximate)
    got = compiled(xg)
    rtol, atol = tolerance(torch.float32, 2048)
    torch.testing.assert_close(got.cpu(), expected, rtol=rtol, atol=atol)
    # Calls are repeatable through the reused slot arena.
    torch.testing.assert_close(compiled(xg).cpu(), got.cpu(), rtol=0, atol=0)


def test_internal_gemm_writes_into_its_slot(gpu, monkeypatch):
    model, x = _compiled_mlp(gpu)
    xg = x.to(gpu)
    compiled = forgeml_amd.compile(model.to(gpu), (xg,), backend="hip")
    fused = compiled.graph.nodes[0].name
    slot_view = compiled._views[fused]
    outs = []
    real = kernels.matmul

    def spy(*args, **kw):
        result = real(*args, **kw)
        outs.append(result.data_ptr())
        return result

    monkeypatch.setattr(kernels, "matmul", spy)
    _say("slot write")
    compiled(xg)
    assert outs[0] == slot_view.data_ptr()
    assert outs[1] != slot_view.data_ptr()


def _block():
    torch.manual_seed(0)
    block = TransformerBlock(768, 12, 3072).eval()
    torch.manual_seed(1)
    x = torch.randn(8, 512, 768)
    return block, x


def _assert_block_on_hip(compiled):
    """Every GEMM, LayerNorm and attention node of the block runs this build's kernels."""
    plan = compiled.kernel_plan
    by_op = {}
    for node in compiled.graph.nodes:
        by_op.setdefault(node.op, []).append(node.name)
    gemm_nodes = [n for op in kernels.GEMM_OPS for n in by_op.get(op, [])]
    assert len(gemm_nodes) == 4 and all(plan[n] == "hip" for n in gemm_nodes)
    assert len(by_op["layer_norm"]) == 2 and all(plan[n] == "hip" for n in by_op["layer_norm"])
    assert len(by_op["sdpa"]) == 1 and plan[by_op["sdpa"][0]] == "hip"
    # Both residual adds ride in the out-projection and FFN-down epilogues.
    assert len(compiled.fused_residuals) == 2


def test_compiled_transformer_block_matches_cpu_path(gpu):
    """Pre-LN block d=768, 12 heads, FFN 3072 (fused linear+GELU), seq 512, batch 8, fp32.

    Gated at the fp32 tolerance with K of the widest GEMM (3072): the block's
    GEMMs, LayerNorms and attention all run on this build's kernels, and its
    fp32 error through one block is far inside that gate."""
    block, x = _block()
    expected = _cpu_reference(block, x)
    xg = x.to(gpu)
    compiled = forgeml_amd.compile(block.to(gpu), (xg,), backend="hip")
    _assert_block_on_hip(compiled)
    _say("compiled transformer block")
    got = compiled(xg).cpu()
    rtol, atol = tolerance(torch.float32, 3072)
    torch.testing.assert_close(got, expected, rtol=rtol, atol=atol)


def _cpu_values(compiled, x):
    """Every node's value of a CPU compiled model's call (nothing released)."""
    values = dict(compiled._check_inputs((x,)))
    values.update(compiled.graph.constants)
    with torch.inference_mode():
        for node, run, inputs in compiled._steps:
            values[node.name] = run(tuple(values[i] for i in inputs))
            if node.name in compiled._views:
                values[node.name] = values[node.name].clone()  # slots are reused later in the call
    return values


def test_transformer_block_gemms_on_block_activations(gpu):
    """Each of the block's four GEMMs on its own activations (QKV 4096x2304x768,
    out-proj 4096x768x768, FFN up 4096x3072x768 + tanh GELU, FFN down
    4096x768x3072), fed from the CPU compile's intermediates to the kernel
    and to the CPU path, at the fp32 gate rtol 1e-4 / atol 1e-5 sqrt(K)."""
    block, x = _block()
    cpu = forgeml_amd.compile(block, (x,), backend="torch")
    values = _cpu_values(cpu, x)
    gemms = [n for n in cpu.graph.nodes if n.op in kernels.GEMM_OPS]
    shapes = []
    for node in gemms:
        a, b = values[node.inputs[0]], values[node.inputs[1]]
        bias = values[node.inputs[2]] if len(node.inputs) == 3 else None
        act = "gelu" if node.op == "fused_linear_gelu" else "none"
        approx = node.attrs.get("approximate", "none")
        m, k = a.shape
        n = b.shape[1]
        shapes.append((m, n, k))
        expected = reference_cpu(a, b, bias, act, approx)
        rtol, atol = tolerance(torch.float32, k)
        # B as the compiled model stores it (K-contiguous) and row-major.
        for name, b_d in (("W^T", b.t().contiguous().to(gpu).t()), ("[K,N]", b.contiguous().to(gpu))):
            what = f"block GEMM {node.name} {m}x{n}x{k} act={act}/{approx} B={name}"
            _say(what)
            got = kernels.matmul(a.to(gpu), b_d, None if bias is None else bias.to(gpu), activation=act,
                                 approximate=approx).cpu()
            torch.testing.assert_close(got, expected, rtol=rtol, atol=atol, msg=lambda msg: f"{what}: {msg}")
    assert sorted(shapes) == sorted([(4096, 2304, 768), (4096, 768, 768), (4096, 3072, 768), (4096, 768, 3072)])


def test_autotune_on_gpu_gates_and_picks(gpu):
    model, x = _compiled_mlp(gpu)
    expected = _cpu_reference(model, x)  # before .to(gpu), which moves the module in place
    xg = x.to(gpu)
    compiled = forgeml_amd.compile(model.to(gpu), (xg,), backend="hip")
    _say("autotune")
    report = compiled.autotune(xg, warmup=1, repeats=3)
    assert set(report["nodes"]) == {n.name for n in compiled.graph.nodes}
    for name, rec in report["nodes"].items():
        assert not rec["rejected"], rec["rejected"]
        assert rec["winner"] in rec["candidates"]
        assert compiled.kernel_configs[name] in kernels.candidates(torch.float32)
    rtol, atol = tolerance(torch.float32, 2048)
    torch.testing.assert_close(compiled(xg).cpu(), expected, rtol=rtol, atol=atol)


def test_mixed_plan_relu_residual(gpu):
    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.lin = nn.Linear(16, 16)

        def forward(self, x):
            return torch.relu(self.lin(x)) + x

    torch.manual_seed(2)
    m = M().eval()
    x = torch.randn(4, 16)
    expected = _cpu_reference(m, x)
    c = forgeml_amd.compile(m.to(gpu), (x.to(gpu),), backend="auto")
    assert "hip" in c.kernel_plan.values() and "torch" in c.kernel_plan.values()
    _say("mixed plan")
    torch.testing.assert_close(c(x.to(gpu)).cpu(), expected, rtol=1e-4, atol=1e-4)


# -- HIP-graph capture of a compiled model --------------------------------------

def _graph_replays_match_eager(compiled, make_input, rtol=0.0, atol=0.0, replays=3):
    graphed = compiled.capture_graph(make_input(0))
    for r in range(1, replays + 1):
        x = make_input(r)
        _say("graph replay", r)
        got = graphed(x).clone()
        # Eager work of the program between replays, on the same arena.
        eager = compiled(x)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, eager, rtol=rtol, atol=atol)
    return graphed


def test_graphed_mlp_matches_eager_and_cpu(gpu):
    model, x = _compiled_mlp(gpu)
    expected = _cpu_reference(model, x)
    compiled = forgeml_amd.compile(model.to(gpu), (x.to(gpu),), backend="hip")

    def make_input(r):
        g = torch.Generator().manual_seed(100 + r)
        return torch.randn(64, 512, generator=g).to(gpu)

    graphed = _graph_replays_match_eager(compiled, make_input)
    rtol, atol = tolerance(torch.float32, 2048)
    torch.testing.assert_close(graphed(x.to(gpu)).cpu(), expected, rtol=rtol, atol=atol)


def test_graphed_transformer_block_matches_eager(gpu):
    block, x = _block()
    expected = _cpu_reference(block, x)
    compiled = forgeml_amd.compile(block.to(gpu), (x.to(gpu),), backend="hip")
    _assert_block_on_hip(compiled)

    def make_input(r):
        g = torch.Generator().manual_seed(200 + r)
        return torch.randn(8, 512, 768, generator=g).to(gpu)

    graphed = _graph_replays_match_eager(compiled, make_input, rtol=1e-6, atol=1e-6)
    rtol, atol = tolerance(torch.float32, 3072)
    torch.testing.assert_close(graphed(x.to(gpu)).cpu(), expected, rtol=rtol, atol=atol)
