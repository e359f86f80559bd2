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
from oracle.fused_linear import tolerance

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


def test_compiled_transformer_block_matches_cpu_path(gpu):
    """Pre-LN block d=768, 12 heads, FFN 3072 (fused linear+GELU), seq 512, batch 8, fp32."""
    torch.manual_seed(0)
    block = TransformerBlock(768, 12, 3072).eval()
    torch.manual_seed(1)
    x = torch.randn(8, 512, 768)
    expected = _cpu_reference(block, x)
    blk = block.to(gpu)
    xg = x.to(gpu)
    compiled = forgeml_amd.compile(blk, (xg,), backend="hip")
    plan = compiled.kernel_plan
    gemm_nodes = [n.name for n in compiled.graph.nodes if n.op in kernels.GEMM_OPS]
    assert len(gemm_nodes) == 4 and all(plan[n] == "hip" for n in gemm_nodes)
    # Both residual adds ride in the out-projection and FFN-down epilogues.
    assert len(compiled.fused_residuals) == 2
    _say("compiled transformer block")
    torch.backends.cuda.matmul.allow_tf32 = False
    got = compiled(xg).cpu()
    # Non-GEMM ops (LayerNorm, SDPA) run on torch-ROCm; compounding over four
    # GEMMs and attention, the fp32 gate is applied with K of the widest GEMM.
    rtol, atol = tolerance(torch.float32, 3072)
    torch.testing.assert_close(got, expected, rtol=rtol * 10, atol=atol * 10)


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
    torch.manual_seed(0)
    block = TransformerBlock(768, 12, 3072).eval()
    torch.manual_seed(1)
    x = torch.randn(8, 512, 768)
    expected = _cpu_reference(block, x)
    torch.backends.cuda.matmul.allow_tf32 = False
    compiled = forgeml_amd.compile(block.to(gpu), (x.to(gpu),), backend="hip")

    def make_input(r):
        g = torch.Generator().manual_seed(200 + r)
        return torch.randn(8, 512, 768, generator=g).to(gpu)

    graphed = _graph_replays_match_eager(compiled, make_input, rtol=1e-6, atol=1e-6)
    rtol, atol = tolerance(torch.float32, 3072)
    torch.testing.assert_close(graphed(x.to(gpu)).cpu(), expected, rtol=rtol * 10, atol=atol * 10)
