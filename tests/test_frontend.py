"""FX lowering of the models on the linear path (src/forgeml/frontend.py)."""

import pytest
import torch
import torch.nn.functional as F
from torch import nn

import forgeml_amd
from forgeml_amd.frontend import UnsupportedOperator, from_torch
from forgeml_amd.ir import GraphError
from forgeml_amd.neural import TransformerBlock


def check(model, *xs, **kw):
    c = forgeml_amd.compile(model.eval(), xs, **kw)
    torch.testing.assert_close(c(*xs), model(*xs))
    return c


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_mlp_parity(approximate):
    check(nn.Sequential(nn.Linear(8, 16), nn.GELU(approximate=approximate), nn.Linear(16, 4)), torch.randn(3, 8))


def test_linear_weight_stored_transposed_contiguous():
    lin = nn.Linear(8, 5)
    g = from_torch(lin, (torch.randn(2, 8),))
    w = next(v for k, v in g.constants.items() if "weight_t" in k)
    assert w.shape == (8, 5) and w.is_contiguous()
    torch.testing.assert_close(w, lin.weight.t())


def test_rank3_linear_is_flattened_and_restored():
    c = check(nn.Linear(8, 6), torch.randn(2, 3, 8))
    assert [n.op for n in c.graph.nodes] == ["reshape", "linear", "reshape"]


def test_functional_linear_and_mm():
    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.w = nn.Parameter(torch.randn(6, 8))
            self.b = nn.Parameter(torch.randn(6))
            self.m = nn.Parameter(torch.randn(6, 3))

        def forward(self, x):
            return torch.mm(F.linear(x, self.w, self.b), self.m)

    check(M(), torch.randn(4, 8))


def test_transformer_block_parity():
    torch.manual_seed(0)
    c = check(TransformerBlock(64, 4, 128), torch.randn(2, 16, 64))
    ops = [n.op for n in c.graph.nodes]
    assert ops.count("fused_linear_gelu") == 1 and ops.count("sdpa") == 1
    assert ops.count("linear") == 3  # wide QKV, output projection, down projection


def test_static_shape_queries_and_view():
    class M(nn.Module):
        def forward(self, x):
            b, s, h = x.shape
            return x.view(b * s, h).reshape(-1, x.size(-1)).softmax(dim=-1)

    check(M(), torch.randn(2, 3, 4))


def test_unsupported_and_training_mode_rejected():
    class Sin(nn.Module):
        def forward(self, x):
            return torch.sin(x)

    with pytest.raises(UnsupportedOperator):
        from_torch(Sin(), (torch.randn(2),))
    with pytest.raises(GraphError, match="training mode"):
        from_torch(nn.Sequential(nn.Linear(4, 4), nn.Dropout(0.1)).train(), (torch.randn(2, 4),))
    with pytest.raises(GraphError, match="example inputs"):
        from_torch(nn.Linear(4, 4), ())


def test_weight_snapshot_isolated_from_mutation():
    lin = nn.Linear(4, 3).eval()
    x = torch.randn(2, 4)
    c = forgeml_amd.compile(lin, (x,))
    expected = lin(x)
    with torch.no_grad():
        lin.weight.add_(1.0)
    torch.testing.assert_close(c(x), expected)
