"""Workload models compiled by the benchmarks and tests.

``TransformerBlock`` has the structure of ForgeML's block
(src/forgeml/neural.py:18-53): pre-LayerNorm, separate Q/K/V projections
(fused into one wide GEMM by the pass pipeline), causal SDPA, output
projection with residual, then a GELU(tanh) FFN with residual.
``make_mlp`` builds the Linear -> GELU -> Linear stack of the compiler
benchmark (src/forgeml/benchmarks.py:33-38).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


class TransformerBlock(nn.Module):
    def __init__(self, hidden_size: int = 128, num_heads: int = 8, intermediate_size: int = 256,
                 causal: bool = True, approximate: str = "tanh"):
        super().__init__()
        if hidden_size <= 0 or num_heads <= 0 or hidden_size % num_heads:
            raise ValueError("hidden size must be positive and divisible by heads")
        self.num_heads = num_heads
        self.head_dim = hidden_size // num_heads
        self.causal = causal
        self.approximate = approximate
        self.ln1 = nn.LayerNorm(hidden_size)
        self.ln2 = nn.LayerNorm(hidden_size)
        self.q = nn.Linear(hidden_size, hidden_size)
        self.k = nn.Linear(hidden_size, hidden_size)
        self.v = nn.Linear(hidden_size, hidden_size)
        self.o = nn.Linear(hidden_size, hidden_size)
        self.up = nn.Linear(hidden_size, intermediate_size)
        self.down = nn.Linear(intermediate_size, hidden_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch, seq, hidden = x.shape
        residual = x
        normalized = self.ln1(x).reshape(batch * seq, hidden)
        q = self.q(normalized).view(batch, seq, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k(normalized).view(batch, seq, self.num_heads, self.head_dim).transpose(1, 2)
        v = self.v(normalized).view(batch, seq, self.num_heads, self.head_dim).transpose(1, 2)
        attended = F.scaled_dot_product_attention(q, k, v, is_causal=self.causal)
        attended = attended.transpose(1, 2).reshape(batch * seq, hidden)
        x = residual + self.o(attended).reshape(batch, seq, hidden)
        residual = x
        normalized = self.ln2(x).reshape(batch * seq, hidden)
        hidden_act = F.gelu(self.up(normalized), approximate=self.approximate)
        return residual + self.down(hidden_act).reshape(batch, seq, hidden)


def make_mlp(width: int, hidden: int, output: int, approximate: str = "none") -> nn.Module:
    """Linear(width->hidden) + bias -> GELU -> Linear(hidden->output) + bias, eval mode."""
    return nn.Sequential(
        nn.Linear(width, hidden), nn.GELU(approximate=approximate), nn.Linear(hidden, output)
    ).eval()


class ResidualMLP(nn.Module):
    def __init__(self, width: int, hidden: int, approximate: str = "tanh"):
        super().__init__()
        self.up = nn.Linear(width, hidden)
        self.activation = nn.GELU(approximate=approximate)
        self.down = nn.Linear(hidden, width)

    def forward(self, x):
        return self.down(self.activation(self.up(x))) + x
