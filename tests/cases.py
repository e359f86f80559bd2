"""Seeded inputs for the parity tests."""

from __future__ import annotations

import zlib

import torch


def case_seed(*parts) -> int:
    """Deterministic seed from a case description (recorded in failures)."""
    return zlib.crc32(repr(parts).encode()) & 0x7FFFFFFF


def gemm_inputs(m: int, n: int, k: int, dtype: torch.dtype, *, seed: int, b_layout: str = "nt",
                bias: bool = True):
    """A [M,K] and B [K,N] with entries N(0, 1/sqrt(K)) (std K**-0.25, so C is O(1)),
    bias U(-0.1, 0.1); all generated in fp32 on the CPU and cast.

    b_layout "nt": B is the transposed view of a contiguous nn.Linear weight
    W[N,K] (strides (1, K)); "nn": B is contiguous [K,N].
    """
    g = torch.Generator().manual_seed(seed)
    std = k ** -0.25
    a = (torch.randn(m, k, generator=g) * std).to(dtype)
    w = (torch.randn(n, k, generator=g) * std).to(dtype)
    bvec = ((torch.rand(n, generator=g) * 0.2 - 0.1).to(dtype)) if bias else None
    b = w.t() if b_layout == "nt" else w.t().contiguous()
    return a, b, bvec


def to_gpu(t, device):
    if t is None:
        return None
    # Keep the layout (a transposed view stays a transposed view).
    if t.dim() == 2 and not t.is_contiguous() and t.t().is_contiguous():
        return t.t().contiguous().to(device).t()
    return t.to(device)
