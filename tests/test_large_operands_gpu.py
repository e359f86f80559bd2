"""GPU parity on operands larger than 2 GiB and 4 GiB.

The kernels address each workgroup's operand panel through buffer resources
with 32-bit byte offsets from a 64-bit per-workgroup base, and store through
64-bit addresses; operands whose panels would not fit 32 bits take the
element-load path.  These cases put row starts, whole operands and outputs
across the 2^31 and 2^32 byte boundaries, and compare sampled rows (or
columns) with ForgeML's CPU path (the oracle) on the same inputs, at the
fused-linear parity gate.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from forgeml_amd import kernels
from oracle.fused_linear import reference_cpu, tolerance
from tests.cases import case_seed

pytestmark = pytest.mark.gpu

GIB = 1 << 30


def _say(*parts):
    print("case:", *parts, flush=True)


def _randn(shape, seed, gpu, scale, dtype):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=gpu) * scale).to(dtype)


def _around(*centres, width=24, lo=0, hi=None):
    idx = set()
    for c in centres:
        idx.update(range(max(lo, c - width), min(hi, c + width)))
    return torch.tensor(sorted(idx), dtype=torch.long)


def _release():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_tiled_bf16_a_and_c_beyond_4gib(gpu):
    """A [M, K] K-contiguous, 4.45 GB; C [M, N] 3.15 GB; ragged M and N."""
    m, n, k = 1_450_003, 1088, 1536
    seed = case_seed("large-tiled", m, n, k)
    _say("large tiled bf16", m, n, k, seed)
    a = _randn((m, k), seed, gpu, k ** -0.25, torch.bfloat16)
    w = _randn((n, k), seed + 1, gpu, k ** -0.25, torch.bfloat16)
    bias = _randn((n,), seed + 2, gpu, 0.05, torch.bfloat16)
    assert a.numel() * 2 > 4 * GIB
    plan = kernels.plan(a, w.t())
    assert plan["kernel"] == "tiled" and plan["k_splits"] == 1
    c = kernels.matmul(a, w.t(), bias, activation="gelu")
    torch.cuda.synchronize()
    a_row, c_row = k * 2, n * 2
    rows = _around(0, (2 * GIB) // a_row, (4 * GIB) // a_row, (2 * GIB) // c_row, (3 * GIB) // c_row, m - 1,
                   hi=m)
    expected = reference_cpu(a[rows.to(gpu)].cpu(), w.cpu().t(), bias.cpu(), "gelu")
    got = c[rows.to(gpu)].cpu()
    rtol, atol = tolerance(torch.bfloat16, k)
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got.float(), expected.float(), rtol=rtol, atol=atol)
    del a, w, bias, c
    _release()


def test_few_row_bf16_weight_beyond_4gib(gpu):
    """Decode-shaped: M = 8, W [N, K] of 4.5 GB read through per-column-group bases."""
    m, n, k = 8, 2_200_013, 1024
    seed = case_seed("large-few-row", m, n, k)
    _say("large few-row bf16", m, n, k, seed)
    a = _randn((m, k), seed, gpu, k ** -0.25, torch.bfloat16)
    w = _randn((n, k), seed + 1, gpu, k ** -0.25, torch.bfloat16)
    bias = _randn((n,), seed + 2, gpu, 0.05, torch.bfloat16)
    assert w.numel() * 2 > 4 * GIB
    assert kernels.plan(a, w.t(), kernels.SKINNY_H16)["kernel"] == "few-row"
    c = kernels.matmul(a, w.t(), bias, activation="gelu", config=kernels.SKINNY_H16)
    torch.cuda.synchronize()
    w_row = k * 2
    cols = _around(0, (2 * GIB) // w_row, (4 * GIB) // w_row, n - 1, hi=n)
    cg = cols.to(gpu)
    expected = reference_cpu(a.cpu(), w[cg].cpu().t(), bias[cg].cpu(), "gelu")
    got = c[:, cg].cpu()
    rtol, atol = tolerance(torch.bfloat16, k)
    torch.testing.assert_close(got.float(), expected.float(), rtol=rtol, atol=atol)
    del a, w, bias, c
    _release()


def test_tiled_fp32_m_contiguous_a_beyond_2gib(gpu):
    """A = X^T with X [K, M] fp32 of 2.2 GB: too large for 32-bit offsets over
    the panel's K extent, so A takes the element-load path."""
    m, n, k = 530_000, 200, 1040
    seed = case_seed("large-mn", m, n, k)
    _say("large fp32 M-contiguous A", m, n, k, seed)
    x = _randn((k, m), seed, gpu, k ** -0.25, torch.float32)
    w = _randn((n, k), seed + 1, gpu, k ** -0.25, torch.float32)
    bias = _randn((n,), seed + 2, gpu, 0.05, torch.float32)
    a = x.t()
    assert x.numel() * 4 > 2 * GIB and a.stride() == (1, m)
    assert kernels.plan(a, w.t())["kernel"] == "tiled"
    c = kernels.matmul(a, w.t(), bias, activation="gelu", approximate="tanh")
    torch.cuda.synchronize()
    rows = _around(0, m // 2, m - 1, hi=m)
    expected = reference_cpu(a[rows.to(gpu)].cpu(), w.cpu().t(), bias.cpu(), "gelu", "tanh")
    got = c[rows.to(gpu)].cpu()
    rtol, atol = tolerance(torch.float32, k)
    torch.testing.assert_close(got, expected, rtol=rtol, atol=atol)
    del x, a, w, bias, c
    _release()


def test_layer_norm_beyond_4gib(gpu):
    """8.6 GB in and out; 2^21 + 3 rows, so the rows take two launches."""
    rows, cols = (1 << 21) + 3, 1024
    seed = case_seed("large-ln", rows, cols)
    _say("large layer_norm fp32", rows, cols, seed)
    x = _randn((rows, cols), seed, gpu, 2.0, torch.float32)
    w = _randn((cols,), seed + 1, gpu, 1.0, torch.float32)
    b = _randn((cols,), seed + 2, gpu, 0.1, torch.float32)
    assert x.numel() * 4 > 8 * GIB
    y = kernels.layer_norm(x, (cols,), w, b, 1e-5)
    torch.cuda.synchronize()
    r = _around(0, (2 * GIB) // (cols * 4), (4 * GIB) // (cols * 4), 1 << 21, rows - 1, hi=rows).to(gpu)
    expected = F.layer_norm(x[r].cpu(), (cols,), w.cpu(), b.cpu(), 1e-5)
    torch.testing.assert_close(y[r].cpu(), expected, rtol=1e-4, atol=1e-5)
    del x, w, b, y
    _release()
