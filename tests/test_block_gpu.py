"""GPU parity of the transformer block's LayerNorm and attention kernels
against ForgeML's CPU path for those ops (torch F.layer_norm and
F.scaled_dot_product_attention on the CPU, src/forgeml/ops.py), on the same
seeded inputs.  fp32 outputs are gated at rtol 1e-4 / atol 1e-5; 16-bit
LayerNorm outputs at one rounding step of the dtype."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from forgeml_amd import kernels
from forgeml_amd.ir import GraphError
from tests.cases import case_seed

pytestmark = pytest.mark.gpu


def _say(*parts):
    print("case:", *parts, flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(4096, 768), (8, 512, 768), (7, 100), (3, 5000), (5, 1030), (64, 4096), (6, 16384), (2, 20000), (2, 40000), (1, 140000)])
def test_layer_norm(gpu, dtype, shape):
    g = torch.Generator().manual_seed(case_seed("ln", shape, dtype))
    x = (torch.randn(*shape, generator=g) * 2 + 0.5).to(dtype)
    d = shape[-1]
    w = (torch.rand(d, generator=g) + 0.5).to(dtype)
    b = (torch.randn(d, generator=g) * 0.1).to(dtype)
    for affine in (True, False):
        _say("layer_norm", shape, dtype, affine)
        wa, ba = (w, b) if affine else (None, None)
        expected = F.layer_norm(x.float(), (d,), None if wa is None else wa.float(), None if ba is None else ba.float(),
                                1e-5)
        got = kernels.layer_norm(x.to(gpu), (d,), None if wa is None else wa.to(gpu),
                                 None if ba is None else ba.to(gpu), 1e-5).cpu()
        if dtype == torch.float32:
            torch.testing.assert_close(got, expected, rtol=1e-4, atol=1e-5)
        else:
            # fp32 statistics rounded once: within one rounding step of the dtype
            # of the fp32 result (the CPU reference in the dtype rounds more often).
            torch.testing.assert_close(got.float(), expected.to(dtype).float(), rtol=1e-2, atol=1e-2)


def _attention_inputs(b, h, lq, lk, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, lq, d, generator=g)
    k = torch.randn(b, h, lk, d, generator=g)
    v = torch.randn(b, h, lk, d, generator=g)
    return q, k, v


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,h,lq,lk,d", [(2, 3, 100, 100, 64), (1, 2, 33, 33, 32), (2, 2, 64, 64, 96),
                                          (1, 4, 512, 512, 64), (2, 1, 40, 70, 64), (1, 1, 1, 1, 64),
                                          (2, 3, 100, 100, 128), (1, 2, 300, 300, 128)])
def test_attention(gpu, causal, b, h, lq, lk, d):
    seed = case_seed("attn", b, h, lq, lk, d, causal)
    q, k, v = _attention_inputs(b, h, lq, lk, d, seed)
    _say("attention", b, h, lq, lk, d, causal, seed)
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    got = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=causal)
    assert got.shape == expected.shape
    torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-5)


def test_attention_strided_views_and_scale(gpu):
    # q, k, v as the transformer block makes them: narrow + view + transpose of
    # one packed projection, i.e. strided [B, H, S, D] views; explicit scale.
    bsz, s, h, d = 2, 96, 4, 64
    g = torch.Generator().manual_seed(case_seed("attn_views"))
    qkv = torch.randn(bsz * s, 3 * h * d, generator=g)
    def split(t):
        return [t[:, i * h * d:(i + 1) * h * d].reshape(bsz, s, h, d).transpose(1, 2) for i in range(3)]
    q, k, v = split(qkv)
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.2)
    qd, kd, vd = split(qkv.to(gpu))
    _say("attention strided views")
    got = kernels.attention(qd, kd, vd, is_causal=True, scale=0.2)
    torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-5)
    # Stored [B, S, H, D]: the block's transpose + reshape is a free view.
    assert got.transpose(1, 2).is_contiguous()
    assert torch.equal(got, kernels.attention(qd, kd, vd, is_causal=True, scale=0.2))


def test_block_kernel_argument_checks(gpu):
    with pytest.raises(GraphError, match="fp32"):
        kernels.attention(*(torch.randn(1, 1, 8, 64, device=gpu, dtype=torch.bfloat16),) * 3)
    with pytest.raises(GraphError, match="not supported"):
        kernels.attention(*(torch.randn(1, 1, 8, 48, device=gpu),) * 3)
    with pytest.raises(GraphError, match="does not end"):
        kernels.layer_norm(torch.randn(4, 8, device=gpu), (16,))
