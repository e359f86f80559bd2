"""GPU parity of the transformer block's LayerNorm and attention kernels
against ForgeML's CPU path for those ops (torch F.layer_norm and
F.scaled_dot_product_attention on the CPU, src/forgeml/ops.py), on the same
seeded inputs.  fp32 outputs are gated at rtol 1e-4 / atol 1e-5.  16-bit
LayerNorm outputs are held to one rounding of the exact result: within one
ulp of the fp64 LayerNorm of the same inputs rounded to the dtype, or
within the error bound of the kernel's fp32 arithmetic where the result
cancels to near zero."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from forgeml_amd import kernels
from forgeml_amd.ir import GraphError
from oracle.fused_linear import ulp_index
from tests.cases import case_seed

pytestmark = pytest.mark.gpu


def _say(*parts):
    print("case:", *parts, flush=True)


def _layer_norm_one_rounding(got, x, w, b, eps, what):
    """got (16-bit) against F.layer_norm's definition in fp64 rounded once."""
    x64 = x.double()
    mean = x64.mean(-1, keepdim=True)
    var = ((x64 - mean) ** 2).mean(-1, keepdim=True)
    xhat = (x64 - mean) / torch.sqrt(var + eps)
    scaled = xhat if w is None else xhat * w.double()
    exact = scaled if b is None else scaled + b.double()
    rounded = exact.to(got.dtype)
    ulps = (ulp_index(got) - ulp_index(rounded)).abs()
    # Where x is within a few fp32 ulps of the mean, x - mean cancels and the
    # fp32 mean's own error (its rounding plus the sum's, up to log2(cols)
    # roundings of mean |x|) dominates: allow the fp32 evaluation bound of
    # (x - mean) * rstd * w + b computed from its terms before cancellation.
    cols = x.shape[-1]
    rstd = 1.0 / torch.sqrt(var + eps)
    w_abs = 1.0 if w is None else w.double().abs()
    spread = x64.abs() + mean.abs() + math.log2(cols) * x64.abs().mean(-1, keepdim=True)
    terms = spread * rstd * w_abs + (0.0 if b is None else b.double().abs())
    near = (got.double() - exact).abs() <= 16 * 2.0 ** -24 * terms
    bad = ~((ulps <= 1) | near)
    assert torch.isfinite(got).all() and int(bad.sum()) == 0, f"{what}: {int(bad.sum())} elements off, max {int(ulps.max())} ulps"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(4096, 768), (8, 512, 768), (7, 100), (3, 5000), (5, 1030), (64, 4096), (6, 16384),
                                   (2, 20000), (2, 40000), (1, 140000), (8, 140000), (3, 200000)])
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
            _layer_norm_one_rounding(got, x, wa, ba, 1e-5, f"layer_norm {shape} {dtype} affine={affine}")


def _attention_inputs(b, h, lq, lk, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, lq, d, generator=g)
    k = torch.randn(b, h, lk, d, generator=g)
    v = torch.randn(b, h, lk, d, generator=g)
    return q, k, v


# Two waves per work item at head dim 96 and 128, and for causal problems of
# at least 1024 query blocks (2x32x512 at dim 64, 8x8x512 at dim 32); four
# otherwise.
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,h,lq,lk,d", [(2, 3, 100, 100, 64), (1, 2, 33, 33, 32), (2, 2, 64, 64, 96),
                                          (1, 4, 512, 512, 64), (2, 1, 40, 70, 64), (1, 1, 1, 1, 64),
                                          (2, 3, 100, 100, 128), (1, 2, 300, 300, 128), (2, 32, 512, 512, 64),
                                          (8, 8, 512, 512, 32), (1, 2, 70, 40, 96)])
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


def test_attention_misaligned_contiguous_inputs(gpu):
    # Contiguous tensors whose storage starts one element past a 16-byte
    # boundary: the boundary copies them into aligned storage.
    b, h, s, d = 1, 2, 40, 64
    q, k, v = _attention_inputs(b, h, s, s, d, case_seed("attn_offset"))
    def shifted(t):
        flat = torch.empty(t.numel() + 1, device=gpu)
        view = flat[1:].view(t.shape)
        view.copy_(t.to(gpu))
        assert view.is_contiguous() and view.data_ptr() % 16 != 0
        return view
    _say("attention misaligned contiguous inputs")
    got = kernels.attention(shifted(q), shifted(k), shifted(v), is_causal=True)
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-5)


def test_attention_broadcast_keys(gpu):
    # K and V broadcast along the sequence (stride 0): rows that overlap are
    # copied out by the boundary before the kernel runs.
    b, h, s, d = 2, 3, 50, 64
    q, k, v = _attention_inputs(b, h, s, 1, d, case_seed("attn_bcast"))
    kx, vx = k.expand(b, h, s, d), v.expand(b, h, s, d)
    _say("attention broadcast keys")
    got = kernels.attention(q.to(gpu), k.to(gpu).expand(b, h, s, d), v.to(gpu).expand(b, h, s, d), is_causal=True)
    expected = F.scaled_dot_product_attention(q, kx, vx, is_causal=True)
    torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lk,d", [(70, 64), (45, 128), (33, 32), (100, 96), (20, 64), (1, 32), (31, 128)])
def test_attention_keys_past_the_end_are_not_read(gpu, causal, lk, d):
    # K and V are views of the first lk rows of buffers whose rows past lk
    # hold NaN: a kernel that read a key past lk (the last 32-key block runs
    # over it when lk is not a multiple of 32) would put a NaN into O, even
    # with that key masked, through 0 * NaN in P V.  lk < 32: one key block.
    b, h, lq = 2, 3, 77
    q, k, v = _attention_inputs(b, h, lq, lk, d, case_seed("attn_tail", lk, d, causal))
    def padded(t):
        buf = torch.full((b, h, lk + 32, d), float("nan"), device=gpu)
        buf[:, :, :lk] = t.to(gpu)
        return buf[:, :, :lk]
    _say("attention keys past the end", lk, d, causal)
    got = kernels.attention(q.to(gpu), padded(k), padded(v), is_causal=causal)
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    assert not got.isnan().any()
    torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-5)


def test_block_kernel_argument_checks(gpu):
    with pytest.raises(GraphError, match="fp32"):
        kernels.attention(*(torch.randn(1, 1, 8, 64, device=gpu, dtype=torch.bfloat16),) * 3)
    with pytest.raises(GraphError, match="not supported"):
        kernels.attention(*(torch.randn(1, 1, 8, 48, device=gpu),) * 3)
    with pytest.raises(GraphError, match="does not end"):
        kernels.layer_norm(torch.randn(4, 8, device=gpu), (16,))


def test_attention_random_problems(gpu):
    """60 seeded random attention problems: batch and heads 1..4, lengths 1..300
    (L_q and L_k independent), every head dim, causal or not, against torch's
    CPU SDPA."""
    g = torch.Generator().manual_seed(case_seed("attn_random"))
    for i in range(60):
        b, h = (int(v) for v in torch.randint(1, 5, (2,), generator=g))
        lq, lk = (int(v) for v in torch.randint(1, 301, (2,), generator=g))
        d = (32, 64, 96, 128)[int(torch.randint(0, 4, (1,), generator=g))]
        causal = bool(torch.randint(0, 2, (1,), generator=g))
        seed = case_seed("attn_random", i)
        q, k, v = _attention_inputs(b, h, lq, lk, d, seed)
        _say("attention random", i, b, h, lq, lk, d, causal, seed)
        expected = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        got = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), is_causal=causal)
        torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-5,
                                   msg=lambda msg: f"attention random #{i} {b}x{h}x{lq}x{lk}x{d} causal={causal}: {msg}")
