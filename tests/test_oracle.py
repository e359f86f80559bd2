"""Pins the oracle (ForgeML's CPU path restated) before it is trusted.

Checks, each chosen so a plausible restatement mistake fails one of them:
* the fp64 C brute force and the torch restatement agree on non-square,
  strided cases for every epilogue (catches transposed operands, dropped
  bias, wrong activation);
* GELU known values from the standard normal CDF table and the identity
  gelu(x) - gelu(-x) = x (catches sign and scale errors);
* closed forms: A = 0 gives act(bias), B = I gives act(A + bias), K = 1 is an
  outer product;
* the bf16 rounding contract is round-to-nearest-even at exact ties;
* the reference tests' own expected-value formula for bias + GELU
  (tests/test_kernels.py:124-126) equals the kernel contract;
* committed golden vectors (tests/golden/fused_linear_small.npz).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.fused_linear import act_scalar, brute_force, kernel_contract, reference_cpu, tolerance

GOLDEN = Path(__file__).resolve().parent / "golden" / "fused_linear_small.npz"

_EPILOGUES = [("none", "none"), ("gelu", "none"), ("gelu", "tanh"), ("relu", "none")]


@pytest.mark.parametrize("activation,approximate", _EPILOGUES)
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("m,n,k", [(1, 5, 3), (7, 3, 11), (33, 17, 9)])
def test_brute_force_matches_torch_restatement(m, n, k, with_bias, activation, approximate):
    rng = np.random.default_rng(m * 1000 + n * 10 + k)
    a = rng.standard_normal((m, k))
    w = rng.standard_normal((n, k))
    bias = rng.uniform(-1, 1, n) if with_bias else None
    c = brute_force(a, w.T, bias, activation, approximate)  # B = W^T: strided view
    t = reference_cpu(
        torch.from_numpy(a), torch.from_numpy(w).t(), None if bias is None else torch.from_numpy(bias),
        activation, approximate,
    )
    assert t.dtype == torch.float64
    np.testing.assert_allclose(t.numpy(), c, rtol=1e-12, atol=1e-12)


def test_gelu_known_values():
    # x * Phi(x) with Phi from the standard normal table.
    phi = {-2.0: 0.022750131948179195, -1.0: 0.15865525393145707, -0.5: 0.3085375387259869,
           0.5: 0.6914624612740131, 1.0: 0.8413447460685429, 2.0: 0.9772498680518208}
    for x, p in phi.items():
        assert act_scalar(x) == pytest.approx(x * p, rel=1e-14, abs=1e-15)
        got = reference_cpu(torch.tensor([[x]], dtype=torch.float64), torch.ones(1, 1, dtype=torch.float64),
                            None, "gelu", "none")
        assert got.item() == pytest.approx(x * p, rel=1e-14, abs=1e-15)
    assert act_scalar(0.0) == 0.0 and act_scalar(0.0, "gelu", "tanh") == 0.0


def test_gelu_odd_part_identity_and_tanh_closeness():
    xs = np.linspace(-6, 6, 241)
    for approx in ("none", "tanh"):
        diff = np.array([act_scalar(x, "gelu", approx) - act_scalar(-x, "gelu", approx) for x in xs])
        np.testing.assert_allclose(diff, xs, atol=1e-12)
    gap = max(abs(act_scalar(x, "gelu", "tanh") - act_scalar(x)) for x in xs)
    assert 1e-5 < gap < 1e-3  # the tanh form is a close but distinct approximation


def test_closed_forms():
    rng = np.random.default_rng(7)
    m, n, k = 6, 9, 5
    bias = rng.uniform(-1, 1, n)
    zero_a = np.zeros((m, k))
    b = rng.standard_normal((k, n))
    for act, approx in _EPILOGUES:
        c = brute_force(zero_a, b, bias, act, approx)
        expected = np.array([act_scalar(v, act, approx) for v in bias])
        np.testing.assert_allclose(c, np.broadcast_to(expected, (m, n)), atol=1e-15)
    a = rng.standard_normal((m, n))
    c = brute_force(a, np.eye(n), bias, "gelu", "none")
    np.testing.assert_allclose(c, np.vectorize(act_scalar)(a + bias), atol=1e-14)
    u, v = rng.standard_normal((m, 1)), rng.standard_normal((1, n))
    np.testing.assert_allclose(brute_force(u, v), u * v, atol=1e-15)


def test_bf16_rounding_contract_is_rne():
    one = torch.ones(1, 1, dtype=torch.bfloat16)
    cases = {
        2.0 ** -8: 1.0,                  # tie between 1 and 1+2^-7: to even (1.0)
        3 * 2.0 ** -8: 1.0 + 2.0 ** -6,  # tie between 1+2^-7 and 1+2^-6: to even
        2.0 ** -9: 1.0,                  # below half an ulp
        2.0 ** -8 + 2.0 ** -12: 1.0 + 2.0 ** -7,  # above the tie
    }
    for frac, expected in cases.items():
        # acc = 1*1 + 1*frac, exactly representable in fp64
        a = torch.tensor([[1.0, 1.0]], dtype=torch.float64).to(torch.bfloat16)
        b_vals = torch.tensor([[1.0], [frac]], dtype=torch.float64)
        # b must hold frac exactly in bf16; all chosen fractions are powers of two or sums of two.
        b = b_vals.to(torch.bfloat16)
        assert b.double()[1, 0].item() == frac
        got = kernel_contract(a, b)
        assert got.dtype == torch.bfloat16 and got.double().item() == expected
    del one


def test_reference_test_formula_equals_contract():
    # tests/test_kernels.py:124-126 expects gelu((a.float() @ b.float()).to(dtype) + bias)
    g = torch.Generator().manual_seed(3)
    for dtype in (torch.bfloat16, torch.float16):
        a = torch.randn(16, 32, generator=g).to(dtype)
        b = torch.randn(32, 24, generator=g).to(dtype)
        bias = torch.randn(24, generator=g).to(dtype)
        for approx in ("none", "tanh"):
            formula = F.gelu((a.float() @ b.float()).to(dtype) + bias, approximate=approx)
            contract = kernel_contract(a, b, bias, "gelu", approx)
            # fp32 vs fp64 accumulation may land on either side of a rounding
            # boundary: allow one ulp of the dtype.
            ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
            diff = (formula.double() - contract.double()).abs()
            assert (diff <= ulp * contract.double().abs().clamp_min(1.0)).all()
            assert (diff == 0).float().mean() > 0.95


def test_golden_vectors():
    data = np.load(GOLDEN, allow_pickle=False)
    names = sorted({key.split("/")[0] for key in data.files})
    assert len(names) >= 6
    for name in names:
        act = "relu" if name.startswith("relu") else ("gelu" if "gelu" in name else "none")
        approx = "tanh" if "tanh" in name else "none"
        a, w = data[f"{name}/a"], data[f"{name}/w"]
        bias = data[f"{name}/bias"] if f"{name}/bias" in data.files else None
        expected = data[f"{name}/expected"]
        np.testing.assert_array_equal(brute_force(a, w.T, bias, act, approx), expected)
        got = reference_cpu(torch.from_numpy(a), torch.from_numpy(w).t(),
                            None if bias is None else torch.from_numpy(bias), act, approx)
        np.testing.assert_allclose(got.numpy(), expected, rtol=1e-12, atol=1e-12)
        # fp32 run of the CPU path passes the fp32 gate against the fp64 vectors.
        got32 = reference_cpu(torch.from_numpy(a).float(), torch.from_numpy(w).float().t(),
                              None if bias is None else torch.from_numpy(bias).float(), act, approx)
        rtol, atol = tolerance(torch.float32, a.shape[1])
        np.testing.assert_allclose(got32.double().numpy(), expected, rtol=rtol, atol=atol)


def test_tolerances():
    assert tolerance(torch.float32, 4096) == (1e-4, pytest.approx(6.4e-4))
    assert tolerance(torch.bfloat16, 14336) == (2e-2, 5e-2)
    with pytest.raises(ValueError):
        tolerance(torch.int32, 4)


# -- the ulp-level contract check for 16-bit outputs ---------------------------
#
# A faithful CPU model of the kernels' 16-bit epilogue (fp32 sums in another
# order, one rounding, fp32 bias add and rounding, the relative-accurate fp32
# GELU forms) must pass contract_ulp_check; the same model with one mistake
# planted must fail it.  The models live here, on the CPU, only to pin the
# checker.

_NR_ERFC = (0.17087277, -0.82215223, 1.48851587, -1.13520398, 0.27886807, -0.18628806, 0.09678418,
            0.37409196, 1.00002368, -1.26551223)


def _phi_neg_chebyshev(x: np.ndarray) -> np.ndarray:
    """Phi(-|x|) in fp32 from the Chebyshev erfc fit of Numerical Recipes 6.2."""
    z = np.abs(x).astype(np.float32) * np.float32(0.7071067811865476)
    t = np.float32(1) / (np.float32(1) + np.float32(0.5) * z)
    p = np.float32(_NR_ERFC[0])
    for c in _NR_ERFC[1:]:
        p = (p * t + np.float32(c)).astype(np.float32)
    return (np.float32(0.5) * t * np.exp(-z * z + p)).astype(np.float32)


def _phi_neg_as7126(x: np.ndarray) -> np.ndarray:
    """Phi(-|x|) from Abramowitz & Stegun 7.1.26 (absolute error 1.5e-7)."""
    z = np.abs(x).astype(np.float32) * np.float32(0.7071067811865476)
    t = np.float32(1) / (np.float32(1) + np.float32(0.3275911) * z)
    poly = ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592)
    return (0.5 * poly * t * np.exp(-z * z)).astype(np.float32)


def _model_16bit(a, b, bias, approximate, *, form=None, skip_round=False, truncate=False):
    dtype = a.dtype
    acc = a.float() @ b.float()
    if truncate:
        v = (acc.view(torch.int32) & ~0xFFFF).view(torch.float32) if dtype == torch.bfloat16 else acc.to(dtype).float()
    elif skip_round:
        v = acc
    else:
        v = acc.to(dtype).float()
    if bias is not None:
        v = (v + bias.float()).to(dtype).float()
    x = v.numpy().astype(np.float32)
    form = form or ("tanh" if approximate == "tanh" else "chebyshev")
    if form == "tanh":
        u = np.float32(0.7978845608028654) * (x + np.float32(0.044715) * x * x * x)
        y = x / (np.float32(1) + np.exp(np.float32(-2) * u))
    else:
        q = _phi_neg_chebyshev(x) if form == "chebyshev" else _phi_neg_as7126(x)
        y = x * np.where(x >= 0, np.float32(1) - q, q)
    return torch.from_numpy(y.astype(np.float32)).to(dtype)


def _contract_inputs(dtype, tail: bool):
    if tail:
        # Pre-activations spanning the GELU tail: C = A[:, 0] exactly (K = 2, B selects column 0).
        vals = torch.linspace(-10.0, 4.0, 3001)
        a = torch.stack([vals, torch.zeros_like(vals)], 1).to(dtype)
        b = torch.zeros(2, 8)
        b[0] = 1.0
        return a, b.to(dtype), None
    g = torch.Generator().manual_seed(11)
    k = 1024
    a = (torch.randn(200, k, generator=g) * k ** -0.25).to(dtype)
    b = (torch.randn(k, 96, generator=g) * k ** -0.25).to(dtype)
    bias = (torch.rand(96, generator=g) * 0.2 - 0.1).to(dtype)
    return a, b, bias


def _passes(report) -> bool:
    return report["bad"] == 0 and report["exact_frac"] >= 0.99


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("approximate", ["none", "tanh"])
@pytest.mark.parametrize("tail", [False, True])
def test_contract_check_accepts_the_faithful_model(dtype, approximate, tail):
    from oracle.fused_linear import contract_ulp_check

    a, b, bias = _contract_inputs(dtype, tail)
    report = contract_ulp_check(_model_16bit(a, b, bias, approximate), a, b, bias, "gelu", approximate)
    assert _passes(report), report


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mistake", ["tanh_for_erf", "as7126_gelu", "skip_first_round", "truncate"])
def test_contract_check_rejects_planted_mistakes(dtype, mistake):
    from oracle.fused_linear import contract_ulp_check

    if mistake == "truncate" and dtype == torch.float16:
        pytest.skip("the truncating conversion is modelled for bf16 only")
    tail = mistake == "as7126_gelu"  # the absolute-error fit only shows in the tail
    a, b, bias = _contract_inputs(dtype, tail)
    kw = {"tanh_for_erf": {"form": "tanh"}, "as7126_gelu": {"form": "as7126"},
          "skip_first_round": {"skip_round": True}, "truncate": {"truncate": True}}[mistake]
    report = contract_ulp_check(_model_16bit(a, b, bias, "none", **kw), a, b, bias, "gelu", "none")
    assert not _passes(report), report


def test_gelu_f64_is_exact_in_the_tail():
    from oracle.fused_linear import gelu_f64

    # x Phi(x) at table values of the normal CDF, including far tails.
    phi = {-8.0: 6.22096057427178e-16, -5.0: 2.866515718791939e-07, -3.0: 0.0013498980316300946,
           1.0: 0.8413447460685429}
    for x, p in phi.items():
        got = gelu_f64(torch.tensor([x], dtype=torch.float64)).item()
        assert got == pytest.approx(x * p, rel=1e-13)
    xs = torch.linspace(-12, 12, 97, dtype=torch.float64)
    tanh_form = gelu_f64(xs, "tanh")
    u = math.sqrt(2 / math.pi) * (xs + 0.044715 * xs ** 3)
    direct = 0.5 * xs * (1 + torch.tanh(u))
    mask = xs > -3  # where the direct form does not cancel
    torch.testing.assert_close(tanh_form[mask], direct[mask], rtol=1e-13, atol=1e-15)
