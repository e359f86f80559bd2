"""CPU restatements of the fused linear + bias + GELU computation (test only).

See oracle/__init__.py for what may import this module.
"""

from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

ORACLE_DIR = Path(__file__).resolve().parent
BRUTE_LIB = ORACLE_DIR / "liboracle_gemm.so"

ACT_CODES = {("none", "none"): 0, ("gelu", "none"): 1, ("gelu", "tanh"): 2, ("relu", "none"): 3}


def reference_cpu(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None,
                  activation: str = "none", approximate: str = "none") -> torch.Tensor:
    """ForgeML's CPU path on CPU copies of the operands, in their dtype.

    linear: ``addmm(bias, a, b)`` / ``mm(a, b)`` (src/forgeml/ops.py:28-31);
    fused_linear_gelu: the same followed by ``F.gelu(approximate)``
    (src/forgeml/ops.py:48-53).  ``relu`` is ``clamp_min(x, 0)``
    (src/forgeml/compiler.py:103-104).
    """
    a, b = a.detach().cpu(), b.detach().cpu()
    with torch.inference_mode():
        if bias is not None:
            out = torch.addmm(bias.detach().cpu(), a, b)
        else:
            out = torch.mm(a, b)
        if activation == "gelu":
            out = F.gelu(out, approximate=approximate)
        elif activation == "relu":
            out = torch.clamp_min(out, 0)
    return out


def _round(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return x.to(dtype).to(torch.float64)


def kernel_contract(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None,
                    activation: str = "none", approximate: str = "none") -> torch.Tensor:
    """The reference kernel's epilogue order with an fp64 accumulator.

    value = rnd(acc); if bias: value = rnd(value + bias); value = act(value);
    store rounds to the output dtype (src/forgeml/_triton.py:43-62).
    """
    dtype = a.dtype
    a64 = a.detach().cpu().to(torch.float64)
    b64 = b.detach().cpu().to(torch.float64)
    v = _round(a64 @ b64, dtype)
    if bias is not None:
        v = _round(v + bias.detach().cpu().to(torch.float64), dtype)
    # The activation is evaluated in fp32 by the kernel (and by torch for
    # low-precision tensors); evaluate it there too.
    v32 = v.to(torch.float32)
    if activation == "gelu":
        v32 = F.gelu(v32, approximate=approximate)
    elif activation == "relu":
        v32 = torch.clamp_min(v32, 0)
    return v32.to(dtype)


# -- ulp-level check of 16-bit outputs against the epilogue contract -------------

_MANT_BITS = {torch.bfloat16: 7, torch.float16: 10}


def ulp_index(x: torch.Tensor) -> torch.Tensor:
    """16-bit float bit patterns mapped to integers monotone in the value
    (+0 and -0 both 0), so that a difference of ordered values counts ulps."""
    bits = x.contiguous().view(torch.int16).to(torch.int64) & 0xFFFF
    mag = bits & 0x7FFF
    return torch.where(bits >= 0x8000, -mag, mag)


def gelu_f64(x: torch.Tensor, approximate: str = "none") -> torch.Tensor:
    """GELU in fp64 without cancellation for negative x: x/2 erfc(-x/sqrt 2)
    (erf form) and x sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3) (tanh form,
    the identity 0.5 (1 + tanh u) = sigmoid(2u))."""
    x = x.to(torch.float64)
    if approximate == "tanh":
        u = math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)
        return x * torch.sigmoid(2.0 * u)
    return 0.5 * x * torch.special.erfc(-x / math.sqrt(2.0))


def _epilogue_f64(v: torch.Tensor, bias: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor:
    """rnd(v + bias) in fp64 for v already in ``dtype`` (src/forgeml/_triton.py:43-46)."""
    x = v.to(torch.float64)
    if bias is not None:
        x = (x + bias.detach().cpu().to(torch.float64)).to(dtype).to(torch.float64)
    return x


def _activate_f64(x: torch.Tensor, activation: str, approximate: str) -> torch.Tensor:
    if activation == "gelu":
        return gelu_f64(x, approximate)
    if activation == "relu":
        return torch.clamp_min(x, 0)
    return x


def _gelu_argmin(approximate: str) -> float:
    """Where GELU takes its minimum (near -0.75), by ternary search in fp64."""
    lo, hi = -1.5, 0.0
    f = lambda t: float(gelu_f64(torch.tensor([t], dtype=torch.float64), approximate))  # noqa: E731
    for _ in range(200):
        m1, m2 = lo + (hi - lo) / 3, hi - (hi - lo) / 3
        if f(m1) < f(m2):
            hi = m2
        else:
            lo = m1
    return 0.5 * (lo + hi)


_GELU_ARGMIN = {approx: _gelu_argmin(approx) for approx in ("none", "tanh")}


def contract_ulp_check(got: torch.Tensor, a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None,
                       activation: str = "none", approximate: str = "none",
                       acc: torch.Tensor | None = None) -> dict:
    """Ulp-level check of a 16-bit kernel output against the epilogue contract.

    The contract is C = act(rnd(rnd(sum A B) + bias)) (src/forgeml/_triton.py:
    43-57).  The kernel sums the exact products in fp32 in its own order, so
    its sum lies within E = gamma_K sum |A||B| of the exact one (gamma_K =
    K u / (1 - K u), u = 2^-24: the bound for any summation order).  Each
    element's sum is therefore known to an interval [S - E, S + E]; rnd, the
    bias add and the next rnd are monotone, so the pre-activation lies in
    [x_lo, x_hi], and the output must lie within one ulp of act over that
    range (the activation evaluated exactly; GELU's minimum near -0.75 is
    included when the range spans it), or within the dtype's smallest
    normal of it, for results the fp32 arithmetic flushes.  Where the sum
    does not cancel, E is under about one ulp, so the range is one or two
    values wide.

    Reported: ``bad`` (elements outside), ``exact_frac`` (elements equal to
    act(rnd(rnd(S) + bias)) from the exact sum S) and ``max_ulp`` (the
    largest distance outside the range).  A test requires bad == 0 and
    exact_frac >= 0.99: a wrong activation form, a skipped rounding step or
    a truncating conversion moves far more than 1 % of the elements.
    ``acc``: the fp64 sum S, when the caller already has it.
    """
    dtype = got.dtype
    if dtype not in _MANT_BITS:
        raise ValueError(f"contract_ulp_check is for 16-bit outputs, got {dtype}")
    got = got.detach().cpu()
    a64 = a.detach().cpu().to(torch.float64)
    b64 = b.detach().cpu().to(torch.float64)
    if acc is None:
        acc = a64 @ b64
    k = a64.shape[1]
    u = 2.0 ** -24
    err = (k * u / (1 - k * u)) * (a64.abs() @ b64.abs())
    x_lo = _epilogue_f64((acc - err).to(dtype), bias, dtype)
    x_hi = _epilogue_f64((acc + err).to(dtype), bias, dtype)
    y_lo = _activate_f64(x_lo, activation, approximate)
    y_hi = _activate_f64(x_hi, activation, approximate)
    low, high = torch.minimum(y_lo, y_hi), torch.maximum(y_lo, y_hi)
    if activation == "gelu":
        t = _GELU_ARGMIN[approximate]
        spans = (x_lo <= t) & (t <= x_hi)
        low = torch.where(spans, torch.minimum(low, gelu_f64(torch.tensor(t, dtype=torch.float64), approximate)), low)
    low, high = low.to(dtype), high.to(dtype)
    og = ulp_index(got)
    below = (ulp_index(low) - og).clamp_min(0)
    above = (og - ulp_index(high)).clamp_min(0)
    outside = torch.maximum(below, above)
    tiny = torch.finfo(dtype).tiny
    g64 = got.to(torch.float64)
    flushed = ((g64 - low.to(torch.float64)).abs() <= tiny) | ((g64 - high.to(torch.float64)).abs() <= tiny)
    ok = torch.isfinite(got) & ((outside <= 1) | flushed)
    primary = _activate_f64(_epilogue_f64(acc.to(dtype), bias, dtype), activation, approximate).to(dtype)
    return {
        "n": got.numel(),
        "bad": int((~ok).sum()),
        "exact_frac": float((got == primary).double().mean()) if got.numel() else 1.0,
        "max_ulp": int(outside.max()) if got.numel() else 0,
    }


def _brute_lib() -> ctypes.CDLL:
    if not BRUTE_LIB.exists():
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    lib = ctypes.CDLL(str(BRUTE_LIB))
    i64, p = ctypes.c_int64, ctypes.c_void_p
    lib.oracle_fused_linear_f64.argtypes = [p, i64, i64, p, i64, i64, p, i64, p, i64, i64, i64, ctypes.c_int]
    lib.oracle_fused_linear_f64.restype = ctypes.c_int
    lib.oracle_act_f64.argtypes = [ctypes.c_double, ctypes.c_int]
    lib.oracle_act_f64.restype = ctypes.c_double
    return lib


def brute_force(a: np.ndarray, b: np.ndarray, bias: np.ndarray | None = None,
                activation: str = "none", approximate: str = "none") -> np.ndarray:
    """fp64 triple loop in C; operands may be strided numpy views."""
    lib = _brute_lib()
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError("inner dimensions differ")
    out = np.empty((m, n), dtype=np.float64)
    bias_ptr, sbi = None, 0
    if bias is not None:
        bias = np.asarray(bias, dtype=np.float64)
        bias_ptr, sbi = bias.ctypes.data, bias.strides[0] // 8
    rc = lib.oracle_fused_linear_f64(
        a.ctypes.data, a.strides[0] // 8, a.strides[1] // 8,
        b.ctypes.data, b.strides[0] // 8, b.strides[1] // 8,
        bias_ptr, sbi, out.ctypes.data, m, n, k, ACT_CODES[(activation, approximate)],
    )
    if rc != 0:
        raise ValueError("oracle_fused_linear_f64 rejected its arguments")
    return out


def act_scalar(x: float, activation: str = "gelu", approximate: str = "none") -> float:
    return _brute_lib().oracle_act_f64(float(x), ACT_CODES[(activation, approximate)])


def tolerance(dtype: torch.dtype, k: int) -> tuple[float, float]:
    """(rtol, atol) of the parity gate.

    fp32: rtol 1e-4, atol 1e-5*sqrt(K); bf16: rtol 2e-2 with the reference's
    bf16 atol 5e-2 (src/forgeml/measurement.py:84-85); fp16: the reference
    tests' 1e-2/1e-2 (tests/test_kernels.py:31-35).
    """
    if dtype == torch.float32:
        return 1e-4, 1e-5 * math.sqrt(k)
    if dtype == torch.bfloat16:
        return 2e-2, 5e-2
    if dtype == torch.float16:
        return 1e-2, 1e-2
    raise ValueError(f"no tolerance for {dtype}")
