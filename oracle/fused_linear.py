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
