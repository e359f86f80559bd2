"""Torch evaluation of every IR op.

This is the executor's ``"torch"`` backend and the meta-tensor shape engine
behind ``infer_spec``; it has the semantics of ForgeML's ``ops.evaluate``
(src/forgeml/ops.py:25-83).  On a GPU graph it runs on PyTorch-ROCm.  GEMM
nodes planned for the ``"hip"`` backend never come here: they go to the
gfx950 kernels through ``forgeml_amd.kernels.matmul``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from forgeml_amd.ir import SUPPORTED_OPS

__all__ = ["SUPPORTED_OPS", "evaluate"]


def _linear(args: tuple[torch.Tensor, ...]) -> torch.Tensor:
    if len(args) == 3:
        return torch.addmm(args[2], args[0], args[1])
    return torch.mm(args[0], args[1])


def _layer_norm(args, attrs):
    normalized = attrs["normalized_shape"]
    if isinstance(normalized, int):
        normalized = (normalized,)
    weight, bias = (args[1], args[2]) if len(args) == 3 else (None, None)
    return F.layer_norm(args[0], tuple(normalized), weight, bias, attrs["eps"])


def _sdpa(args, attrs):
    return F.scaled_dot_product_attention(
        args[0],
        args[1],
        args[2],
        attn_mask=args[3] if len(args) == 4 else None,
        dropout_p=0.0,
        is_causal=attrs["is_causal"],
        scale=attrs.get("scale"),
    )


def _conv2d(args, attrs):
    return F.conv2d(
        args[0],
        args[1],
        args[2] if len(args) == 3 else None,
        stride=attrs["stride"],
        padding=attrs["padding"],
        dilation=attrs["dilation"],
        groups=attrs["groups"],
    )


_EVAL = {
    "matmul": lambda args, attrs: torch.matmul(args[0], args[1]),
    "linear": lambda args, attrs: _linear(args),
    "add": lambda args, attrs: torch.add(args[0], args[1]),
    "mul": lambda args, attrs: torch.mul(args[0], args[1]),
    "relu": lambda args, attrs: F.relu(args[0]),
    "gelu": lambda args, attrs: F.gelu(args[0], approximate=attrs.get("approximate", "none")),
    "reshape": lambda args, attrs: torch.reshape(args[0], tuple(attrs["shape"])),
    "transpose": lambda args, attrs: torch.transpose(args[0], attrs["dim0"], attrs["dim1"]),
    "softmax": lambda args, attrs: torch.softmax(args[0], dim=attrs["dim"]),
    "narrow": lambda args, attrs: torch.narrow(
        args[0], attrs["dim"] % args[0].dim(), attrs["start"], attrs["length"]
    ),
    "fused_linear_gelu": lambda args, attrs: F.gelu(
        _linear(args), approximate=attrs.get("approximate", "none")
    ),
    "layer_norm": _layer_norm,
    "sdpa": _sdpa,
    "conv2d": _conv2d,
    "embedding": lambda args, attrs: F.embedding(args[0], args[1]),
}
assert set(_EVAL) == set(SUPPORTED_OPS)


def evaluate(op: str, args: tuple[torch.Tensor, ...], attrs: dict) -> torch.Tensor:
    fn = _EVAL.get(op)
    if fn is None:
        raise ValueError(f"unsupported op {op!r}")
    return fn(args, attrs)
