"""Static-shape graph IR: tensor specs, nodes, graphs and a checked builder.

Semantics follow ForgeML's IR (src/forgeml/ir.py) so that graphs, specs and
errors are interchangeable with the reference's:

* ``TensorSpec`` (ir.py:29-66) holds static positive dims, a supported dtype
  and a device string; an index-less ``"cuda"`` is canonicalised to
  ``"cuda:0"`` (on ROCm torch, ``cuda`` devices are the HIP GPUs).
* ``infer_spec`` (ir.py:148-383) checks arity, attributes and per-op rules,
  then derives the output spec by running the op on meta tensors.
* ``Graph.validate`` (ir.py:406-454) re-infers every node's spec in order.
* ``GraphBuilder`` (ir.py:513-571) snapshots constants and infers specs as
  nodes are added.
"""

from __future__ import annotations

import copy
import math
from dataclasses import dataclass
from typing import Any

import torch


class GraphError(ValueError):
    """Invalid graph, op, argument or kernel request (a ``ValueError``, ir.py:11)."""


SUPPORTED_DTYPES = frozenset(
    {
        torch.float16,
        torch.bfloat16,
        torch.float32,
        torch.float64,
        torch.int8,
        torch.int16,
        torch.int32,
        torch.int64,
        torch.uint8,
        torch.bool,
    }
)


def _is_int(v: Any) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _is_number(v: Any) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


@dataclass(frozen=True)
class TensorSpec:
    shape: tuple[int, ...]
    dtype: torch.dtype
    device: str

    def __post_init__(self) -> None:
        if not isinstance(self.shape, tuple) or not all(_is_int(d) for d in self.shape):
            raise GraphError(f"shape must be a tuple of ints, got {self.shape!r}")
        if any(d <= 0 for d in self.shape):
            raise GraphError(f"shape dims must be positive integers, got {self.shape!r}")
        if not isinstance(self.dtype, torch.dtype):
            raise GraphError(f"dtype must be a torch.dtype, got {self.dtype!r}")
        if self.dtype not in SUPPORTED_DTYPES:
            raise GraphError(f"unsupported dtype {self.dtype}")
        if not isinstance(self.device, str) or not self.device:
            raise GraphError(f"device must be a non-empty string, got {self.device!r}")
        try:
            parsed = torch.device(self.device)
        except (RuntimeError, TypeError) as e:
            raise GraphError(f"invalid device {self.device!r}") from e
        if parsed.type == "cuda" and parsed.index is None:
            # "cuda" and "cuda:0" must compare equal wherever specs meet.
            object.__setattr__(self, "device", "cuda:0")

    @property
    def nbytes(self) -> int:
        return math.prod(self.shape) * self.dtype.itemsize

    def to_dict(self) -> dict:
        return {
            "shape": list(self.shape),
            "dtype": str(self.dtype).replace("torch.", ""),
            "device": self.device,
        }


@dataclass(frozen=True)
class Node:
    name: str
    op: str
    inputs: tuple[str, ...]
    attrs: dict[str, Any]
    spec: TensorSpec


def spec_of(t: torch.Tensor, device: str | None = None) -> TensorSpec:
    return TensorSpec(tuple(t.shape), t.dtype, device or str(t.device))


# op -> (allowed attrs, required attrs, accepted input counts)
_OP_SIGNATURES: dict[str, tuple[frozenset, frozenset, tuple[int, ...]]] = {
    "matmul": (frozenset(), frozenset(), (2,)),
    "linear": (frozenset(), frozenset(), (2, 3)),
    "add": (frozenset(), frozenset(), (2,)),
    "mul": (frozenset(), frozenset(), (2,)),
    "relu": (frozenset(), frozenset(), (1,)),
    "gelu": (frozenset({"approximate"}), frozenset(), (1,)),
    "reshape": (frozenset({"shape"}), frozenset({"shape"}), (1,)),
    "transpose": (frozenset({"dim0", "dim1"}), frozenset({"dim0", "dim1"}), (1,)),
    "softmax": (frozenset({"dim"}), frozenset({"dim"}), (1,)),
    "narrow": (frozenset({"dim", "start", "length"}), frozenset({"dim", "start", "length"}), (1,)),
    "fused_linear_gelu": (frozenset({"approximate"}), frozenset(), (2, 3)),
    "layer_norm": (frozenset({"normalized_shape", "eps"}), frozenset({"normalized_shape", "eps"}), (1, 3)),
    "sdpa": (frozenset({"is_causal", "scale"}), frozenset({"is_causal"}), (3, 4)),
    "conv2d": (
        frozenset({"stride", "padding", "dilation", "groups"}),
        frozenset({"stride", "padding", "dilation", "groups"}),
        (2, 3),
    ),
    "embedding": (frozenset(), frozenset(), (2,)),
}

SUPPORTED_OPS = frozenset(_OP_SIGNATURES)

_FLOAT_ONLY_OPS = frozenset({"gelu", "softmax", "fused_linear_gelu", "layer_norm", "sdpa", "conv2d"})


def _check_signature(op: str, attrs: dict[str, Any], n_inputs: int) -> None:
    if op not in _OP_SIGNATURES:
        raise GraphError(f"unsupported op {op!r}")
    if not isinstance(attrs, dict):
        raise GraphError(f"op {op!r} attrs must be a dict, got {type(attrs).__name__}")
    allowed, required, arity = _OP_SIGNATURES[op]
    extra = set(attrs) - allowed
    if extra:
        raise GraphError(f"op {op!r} got unsupported attrs {sorted(extra)}")
    missing = required - set(attrs)
    if missing:
        raise GraphError(f"op {op!r} requires attrs {sorted(missing)}")
    if n_inputs not in arity:
        choices = "/".join(str(v) for v in arity)
        raise GraphError(f"op {op!r} expects {choices} inputs, got {n_inputs}")


def _check_pair(value: Any, name: str, *, positive: bool) -> None:
    if _is_int(value):
        pair = (value, value)
    elif isinstance(value, (tuple, list)) and len(value) == 2 and all(_is_int(v) for v in value):
        pair = tuple(value)
    else:
        raise GraphError(f"conv2d {name} must be an int or pair of ints, got {value!r}")
    lo = 1 if positive else 0
    if any(v < lo for v in pair):
        kind = "positive" if positive else "non-negative"
        raise GraphError(f"conv2d {name} values must be {kind}, got {pair!r}")


def _check_gemm_like(op: str, specs: list[TensorSpec]) -> None:
    a, b = specs[:2]
    if op == "fused_linear_gelu":
        if len(a.shape) != 2 or len(b.shape) != 2:
            raise GraphError("fused_linear_gelu requires rank-2 matmul inputs")
        if a.shape[1] != b.shape[0]:
            raise GraphError("fused_linear_gelu shape mismatch")
        if len(specs) == 3:
            bias = specs[2]
            if len(bias.shape) != 1 or bias.shape[0] != b.shape[1]:
                raise GraphError("fused_linear_gelu bias must be a 1-D output-width tensor")
            if bias.dtype != a.dtype:
                raise GraphError("fused_linear_gelu bias dtype mismatch")
        if a.dtype != b.dtype:
            raise GraphError("fused_linear_gelu dtype mismatch")
        return
    what = "input and weight tensors" if op == "linear" else "inputs"
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise GraphError(f"{op} requires rank-2 {what}")
    if a.dtype != b.dtype:
        raise GraphError(f"{op} dtype mismatch {a.dtype} vs {b.dtype}")
    if a.dtype == torch.bool:
        raise GraphError(f"{op} does not support bool inputs")
    if a.shape[1] != b.shape[0]:
        raise GraphError(f"{op} shape mismatch {a.shape} x {b.shape}")
    if op == "linear" and len(specs) == 3:
        bias = specs[2]
        if len(bias.shape) != 1 or bias.shape[0] != b.shape[1]:
            raise GraphError("linear bias must be a 1-D tensor of output width")
        if bias.dtype != a.dtype:
            raise GraphError("linear bias dtype mismatch")


def _check_dim(value: Any, rank: int, what: str) -> None:
    if not _is_int(value) or not -rank <= value < rank:
        raise GraphError(f"{what}={value!r} out of range for rank {rank}")


def _check_op_rules(op: str, specs: list[TensorSpec], attrs: dict[str, Any]) -> None:
    if op in ("matmul", "linear", "fused_linear_gelu"):
        _check_gemm_like(op, specs)
        if op == "fused_linear_gelu" and attrs.get("approximate", "none") not in ("none", "tanh"):
            raise GraphError("fused_linear_gelu approximate must be 'none' or 'tanh'")
    elif op in ("add", "mul"):
        x, y = specs
        if x.dtype != y.dtype and x.shape != () and y.shape != ():
            raise GraphError(f"{op} dtype mismatch")
    elif op == "gelu":
        if attrs.get("approximate", "none") not in ("none", "tanh"):
            raise GraphError("gelu approximate must be 'none' or 'tanh'")
    elif op == "reshape":
        shape = attrs["shape"]
        if not isinstance(shape, (tuple, list)) or not all(_is_int(d) and d > 0 for d in shape):
            raise GraphError(f"reshape shape must be positive ints, got {shape!r}")
        if math.prod(shape) != math.prod(specs[0].shape):
            raise GraphError(f"reshape numel mismatch {specs[0].shape} -> {tuple(shape)}")
    elif op == "transpose":
        rank = len(specs[0].shape)
        for key in ("dim0", "dim1"):
            _check_dim(attrs[key], rank, f"transpose {key}")
    elif op == "softmax":
        _check_dim(attrs["dim"], len(specs[0].shape), "softmax dim")
    elif op == "narrow":
        x = specs[0]
        rank = len(x.shape)
        for key in ("dim", "start", "length"):
            if not _is_int(attrs[key]):
                raise GraphError(f"narrow {key} must be an int, got {attrs[key]!r}")
        if rank == 0 or not -rank <= attrs["dim"] < rank:
            raise GraphError(f"narrow dim={attrs['dim']!r} out of range for rank {rank}")
        dim = attrs["dim"] % rank
        start, length = attrs["start"], attrs["length"]
        if length <= 0 or start < 0 or start + length > x.shape[dim]:
            raise GraphError(
                f"narrow range start={start} length={length} exceeds dim {dim} of size {x.shape[dim]}"
            )
    elif op == "layer_norm":
        x = specs[0]
        normalized = attrs["normalized_shape"]
        if _is_int(normalized):
            normalized = (normalized,)
        if (
            not isinstance(normalized, (tuple, list))
            or not normalized
            or not all(_is_int(d) and d > 0 for d in normalized)
        ):
            raise GraphError(f"layer_norm normalized_shape must be positive ints, got {normalized!r}")
        normalized = tuple(normalized)
        if len(x.shape) < len(normalized) or x.shape[-len(normalized):] != normalized:
            raise GraphError(f"layer_norm shape {x.shape} does not end with {normalized!r}")
        if len(specs) == 3:
            w, b = specs[1:]
            if w.shape != normalized or b.shape != normalized:
                raise GraphError("layer_norm weight/bias must match normalized_shape")
            if not (x.dtype == w.dtype == b.dtype):
                raise GraphError("layer_norm dtype mismatch")
        eps = attrs["eps"]
        if not _is_number(eps) or not math.isfinite(float(eps)) or float(eps) <= 0:
            raise GraphError("layer_norm eps must be a finite positive number")
    elif op == "sdpa":
        q, k, v = specs[:3]
        if not (len(q.shape) == len(k.shape) == len(v.shape) == 4):
            raise GraphError("sdpa requires rank-4 [batch, heads, sequence, dim] tensors")
        if q.shape[0:2] != k.shape[0:2] or k.shape != v.shape or q.shape[3] != k.shape[3]:
            raise GraphError("sdpa batch/head/key-value shapes are incompatible")
        if not (q.dtype == k.dtype == v.dtype):
            raise GraphError("sdpa dtype mismatch")
        if not isinstance(attrs["is_causal"], bool):
            raise GraphError("sdpa is_causal must be a bool")
        if len(specs) == 4:
            mask = specs[3]
            if attrs["is_causal"]:
                raise GraphError("sdpa attn_mask cannot be combined with is_causal")
            if mask.dtype != torch.bool and mask.dtype != q.dtype:
                raise GraphError("sdpa attn_mask must be bool or match the query dtype")
            target = (q.shape[0], q.shape[1], q.shape[2], k.shape[2])
            try:
                merged = torch.broadcast_shapes(mask.shape, target)
            except RuntimeError as e:
                raise GraphError(f"sdpa attn_mask shape {mask.shape} cannot broadcast to {target}") from e
            if merged != target:
                raise GraphError(f"sdpa attn_mask shape {mask.shape} cannot broadcast to {target}")
        scale = attrs.get("scale")
        if scale is not None and (not _is_number(scale) or not math.isfinite(float(scale)) or float(scale) <= 0):
            raise GraphError("sdpa scale must be a finite positive number or None")
    elif op == "conv2d":
        x, w = specs[:2]
        if len(x.shape) != 4 or len(w.shape) != 4:
            raise GraphError("conv2d requires NCHW input and OIHW weight tensors")
        groups = attrs["groups"]
        if not _is_int(groups) or groups <= 0:
            raise GraphError("conv2d groups must be a positive integer")
        if x.shape[1] % groups or w.shape[0] % groups or x.shape[1] != w.shape[1] * groups:
            raise GraphError("conv2d channels/groups are incompatible")
        if len(specs) == 3:
            bias = specs[2]
            if len(bias.shape) != 1 or bias.shape[0] != w.shape[0]:
                raise GraphError("conv2d bias must be a 1-D tensor of output channels")
            if bias.dtype != x.dtype:
                raise GraphError("conv2d bias dtype mismatch")
        if x.dtype != w.dtype:
            raise GraphError("conv2d dtype mismatch")
        _check_pair(attrs["stride"], "stride", positive=True)
        _check_pair(attrs["padding"], "padding", positive=False)
        _check_pair(attrs["dilation"], "dilation", positive=True)
    elif op == "embedding":
        idx, w = specs
        if idx.dtype != torch.int64:
            raise GraphError("embedding indices must be int64")
        if len(w.shape) != 2:
            raise GraphError("embedding weight must be rank-2 [vocab, dim]")


def _result_device(op: str, specs: list[TensorSpec]) -> str:
    # A scalar (rank-0) operand may live on the CPU next to a device tensor;
    # the result lives where the non-scalar operands are (ir.py:373-382).
    if op in ("add", "mul") and all(len(s.shape) == 0 for s in specs):
        for s in specs:
            if torch.device(s.device).type != "cpu":
                return s.device
        return specs[0].device
    for s in specs:
        if len(s.shape) > 0:
            return s.device
    return specs[0].device


def infer_spec(op: str, input_specs: list[TensorSpec], attrs: dict[str, Any]) -> TensorSpec:
    """Validate one op application and return its output spec."""
    from forgeml_amd.ops import evaluate

    _check_signature(op, attrs, len(input_specs))
    if op in _FLOAT_ONLY_OPS:
        # sdpa's optional mask may be boolean; the q/k/v operands may not.
        gated = input_specs[:3] if op == "sdpa" else input_specs
        if any(not s.dtype.is_floating_point for s in gated):
            raise GraphError(f"op {op!r} requires floating-point inputs")
    _check_op_rules(op, input_specs, attrs)
    devices = {s.device for s in input_specs}
    if len(devices) > 1:
        scalar_ok = op in ("add", "mul") and any(
            s.shape == () and torch.device(s.device).type == "cpu" for s in input_specs
        )
        if not scalar_ok:
            raise GraphError(f"{op} device mismatch {sorted(devices)}")
    metas = tuple(torch.empty(s.shape, dtype=s.dtype, device="meta") for s in input_specs)
    try:
        out = evaluate(op, metas, dict(attrs))
    except GraphError:
        raise
    except Exception as e:  # noqa: BLE001 - any torch failure is an invalid graph
        raise GraphError(f"op {op!r} failed spec inference: {e}") from e
    return TensorSpec(tuple(out.shape), out.dtype, _result_device(op, input_specs))


def _mermaid_label(text: str) -> str:
    return text.replace("&", "#amp;").replace('"', "#quot;").replace("\n", "#32;").replace("\r", "")


@dataclass
class Graph:
    inputs: dict[str, TensorSpec]
    constants: dict[str, torch.Tensor]
    nodes: list[Node]
    outputs: tuple[str, ...]
    output_is_tuple: bool = False

    def specs(self) -> dict[str, TensorSpec]:
        out = dict(self.inputs)
        for name, t in self.constants.items():
            out[name] = spec_of(t)
        for node in self.nodes:
            out[node.name] = node.spec
        return out

    def validate(self) -> None:
        seen: set[str] = set()
        for name in [*self.inputs, *self.constants]:
            if not isinstance(name, str) or not name:
                raise GraphError("value names must be non-empty strings")
            if name in seen:
                raise GraphError(f"duplicate name {name!r}")
            seen.add(name)
        for name, spec in self.inputs.items():
            if not isinstance(spec, TensorSpec):
                raise GraphError(f"input {name!r} spec must be a TensorSpec")
        env: dict[str, TensorSpec] = dict(self.inputs)
        for name, t in self.constants.items():
            if not isinstance(t, torch.Tensor):
                raise GraphError(f"constant {name!r} is not a torch.Tensor")
            env[name] = spec_of(t)
        for node in self.nodes:
            if not isinstance(node.name, str) or not node.name:
                raise GraphError("node names must be non-empty strings")
            if not isinstance(node.spec, TensorSpec):
                raise GraphError(f"node {node.name!r} spec must be a TensorSpec")
            if node.name in seen:
                raise GraphError(f"duplicate name {node.name!r}")
            seen.add(node.name)
            for inp in node.inputs:
                if inp not in env:
                    raise GraphError(f"node {node.name!r} input {inp!r} is not defined before use")
            if not isinstance(node.attrs, dict):
                raise GraphError(f"node {node.name!r} attrs must be a dict, got {type(node.attrs).__name__}")
            try:
                spec = infer_spec(node.op, [env[i] for i in node.inputs], dict(node.attrs))
            except GraphError as e:
                raise GraphError(f"node {node.name!r}: {e}") from e
            if spec != node.spec:
                raise GraphError(f"node {node.name!r} spec mismatch: declared {node.spec}, inferred {spec}")
            env[node.name] = node.spec
        if not self.outputs:
            raise GraphError("graph outputs must be non-empty")
        if not isinstance(self.output_is_tuple, bool):
            raise GraphError("output_is_tuple must be a bool")
        if len(self.outputs) > 1 and not self.output_is_tuple:
            raise GraphError("multiple graph outputs require output_is_tuple=True")
        for name in self.outputs:
            if name not in env:
                raise GraphError(f"graph output {name!r} is not defined")

    def clone(self) -> Graph:
        return Graph(
            inputs=dict(self.inputs),
            constants={k: v.detach().clone() for k, v in self.constants.items()},
            nodes=[Node(n.name, n.op, tuple(n.inputs), copy.deepcopy(n.attrs), n.spec) for n in self.nodes],
            outputs=tuple(self.outputs),
            output_is_tuple=self.output_is_tuple,
        )

    def to_dict(self) -> dict:
        def attr_value(v: Any) -> Any:
            return list(v) if isinstance(v, tuple) else v

        return {
            "inputs": {k: v.to_dict() for k, v in self.inputs.items()},
            "constants": {k: spec_of(v).to_dict() for k, v in self.constants.items()},
            "nodes": [
                {
                    "name": n.name,
                    "op": n.op,
                    "inputs": list(n.inputs),
                    "attrs": {k: attr_value(v) for k, v in n.attrs.items()},
                    "spec": n.spec.to_dict(),
                }
                for n in self.nodes
            ],
            "outputs": list(self.outputs),
            "output_is_tuple": self.output_is_tuple,
        }

    def to_mermaid(self) -> str:
        names = [*self.inputs, *self.constants, *(n.name for n in self.nodes)]
        ids = {name: f"v{i}" for i, name in enumerate(dict.fromkeys(names))}
        lines = ["graph TD"]
        for name, spec in self.inputs.items():
            lines.append(f'    {ids[name]}["{_mermaid_label(name)} input {list(spec.shape)} {spec.dtype}"]')
        for name, t in self.constants.items():
            lines.append(f'    {ids[name]}["{_mermaid_label(name)} const {list(t.shape)} {t.dtype}"]')
        for node in self.nodes:
            lines.append(
                f'    {ids[node.name]}["{_mermaid_label(node.name)} {node.op} {list(node.spec.shape)} {node.spec.dtype}"]'
            )
            lines.extend(f"    {ids[i]} --> {ids[node.name]}" for i in node.inputs)
        lines.extend(f"    {ids[name]}:::output" for name in self.outputs)
        lines.append("    classDef output fill:#dfd")
        return "\n".join(lines)


class GraphBuilder:
    """Incremental graph construction with spec inference at every step."""

    def __init__(self, inputs: dict[str, TensorSpec]):
        self._inputs = dict(inputs)
        for name, spec in self._inputs.items():
            if not isinstance(name, str) or not name:
                raise GraphError("input names must be non-empty strings")
            if not isinstance(spec, TensorSpec):
                raise GraphError(f"input {name!r} spec must be a TensorSpec")
        self._constants: dict[str, torch.Tensor] = {}
        self._nodes: list[Node] = []
        self._names = set(self._inputs)
        self._env: dict[str, TensorSpec] = dict(self._inputs)

    def _claim(self, name: str) -> None:
        if not isinstance(name, str) or not name:
            raise GraphError("names must be non-empty strings")
        if name in self._names:
            raise GraphError(f"duplicate name {name!r}")
        self._names.add(name)

    def spec(self, name: str) -> TensorSpec:
        return self._env[name]

    def constant(self, name: str, value: torch.Tensor) -> str:
        self._claim(name)
        if not isinstance(value, torch.Tensor):
            self._names.discard(name)
            raise GraphError(f"constant {name!r} must be a torch.Tensor")
        snapshot = value.detach().clone()
        self._env[name] = spec_of(snapshot)
        self._constants[name] = snapshot
        return name

    def add(self, name: str, op: str, inputs: tuple[str, ...], **attrs) -> str:
        self._claim(name)
        for inp in inputs:
            if inp not in self._env:
                self._names.discard(name)
                raise GraphError(f"node {name!r} input {inp!r} is not defined")
        try:
            spec = infer_spec(op, [self._env[i] for i in inputs], attrs)
        except GraphError as e:
            self._names.discard(name)
            raise GraphError(f"node {name!r}: {e}") from e
        self._nodes.append(Node(name, op, tuple(inputs), dict(attrs), spec))
        self._env[name] = spec
        return name

    def finish(self, outputs: tuple[str, ...], output_is_tuple: bool = False) -> Graph:
        graph = Graph(
            inputs=dict(self._inputs),
            constants=dict(self._constants),
            nodes=list(self._nodes),
            outputs=tuple(outputs),
            output_is_tuple=output_is_tuple or len(outputs) > 1,
        )
        graph.validate()
        return graph
