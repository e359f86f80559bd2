"""torch.fx frontend: lowers an eval-mode ``nn.Module`` to the static IR.

Lowering rules and value naming follow ForgeML's ``from_torch``
(src/forgeml/frontend.py:98-722) so compiled graphs, including constant
names, match the reference's:

* ``nn.Linear`` / ``F.linear`` become ``linear(x, W^T, b)`` with ``W^T``
  stored as a contiguous ``[K, N]`` constant (frontend.py:187-233); inputs of
  rank != 2 are flattened to 2-D and reshaped back afterwards.
* Fresh names are ``<hint>_<n>`` from one counter per lowering
  (frontend.py:109-119).
* Shape queries (``x.shape``, ``size()``, ``dim()``), indexing and integer
  arithmetic on them are resolved statically at trace time.
* Training-mode dropout/batch-norm is rejected (frontend.py:28-48).
"""

from __future__ import annotations

import math
import operator
from typing import Any

import torch
import torch.fx
import torch.nn.functional as F
from torch import nn
from torch.fx import symbolic_trace

from forgeml_amd.ir import Graph, GraphBuilder, GraphError, TensorSpec


class UnsupportedOperator(GraphError):
    pass


class _Static:
    """A trace-time constant (shape, int, dtype ...), not a graph value."""

    def __init__(self, value: Any):
        self.value = value


def _spec(t: torch.Tensor) -> TensorSpec:
    return TensorSpec(tuple(t.shape), t.dtype, str(t.device))


def _check_module_state(model: nn.Module) -> None:
    for m in model.modules():
        if m.training and isinstance(m, (nn.modules.dropout._DropoutNd, nn.modules.batchnorm._BatchNorm)):
            raise GraphError(
                f"module {type(m).__name__} is in training mode; call model.eval() before compiling"
            )
        if isinstance(m, nn.Conv2d) and m.padding_mode != "zeros":
            raise UnsupportedOperator(f"Conv2d padding_mode={m.padding_mode!r} is not supported")
        if isinstance(m, nn.Embedding) and (
            m.padding_idx is not None or m.max_norm is not None or m.norm_type != 2.0
            or m.scale_grad_by_freq or m.sparse
        ):
            raise UnsupportedOperator(
                "Embedding options padding_idx/max_norm/norm_type/scale_grad_by_freq/sparse are not supported"
            )


def _resolve_attr(root: nn.Module, target: str) -> torch.Tensor:
    obj: Any = root
    for part in target.split("."):
        if not isinstance(obj, (nn.Module, torch.Tensor)) or not hasattr(obj, part):
            raise GraphError(f"cannot resolve attribute {target!r}")
        obj = getattr(obj, part)
    if not isinstance(obj, torch.Tensor):
        raise GraphError(f"attribute {target!r} is not a tensor")
    return obj


def _static_shape(raw: Any, in_shape: tuple[int, ...], where: str) -> tuple[int, ...]:
    if not isinstance(raw, (tuple, list)):
        raise UnsupportedOperator(f"{where} requires a static shape tuple/list")
    dims = list(raw)
    if not all(isinstance(d, int) and not isinstance(d, bool) for d in dims):
        raise UnsupportedOperator(f"{where} shape dims must be ints, got {dims!r}")
    if sum(1 for d in dims if d == -1) > 1:
        raise UnsupportedOperator(f"{where} allows at most one -1 dim, got {dims!r}")
    if any(d == 0 or d < -1 for d in dims):
        raise UnsupportedOperator(f"{where} dims must be positive or -1, got {dims!r}")
    if -1 in dims:
        known = math.prod(d for d in dims if d != -1)
        total = math.prod(in_shape)
        if known == 0 or total % known:
            raise GraphError(f"{where} cannot infer -1 dim for input {in_shape}")
        dims[dims.index(-1)] = total // known
    return tuple(dims)


def _flatten_shape(spec: TensorSpec, start_dim: Any, end_dim: Any, where: str) -> tuple[int, ...]:
    rank = len(spec.shape)
    if rank == 0:
        raise UnsupportedOperator(f"{where} requires a tensor of rank >= 1")
    ends = []
    for label, raw in (("start_dim", start_dim), ("end_dim", end_dim)):
        if not isinstance(raw, int) or isinstance(raw, bool) or not -rank <= raw < rank:
            raise UnsupportedOperator(f"{where} {label}={raw!r} out of range for rank {rank}")
        ends.append(raw % rank)
    start, end = ends
    if start > end:
        raise UnsupportedOperator(f"{where} has start_dim > end_dim")
    return spec.shape[:start] + (math.prod(spec.shape[start:end + 1]),) + spec.shape[end + 1:]


_STATIC_BINARY = {
    operator.add: operator.add,
    operator.sub: operator.sub,
    operator.mul: operator.mul,
    operator.floordiv: operator.floordiv,
    operator.truediv: operator.truediv,
    operator.mod: operator.mod,
}

_SDPA_ARGS = ("query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale", "enable_gqa")
_SDPA_DEFAULTS = {"attn_mask": None, "dropout_p": 0.0, "is_causal": False, "scale": None, "enable_gqa": False}


class _Lowerer:
    def __init__(self, model: nn.Module, example_inputs: tuple[torch.Tensor, ...]):
        self.model = model
        self.example_inputs = example_inputs
        self.builder: GraphBuilder | None = None
        self.env: dict[str, str] = {}          # fx node name -> IR value name
        self.const_tensors: dict[str, torch.Tensor] = {}
        self.static_values: dict[str, Any] = {}
        self._counter = 0

    # -- naming and values -------------------------------------------------
    def _fresh(self, hint: str) -> str:
        self._counter += 1
        return f"{hint}_{self._counter}"

    def _add_constant(self, name: str, value: torch.Tensor) -> str:
        self.builder.constant(name, value)
        self.const_tensors[name] = value
        return name

    def _constant(self, hint: str, value: torch.Tensor) -> str:
        return self._add_constant(self._fresh(hint), value.detach().clone().contiguous())

    def _spec(self, value: str) -> TensorSpec:
        return self.builder.spec(value)

    def _maybe_literal(self, value: Any) -> tuple[bool, Any]:
        if isinstance(value, torch.fx.Node):
            if value.name in self.static_values:
                return True, self.static_values[value.name]
            return False, None
        if isinstance(value, torch.Size):
            return True, tuple(int(d) for d in value)
        if isinstance(value, (tuple, list)):
            out = []
            for item in value:
                ok, lit = self._maybe_literal(item)
                if not ok:
                    return False, None
                out.append(lit)
            return True, tuple(out)
        return True, value

    def _literal(self, value: Any) -> Any:
        ok, lit = self._maybe_literal(value)
        if not ok:
            if isinstance(value, torch.fx.Node):
                raise UnsupportedOperator(f"fx value {value.name!r} must resolve statically at compile time")
            raise UnsupportedOperator(f"unsupported static value {value!r}")
        return lit

    def _arg(self, a: Any) -> str:
        if isinstance(a, torch.fx.Node):
            if a.name in self.env:
                return self.env[a.name]
            if a.name not in self.static_values:
                raise GraphError(f"fx node {a.name!r} has no produced value")
            a = self.static_values[a.name]
        if isinstance(a, (int, float, bool)):
            return self._add_constant(self._fresh("scalar"), torch.tensor(a))
        raise UnsupportedOperator(f"unsupported argument {a!r} of type {type(a).__name__}")

    def _bind(self, node, names: tuple[str, ...], defaults: dict | None = None) -> dict:
        if len(node.args) > len(names):
            raise UnsupportedOperator(f"too many arguments at {node.name!r}")
        bound = dict(zip(names, node.args))
        for key, value in node.kwargs.items():
            if key not in names or key in bound:
                raise UnsupportedOperator(f"unsupported or repeated argument {key!r} at {node.name!r}")
            bound[key] = value
        for key, value in (defaults or {}).items():
            bound.setdefault(key, value)
        if set(names) - set(bound):
            raise UnsupportedOperator(f"missing argument at {node.name!r}")
        return bound

    # -- the GEMM lowering ---------------------------------------------------
    def _linear(self, out_name: str, x: str, weight: torch.Tensor, bias: torch.Tensor | None) -> str:
        if weight.dim() != 2:
            raise UnsupportedOperator(f"linear weight at {out_name!r} must be rank-2, got rank {weight.dim()}")
        if bias is not None and bias.dim() != 1:
            raise UnsupportedOperator(f"linear bias at {out_name!r} must be rank-1, got rank {bias.dim()}")
        w_t = weight.t().contiguous()
        w_name = self._add_constant(self._fresh(f"{out_name}_weight_t"), w_t)
        x_shape = self._spec(x).shape
        flat = x
        if len(x_shape) != 2:
            if not x_shape:
                raise UnsupportedOperator(f"linear input at {out_name!r} must have rank >= 1")
            flat = self.builder.add(
                self._fresh(f"{out_name}_flatten"), "reshape", (x,),
                shape=(math.prod(x_shape[:-1]), x_shape[-1]),
            )
        inputs = (flat, w_name)
        if bias is not None:
            inputs += (self._add_constant(self._fresh(f"{out_name}_bias"), bias.contiguous()),)
        if len(x_shape) == 2:
            return self.builder.add(out_name, "linear", inputs)
        result = self.builder.add(self._fresh(f"{out_name}_linear"), "linear", inputs)
        return self.builder.add(out_name, "reshape", (result,), shape=x_shape[:-1] + (w_t.shape[1],))

    # -- driver --------------------------------------------------------------
    def lower(self) -> Graph:
        inputs = {f"input_{i}": _spec(t) for i, t in enumerate(self.example_inputs)}
        try:
            traced = symbolic_trace(self.model)
        except Exception as e:  # noqa: BLE001
            raise UnsupportedOperator(f"symbolic trace failed: {e}") from e
        self.builder = GraphBuilder(inputs)
        placeholders = [n for n in traced.graph.nodes if n.op == "placeholder"]
        if len(placeholders) != len(self.example_inputs):
            raise GraphError(
                f"model expects {len(placeholders)} inputs, got {len(self.example_inputs)} example inputs"
            )
        for i, ph in enumerate(placeholders):
            self.env[ph.name] = f"input_{i}"
        for node in traced.graph.nodes:
            if node.op == "placeholder":
                continue
            if node.op == "output":
                return self._finish(node)
            lowered = self._lower_node(traced, node)
            if isinstance(lowered, _Static):
                self.static_values[node.name] = lowered.value
            else:
                self.env[node.name] = lowered
        raise GraphError("traced graph has no output node")

    def _lower_node(self, traced, node):
        if node.op == "get_attr":
            t = _resolve_attr(traced, node.target).detach().clone().contiguous()
            return self._add_constant(node.name, t)
        if node.op == "call_module":
            mod = traced
            for part in node.target.split("."):
                mod = getattr(mod, part)
            return self._lower_module(node.name, mod, node)
        if node.op == "call_function":
            return self._lower_function(node.name, node)
        if node.op == "call_method":
            return self._lower_method(node.name, node)
        raise UnsupportedOperator(f"unsupported fx node op {node.op!r} at {node.name!r}")

    def _lower_module(self, name: str, mod: nn.Module, node) -> str:
        x = self._arg(self._bind(node, ("input",))["input"])
        if isinstance(mod, nn.Identity):
            return x
        if isinstance(mod, nn.Linear):
            bias = None if mod.bias is None else mod.bias.detach().clone()
            return self._linear(name, x, mod.weight.detach().clone(), bias)
        if isinstance(mod, nn.LayerNorm):
            normalized = tuple(mod.normalized_shape)
            inputs: tuple[str, ...] = (x,)
            if mod.elementwise_affine:
                if mod.weight is None or mod.bias is None:
                    raise UnsupportedOperator(f"partially affine LayerNorm at {name!r}")
                inputs = (x, self._constant(f"{name}_weight", mod.weight), self._constant(f"{name}_bias", mod.bias))
            return self.builder.add(name, "layer_norm", inputs, normalized_shape=normalized, eps=float(mod.eps))
        if isinstance(mod, nn.Conv2d):
            if mod.padding_mode != "zeros":
                raise UnsupportedOperator(f"Conv2d padding_mode={mod.padding_mode!r} at {name!r} is not supported")
            inputs = (x, self._constant(f"{name}_weight", mod.weight))
            if mod.bias is not None:
                inputs += (self._constant(f"{name}_bias", mod.bias),)
            return self.builder.add(name, "conv2d", inputs, stride=mod.stride, padding=mod.padding,
                                    dilation=mod.dilation, groups=mod.groups)
        if isinstance(mod, nn.Embedding):
            if (mod.padding_idx is not None or mod.max_norm is not None or mod.norm_type != 2.0
                    or mod.scale_grad_by_freq or mod.sparse):
                raise UnsupportedOperator(f"Embedding options at {name!r} are not supported in inference lowering")
            return self.builder.add(name, "embedding", (x, self._constant(f"{name}_weight", mod.weight)))
        if isinstance(mod, nn.Flatten):
            shape = _flatten_shape(self._spec(x), mod.start_dim, mod.end_dim, f"Flatten at {name!r}")
            return self.builder.add(name, "reshape", (x,), shape=shape)
        if isinstance(mod, nn.GELU):
            return self.builder.add(name, "gelu", (x,), approximate=mod.approximate)
        if isinstance(mod, nn.ReLU):
            if mod.inplace:
                raise UnsupportedOperator(f"in-place ReLU at {name!r} is not supported")
            return self.builder.add(name, "relu", (x,))
        if isinstance(mod, nn.Softmax):
            if mod.dim is None:
                raise UnsupportedOperator(f"Softmax at {name!r} has no static dim")
            return self.builder.add(name, "softmax", (x,), dim=mod.dim)
        raise UnsupportedOperator(f"unsupported module {type(mod).__name__} at {name!r}")

    def _matmul_operands(self, node, name: str, what: str) -> tuple[str, str]:
        bound = self._bind(node, ("input", "other", "mat2"), {"other": None, "mat2": None})
        if bound["other"] is not None and bound["mat2"] is not None:
            raise UnsupportedOperator(f"{what} got both 'other' and 'mat2' at {name!r}")
        other = bound["other"] if bound["other"] is not None else bound["mat2"]
        if other is None:
            raise UnsupportedOperator(f"{what} at {name!r} needs a second operand")
        return self._arg(bound["input"]), self._arg(other)

    def _softmax_dim(self, bound: dict, name: str) -> int:
        if bound["dtype"] is not None:
            raise UnsupportedOperator(f"softmax dtype= at {name!r} is not supported")
        dim = self._literal(bound["dim"])
        if not isinstance(dim, int) or isinstance(dim, bool):
            raise UnsupportedOperator(f"softmax at {name!r} needs a static int dim")
        return dim

    def _lower_function(self, name: str, node):
        target = node.target
        if target is getattr:
            bound = self._bind(node, ("input", "name"))
            source = bound["input"]
            if not hasattr(source, "name") or source.name not in self.env:
                raise UnsupportedOperator(f"getattr source at {name!r} must be a tensor value")
            spec = self._spec(self.env[source.name])
            attr = bound["name"]
            statics = {
                "shape": lambda: spec.shape,
                "ndim": lambda: len(spec.shape),
                "device": lambda: torch.device(spec.device),
                "dtype": lambda: spec.dtype,
            }
            if attr not in statics:
                raise UnsupportedOperator(f"getattr {attr!r} at {name!r} is not supported")
            return _Static(statics[attr]())
        if target is operator.getitem:
            bound = self._bind(node, ("input", "index"))
            value, index = self._literal(bound["input"]), self._literal(bound["index"])
            try:
                return _Static(value[index])
            except (IndexError, KeyError, TypeError) as e:
                raise UnsupportedOperator(f"invalid static index at {name!r}") from e
        if target in _STATIC_BINARY:
            a_ok, a = self._maybe_literal(node.args[0])
            b_ok, b = self._maybe_literal(node.args[1])
            if a_ok and b_ok:
                return _Static(_STATIC_BINARY[target](a, b))
        if target in (operator.neg, operator.pos):
            ok, value = self._maybe_literal(node.args[0])
            if ok:
                return _Static(target(value))
        if target is torch.arange:
            positional = tuple(self._literal(a) for a in node.args)
            if not 1 <= len(positional) <= 3:
                raise UnsupportedOperator(f"arange at {name!r} expects 1-3 positional arguments")
            extra = set(node.kwargs) - {"dtype", "device", "layout", "requires_grad", "pin_memory"}
            if extra:
                raise UnsupportedOperator(f"arange at {name!r} has unsupported kwargs {sorted(extra)}")
            options = {k: self._literal(v) for k, v in node.kwargs.items()}
            if options.get("layout") not in (None, torch.strided):
                raise UnsupportedOperator(f"arange layout at {name!r} is not supported")
            if options.get("requires_grad") or options.get("pin_memory"):
                raise UnsupportedOperator(f"arange options at {name!r} are not supported")
            try:
                tensor = torch.arange(*positional, **options).detach()
            except (RuntimeError, TypeError, ValueError) as e:
                raise UnsupportedOperator(f"invalid arange arguments at {name!r}: {e}") from e
            return self._constant(name, tensor)
        if target in (torch.matmul, torch.mm, operator.matmul):
            return self.builder.add(name, "matmul", self._matmul_operands(node, name, "matmul"))
        if target in (operator.add, torch.add):
            bound = self._bind(node, ("input", "other", "alpha", "out"), {"alpha": 1, "out": None})
            if "out" in node.kwargs or bound["out"] is not None:
                raise UnsupportedOperator(f"add out= at {name!r} is not supported")
            if bound["alpha"] != 1:
                raise UnsupportedOperator(f"add alpha!=1 at {name!r} is not supported")
            return self.builder.add(name, "add", (self._arg(bound["input"]), self._arg(bound["other"])))
        if target in (operator.mul, torch.mul):
            bound = self._bind(node, ("input", "other", "out"), {"out": None})
            if "out" in node.kwargs or bound["out"] is not None:
                raise UnsupportedOperator(f"mul out= at {name!r} is not supported")
            return self.builder.add(name, "mul", (self._arg(bound["input"]), self._arg(bound["other"])))
        if target is F.relu:
            bound = self._bind(node, ("input", "inplace"), {"inplace": False})
            if bound["inplace"] is not False:
                raise UnsupportedOperator(f"in-place relu at {name!r} is not supported")
            return self.builder.add(name, "relu", (self._arg(bound["input"]),))
        if target is torch.relu:
            return self.builder.add(name, "relu", (self._arg(self._bind(node, ("input",))["input"]),))
        if target is F.gelu or target is getattr(torch, "gelu", None):
            bound = self._bind(node, ("input", "approximate"), {"approximate": "none"})
            if bound["approximate"] not in ("none", "tanh"):
                raise UnsupportedOperator(f"gelu approximate {bound['approximate']!r} at {name!r}")
            return self.builder.add(name, "gelu", (self._arg(bound["input"]),), approximate=bound["approximate"])
        if target is F.linear:
            bound = self._bind(node, ("input", "weight", "bias"), {"bias": None})
            x = self._arg(bound["input"])
            w = self._arg(bound["weight"])
            if w not in self.const_tensors:
                raise UnsupportedOperator(f"linear weight at {name!r} must be constant")
            bias = None
            if bound["bias"] is not None:
                b = self._arg(bound["bias"])
                if b not in self.const_tensors:
                    raise UnsupportedOperator(f"linear bias at {name!r} must be constant")
                bias = self.const_tensors[b]
            return self._linear(name, x, self.const_tensors[w], bias)
        if target in (torch.reshape, torch.Tensor.reshape, torch.Tensor.view):
            bound = self._bind(node, ("input", "shape"))
            x = self._arg(bound["input"])
            shape = _static_shape(self._literal(bound["shape"]), self._spec(x).shape, "reshape")
            return self.builder.add(name, "reshape", (x,), shape=shape)
        if target is torch.transpose:
            bound = self._bind(node, ("input", "dim0", "dim1"))
            return self.builder.add(name, "transpose", (self._arg(bound["input"]),),
                                    dim0=self._literal(bound["dim0"]), dim1=self._literal(bound["dim1"]))
        if target in (F.softmax, torch.softmax):
            bound = self._bind(node, ("input", "dim", "_stacklevel", "dtype"),
                               {"dim": None, "_stacklevel": 3, "dtype": None})
            return self.builder.add(name, "softmax", (self._arg(bound["input"]),), dim=self._softmax_dim(bound, name))
        if target is F.layer_norm:
            bound = self._bind(node, ("input", "normalized_shape", "weight", "bias", "eps"),
                               {"weight": None, "bias": None, "eps": 1e-5})
            x = self._arg(bound["input"])
            normalized = self._literal(bound["normalized_shape"])
            if isinstance(normalized, int):
                normalized = (normalized,)
            if (bound["weight"] is None) != (bound["bias"] is None):
                raise UnsupportedOperator(f"layer_norm at {name!r} needs weight and bias together")
            inputs = (x,)
            if bound["weight"] is not None:
                inputs += (self._arg(bound["weight"]), self._arg(bound["bias"]))
            return self.builder.add(name, "layer_norm", inputs, normalized_shape=tuple(normalized),
                                    eps=float(self._literal(bound["eps"])))
        if target is F.scaled_dot_product_attention:
            bound = self._bind(node, _SDPA_ARGS, _SDPA_DEFAULTS)
            if self._literal(bound["dropout_p"]) != 0:
                raise UnsupportedOperator(f"sdpa dropout_p at {name!r} must be zero")
            if self._literal(bound["enable_gqa"]) is not False:
                raise UnsupportedOperator(f"sdpa enable_gqa at {name!r} is not supported")
            is_causal = self._literal(bound["is_causal"])
            if not isinstance(is_causal, bool):
                raise UnsupportedOperator(f"sdpa is_causal at {name!r} must be a bool")
            scale = self._literal(bound["scale"])
            inputs = (self._arg(bound["query"]), self._arg(bound["key"]), self._arg(bound["value"]))
            if bound["attn_mask"] is not None:
                inputs += (self._arg(bound["attn_mask"]),)
            return self.builder.add(name, "sdpa", inputs, is_causal=is_causal, scale=scale)
        if target in (F.conv2d, torch.conv2d):
            bound = self._bind(node, ("input", "weight", "bias", "stride", "padding", "dilation", "groups"),
                               {"bias": None, "stride": 1, "padding": 0, "dilation": 1, "groups": 1})
            inputs = (self._arg(bound["input"]), self._arg(bound["weight"]))
            if bound["bias"] is not None:
                inputs += (self._arg(bound["bias"]),)
            return self.builder.add(name, "conv2d", inputs, stride=self._literal(bound["stride"]),
                                    padding=self._literal(bound["padding"]),
                                    dilation=self._literal(bound["dilation"]), groups=self._literal(bound["groups"]))
        if target in (F.embedding, torch.embedding):
            bound = self._bind(node, ("input", "weight"))
            return self.builder.add(name, "embedding", (self._arg(bound["input"]), self._arg(bound["weight"])))
        if target is torch.flatten:
            bound = self._bind(node, ("input", "start_dim", "end_dim"), {"start_dim": 0, "end_dim": -1})
            x = self._arg(bound["input"])
            shape = _flatten_shape(self._spec(x), self._literal(bound["start_dim"]),
                                   self._literal(bound["end_dim"]), f"flatten at {name!r}")
            return self.builder.add(name, "reshape", (x,), shape=shape)
        raise UnsupportedOperator(f"unsupported function {getattr(target, '__name__', target)!r} at {name!r}")

    def _lower_method(self, name: str, node):
        method = node.target
        if method in ("size", "dim", "ndim"):
            bound = self._bind(node, ("input", "dim"), {"dim": None})
            shape = self._spec(self._arg(bound["input"])).shape
            if method in ("dim", "ndim") and bound["dim"] is None:
                return _Static(len(shape))
            if bound["dim"] is None:
                return _Static(shape)
            index = self._literal(bound["dim"])
            if not isinstance(index, int) or isinstance(index, bool):
                raise UnsupportedOperator(f"{method} at {name!r} needs an int dimension")
            if not -len(shape) <= index < len(shape):
                raise UnsupportedOperator(f"{method} index {index} out of range for rank {len(shape)} at {name!r}")
            return _Static(shape[index])
        if method in ("matmul", "mm"):
            return self.builder.add(name, "matmul", self._matmul_operands(node, name, method))
        if method in ("view", "reshape"):
            if node.kwargs:
                raise UnsupportedOperator(f"{method} kwargs at {name!r} are not supported")
            if len(node.args) < 2:
                raise UnsupportedOperator(f"{method} at {name!r} needs a shape")
            x = self._arg(node.args[0])
            raw = tuple(self._literal(v) for v in node.args[1:])
            dims = list(raw[0]) if len(raw) == 1 and isinstance(raw[0], (tuple, list)) else list(raw)
            shape = _static_shape(tuple(dims), self._spec(x).shape, method)
            return self.builder.add(name, "reshape", (x,), shape=shape)
        if method == "flatten":
            bound = self._bind(node, ("input", "start_dim", "end_dim"), {"start_dim": 0, "end_dim": -1})
            x = self._arg(bound["input"])
            shape = _flatten_shape(self._spec(x), self._literal(bound["start_dim"]),
                                   self._literal(bound["end_dim"]), f"flatten at {name!r}")
            return self.builder.add(name, "reshape", (x,), shape=shape)
        if method == "transpose":
            bound = self._bind(node, ("input", "dim0", "dim1"))
            return self.builder.add(name, "transpose", (self._arg(bound["input"]),),
                                    dim0=self._literal(bound["dim0"]), dim1=self._literal(bound["dim1"]))
        if method == "t":
            x = self._arg(self._bind(node, ("input",))["input"])
            if len(self._spec(x).shape) != 2:
                raise UnsupportedOperator(f"t() at {name!r} requires a rank-2 tensor")
            return self.builder.add(name, "transpose", (x,), dim0=0, dim1=1)
        if method == "softmax":
            bound = self._bind(node, ("input", "dim", "dtype"), {"dtype": None})
            return self.builder.add(name, "softmax", (self._arg(bound["input"]),), dim=self._softmax_dim(bound, name))
        raise UnsupportedOperator(f"unsupported method {method!r} at {name!r}")

    def _finish(self, output_node) -> Graph:
        result = output_node.args[0]
        if isinstance(result, torch.fx.Node):
            if result.name not in self.env:
                raise UnsupportedOperator("model outputs must be produced tensors; static values are not supported")
            return self.builder.finish((self.env[result.name],), output_is_tuple=False)
        if isinstance(result, tuple):
            names = []
            for r in result:
                if not isinstance(r, torch.fx.Node) or r.name not in self.env:
                    raise UnsupportedOperator("only flat tuples of produced tensors are supported as outputs")
                names.append(self.env[r.name])
            return self.builder.finish(tuple(names), output_is_tuple=True)
        raise UnsupportedOperator(
            f"unsupported output type {type(result).__name__}; only a tensor or flat tuple of tensors is supported"
        )


def from_torch(model: torch.nn.Module, example_inputs: tuple[torch.Tensor, ...]) -> Graph:
    if not isinstance(model, nn.Module):
        raise GraphError("from_torch expects an nn.Module")
    for i, t in enumerate(example_inputs):
        if not isinstance(t, torch.Tensor):
            raise GraphError(f"example input {i} is not a tensor")
    _check_module_state(model)
    with torch.no_grad():
        return _Lowerer(model, tuple(example_inputs)).lower()
