"""torch.fx frontend: lowers an eval-mode ``nn.Module`` to the static IR.

What a compiled graph looks like is fixed by ForgeML's ``from_torch``
(src/forgeml/frontend.py:98-722), whose published captures pin the names:

* inputs are ``input_<i>``; ``get_attr`` constants keep the fx node name;
* every other generated value is ``<hint>_<n>``, ``n`` counting up once per
  lowering (frontend.py:109-119);
* ``nn.Linear`` / ``F.linear`` become ``linear(x, W^T, b)`` with ``W^T`` a
  contiguous ``[K, N]`` constant, generated in the order weight, flatten
  (inputs of rank != 2), bias, inner linear (frontend.py:187-233);
* shape queries, indexing and integer arithmetic on them are evaluated at
  trace time and never enter the graph;
* training-mode dropout / batch-norm is refused (frontend.py:28-48).

How it is built here: each supported fx target (function, tensor method or
module type) has a lowering rule registered in a table; a rule receives the
lowering scope and the fx node, binds the call's arguments against a
declared parameter list, and returns either an IR value name or a
trace-time constant (``Static``).  One environment maps fx names to either.
"""

from __future__ import annotations

import math
import operator
from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

import torch
import torch.fx
import torch.nn.functional as F
from torch import nn

from forgeml_amd.ir import Graph, GraphBuilder, GraphError, TensorSpec


class UnsupportedOperator(GraphError):
    pass


@dataclass(frozen=True)
class Static:
    """A value known at trace time (a shape, an int, a dtype ...), not a graph value."""

    value: Any


class Params:
    """A call signature: positional names in order, defaults for the optional ones."""

    def __init__(self, *names: str, **defaults: Any):
        self.names = names
        self.defaults = defaults

    def bind(self, node: torch.fx.Node) -> dict[str, Any]:
        if len(node.args) > len(self.names):
            raise UnsupportedOperator(f"{node.name!r} passes {len(node.args)} positional arguments; "
                                      f"at most {len(self.names)} are supported")
        bound = dict(zip(self.names, node.args))
        for key, value in node.kwargs.items():
            if key not in self.names:
                raise UnsupportedOperator(f"argument {key!r} at {node.name!r} is not supported")
            if key in bound:
                raise UnsupportedOperator(f"argument {key!r} at {node.name!r} is given twice")
            bound[key] = value
        for key, value in self.defaults.items():
            bound.setdefault(key, value)
        missing = [n for n in self.names if n not in bound]
        if missing:
            raise UnsupportedOperator(f"{node.name!r} is missing argument(s) {missing}")
        return bound


# -- rule tables -------------------------------------------------------------------

Rule = Callable[["_Scope", torch.fx.Node], "str | Static"]
_FUNCTION_RULES: dict[Any, Rule] = {}
_METHOD_RULES: dict[str, Rule] = {}
_MODULE_RULES: list[tuple[type, Callable[["_Scope", torch.fx.Node, nn.Module], str]]] = []


def _on_function(*targets):
    def register(rule):
        for target in targets:
            if target is not None:
                _FUNCTION_RULES[target] = rule
        return rule
    return register


def _on_method(*names):
    def register(rule):
        for name in names:
            _METHOD_RULES[name] = rule
        return rule
    return register


def _on_module(kind: type):
    def register(rule):
        _MODULE_RULES.append((kind, rule))
        return rule
    return register


# -- the lowering scope ------------------------------------------------------------------

class _Scope:
    """State of one lowering: the graph builder, the fx -> IR environment and
    the counter behind every generated name."""

    def __init__(self, inputs: dict[str, TensorSpec]):
        self.builder = GraphBuilder(inputs)
        self.env: dict[str, str | Static] = {}
        self.constants: dict[str, torch.Tensor] = {}
        self._serial = 0

    def fresh(self, hint: str) -> str:
        self._serial += 1
        return f"{hint}_{self._serial}"

    def constant(self, name: str, value: torch.Tensor) -> str:
        self.builder.constant(name, value)
        self.constants[name] = value
        return name

    def hoist(self, hint: str, value: torch.Tensor) -> str:
        """A module parameter or trace-time tensor as a fresh-named constant."""
        return self.constant(self.fresh(hint), value.detach().clone().contiguous())

    def emit(self, name: str, op: str, inputs: tuple[str, ...], **attrs) -> str:
        return self.builder.add(name, op, tuple(inputs), **attrs)

    def spec(self, value: str) -> TensorSpec:
        return self.builder.spec(value)

    # Arguments of an fx call, resolved to statics or graph values.
    def known(self, arg: Any) -> tuple[bool, Any]:
        """(True, python value) when ``arg`` is known at trace time."""
        if isinstance(arg, torch.fx.Node):
            bound = self.env.get(arg.name)
            return (True, bound.value) if isinstance(bound, Static) else (False, None)
        if isinstance(arg, torch.Size):
            return True, tuple(int(d) for d in arg)
        if isinstance(arg, (tuple, list)):
            items = [self.known(a) for a in arg]
            if all(ok for ok, _ in items):
                return True, tuple(v for _, v in items)
            return False, None
        return True, arg

    def static(self, arg: Any) -> Any:
        ok, value = self.known(arg)
        if not ok:
            what = f"fx value {arg.name!r}" if isinstance(arg, torch.fx.Node) else f"value {arg!r}"
            raise UnsupportedOperator(f"{what} must resolve statically at compile time")
        return value

    def tensor(self, arg: Any) -> str:
        """The IR value of a tensor argument; Python numbers become scalar constants."""
        if isinstance(arg, torch.fx.Node):
            if arg.name not in self.env:
                raise GraphError(f"fx node {arg.name!r} has no produced value")
            bound = self.env[arg.name]
            if not isinstance(bound, Static):
                return bound
            arg = bound.value
        if isinstance(arg, (bool, int, float)):
            return self.constant(self.fresh("scalar"), torch.tensor(arg))
        raise UnsupportedOperator(f"unsupported argument {arg!r} of type {type(arg).__name__}")

    def linear(self, out: str, x: str, weight: torch.Tensor, bias: torch.Tensor | None) -> str:
        """x @ W^T + b with W^T stored as a contiguous [K, N] constant."""
        if weight.dim() != 2:
            raise UnsupportedOperator(f"linear weight at {out!r} must be rank-2, got rank {weight.dim()}")
        if bias is not None and bias.dim() != 1:
            raise UnsupportedOperator(f"linear bias at {out!r} must be rank-1, got rank {bias.dim()}")
        w_t = weight.t().contiguous()
        w_name = self.constant(self.fresh(f"{out}_weight_t"), w_t)
        shape = self.spec(x).shape
        if not shape:
            raise UnsupportedOperator(f"linear input at {out!r} must have rank >= 1")
        rows = x
        if len(shape) != 2:
            rows = self.emit(self.fresh(f"{out}_flatten"), "reshape", (x,), shape=(math.prod(shape[:-1]), shape[-1]))
        operands = (rows, w_name)
        if bias is not None:
            operands += (self.constant(self.fresh(f"{out}_bias"), bias.contiguous()),)
        if len(shape) == 2:
            return self.emit(out, "linear", operands)
        flat_out = self.emit(self.fresh(f"{out}_linear"), "linear", operands)
        return self.emit(out, "reshape", (flat_out,), shape=shape[:-1] + (w_t.shape[1],))


# -- shape helpers -------------------------------------------------------------------------

def _is_int(v: Any) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _target_shape(raw: Any, source: tuple[int, ...], where: str) -> tuple[int, ...]:
    """A reshape's static target shape, with at most one -1 inferred."""
    if not isinstance(raw, (tuple, list)) or not all(_is_int(d) for d in raw):
        raise UnsupportedOperator(f"{where} needs a static shape of ints, got {raw!r}")
    dims = list(raw)
    if dims.count(-1) > 1 or any(d == 0 or d < -1 for d in dims):
        raise UnsupportedOperator(f"{where} dims must be positive with at most one -1, got {dims!r}")
    if -1 in dims:
        rest = math.prod(d for d in dims if d != -1)
        total = math.prod(source)
        if total % rest:
            raise GraphError(f"{where} cannot infer -1 dim for input {source}")
        dims[dims.index(-1)] = total // rest
    return tuple(dims)


def _flattened(shape: tuple[int, ...], start: Any, end: Any, where: str) -> tuple[int, ...]:
    rank = len(shape)
    if rank == 0:
        raise UnsupportedOperator(f"{where} requires a tensor of rank >= 1")
    for label, d in (("start_dim", start), ("end_dim", end)):
        if not _is_int(d) or not -rank <= d < rank:
            raise UnsupportedOperator(f"{where} {label}={d!r} out of range for rank {rank}")
    lo, hi = start % rank, end % rank
    if lo > hi:
        raise UnsupportedOperator(f"{where} has start_dim > end_dim")
    return shape[:lo] + (math.prod(shape[lo:hi + 1]),) + shape[hi + 1:]


def _softmax_dim(cx: _Scope, bound: dict, name: str) -> int:
    if bound["dtype"] is not None:
        raise UnsupportedOperator(f"softmax dtype= at {name!r} is not supported")
    dim = cx.static(bound["dim"])
    if not _is_int(dim):
        raise UnsupportedOperator(f"softmax at {name!r} needs a static int dim")
    return dim


# -- function rules ----------------------------------------------------------------------------

@_on_function(getattr)
def _getattr(cx: _Scope, node):
    bound = Params("input", "name").bind(node)
    src = bound["input"]
    value = cx.env.get(src.name) if isinstance(src, torch.fx.Node) else None
    if value is None or isinstance(value, Static):
        raise UnsupportedOperator(f"getattr source at {node.name!r} must be a tensor value")
    spec = cx.spec(value)
    facts = {"shape": spec.shape, "ndim": len(spec.shape), "dtype": spec.dtype}
    attr = bound["name"]
    if attr == "device":
        return Static(torch.device(spec.device))
    if attr not in facts:
        raise UnsupportedOperator(f"getattr {attr!r} at {node.name!r} is not supported")
    return Static(facts[attr])


@_on_function(operator.getitem)
def _getitem(cx: _Scope, node):
    bound = Params("input", "index").bind(node)
    container, index = cx.static(bound["input"]), cx.static(bound["index"])
    try:
        return Static(container[index])
    except (IndexError, KeyError, TypeError) as e:
        raise UnsupportedOperator(f"invalid static index at {node.name!r}") from e


_ARITH = {operator.add: operator.add, operator.sub: operator.sub, operator.mul: operator.mul,
          operator.floordiv: operator.floordiv, operator.truediv: operator.truediv, operator.mod: operator.mod}


def _static_arith(cx: _Scope, node) -> Static | None:
    """Arithmetic on trace-time values (shape math), or None when an operand is a tensor."""
    if node.target in (operator.neg, operator.pos):
        ok, v = cx.known(node.args[0])
        return Static(node.target(v)) if ok else None
    if node.target in _ARITH and len(node.args) == 2:
        (ok_a, a), (ok_b, b) = cx.known(node.args[0]), cx.known(node.args[1])
        if ok_a and ok_b:
            return Static(_ARITH[node.target](a, b))
    return None


@_on_function(operator.sub, operator.floordiv, operator.truediv, operator.mod, operator.neg, operator.pos)
def _shape_math(cx: _Scope, node):
    folded = _static_arith(cx, node)
    if folded is None:
        raise UnsupportedOperator(f"unsupported function {getattr(node.target, '__name__', node.target)!r} "
                                  f"at {node.name!r}")
    return folded


@_on_function(operator.add, torch.add)
def _add(cx: _Scope, node):
    folded = _static_arith(cx, node) if node.target is operator.add else None
    if folded is not None:
        return folded
    bound = Params("input", "other", "alpha", "out", alpha=1, out=None).bind(node)
    if "out" in node.kwargs or bound["out"] is not None:
        raise UnsupportedOperator(f"add out= at {node.name!r} is not supported")
    if bound["alpha"] != 1:
        raise UnsupportedOperator(f"add alpha!=1 at {node.name!r} is not supported")
    return cx.emit(node.name, "add", (cx.tensor(bound["input"]), cx.tensor(bound["other"])))


@_on_function(operator.mul, torch.mul)
def _mul(cx: _Scope, node):
    folded = _static_arith(cx, node) if node.target is operator.mul else None
    if folded is not None:
        return folded
    bound = Params("input", "other", "out", out=None).bind(node)
    if "out" in node.kwargs or bound["out"] is not None:
        raise UnsupportedOperator(f"mul out= at {node.name!r} is not supported")
    return cx.emit(node.name, "mul", (cx.tensor(bound["input"]), cx.tensor(bound["other"])))


@_on_function(torch.arange)
def _arange(cx: _Scope, node):
    positional = tuple(cx.static(a) for a in node.args)
    if not 1 <= len(positional) <= 3:
        raise UnsupportedOperator(f"arange at {node.name!r} expects 1-3 positional arguments")
    allowed = {"dtype", "device", "layout", "requires_grad", "pin_memory"}
    if set(node.kwargs) - allowed:
        raise UnsupportedOperator(f"arange at {node.name!r} has unsupported kwargs {sorted(set(node.kwargs) - allowed)}")
    options = {k: cx.static(v) for k, v in node.kwargs.items()}
    if options.get("layout") not in (None, torch.strided):
        raise UnsupportedOperator(f"arange layout at {node.name!r} is not supported")
    if options.get("requires_grad") or options.get("pin_memory"):
        raise UnsupportedOperator(f"arange options at {node.name!r} are not supported")
    try:
        values = torch.arange(*positional, **options)
    except (RuntimeError, TypeError, ValueError) as e:
        raise UnsupportedOperator(f"invalid arange arguments at {node.name!r}: {e}") from e
    return cx.hoist(node.name, values)


def _matmul_operands(cx: _Scope, node, what: str) -> tuple[str, str]:
    bound = Params("input", "other", "mat2", other=None, mat2=None).bind(node)
    other, mat2 = bound["other"], bound["mat2"]
    if other is not None and mat2 is not None:
        raise UnsupportedOperator(f"{what} got both 'other' and 'mat2' at {node.name!r}")
    second = other if other is not None else mat2
    if second is None:
        raise UnsupportedOperator(f"{what} at {node.name!r} needs a second operand")
    return cx.tensor(bound["input"]), cx.tensor(second)


@_on_function(torch.matmul, torch.mm, operator.matmul)
def _matmul(cx: _Scope, node):
    return cx.emit(node.name, "matmul", _matmul_operands(cx, node, "matmul"))


@_on_function(F.relu)
def _relu_fn(cx: _Scope, node):
    bound = Params("input", "inplace", inplace=False).bind(node)
    if bound["inplace"] is not False:
        raise UnsupportedOperator(f"in-place relu at {node.name!r} is not supported")
    return cx.emit(node.name, "relu", (cx.tensor(bound["input"]),))


@_on_function(torch.relu)
def _relu_torch(cx: _Scope, node):
    return cx.emit(node.name, "relu", (cx.tensor(Params("input").bind(node)["input"]),))


@_on_function(F.gelu, getattr(torch, "gelu", None))
def _gelu(cx: _Scope, node):
    bound = Params("input", "approximate", approximate="none").bind(node)
    if bound["approximate"] not in ("none", "tanh"):
        raise UnsupportedOperator(f"gelu approximate {bound['approximate']!r} at {node.name!r}")
    return cx.emit(node.name, "gelu", (cx.tensor(bound["input"]),), approximate=bound["approximate"])


@_on_function(F.linear)
def _linear_fn(cx: _Scope, node):
    bound = Params("input", "weight", "bias", bias=None).bind(node)
    x = cx.tensor(bound["input"])
    params = {}
    for role in ("weight", "bias"):
        if bound[role] is None:
            continue
        value = cx.tensor(bound[role])
        if value not in cx.constants:
            raise UnsupportedOperator(f"linear {role} at {node.name!r} must be constant")
        params[role] = cx.constants[value]
    return cx.linear(node.name, x, params["weight"], params.get("bias"))


@_on_function(torch.reshape, torch.Tensor.reshape, torch.Tensor.view)
def _reshape_fn(cx: _Scope, node):
    bound = Params("input", "shape").bind(node)
    x = cx.tensor(bound["input"])
    return cx.emit(node.name, "reshape", (x,), shape=_target_shape(cx.static(bound["shape"]), cx.spec(x).shape,
                                                                    "reshape"))


@_on_function(torch.transpose)
def _transpose_fn(cx: _Scope, node):
    bound = Params("input", "dim0", "dim1").bind(node)
    return cx.emit(node.name, "transpose", (cx.tensor(bound["input"]),), dim0=cx.static(bound["dim0"]),
                   dim1=cx.static(bound["dim1"]))


@_on_function(F.softmax, torch.softmax)
def _softmax_fn(cx: _Scope, node):
    bound = Params("input", "dim", "_stacklevel", "dtype", dim=None, _stacklevel=3, dtype=None).bind(node)
    return cx.emit(node.name, "softmax", (cx.tensor(bound["input"]),), dim=_softmax_dim(cx, bound, node.name))


@_on_function(F.layer_norm)
def _layer_norm_fn(cx: _Scope, node):
    bound = Params("input", "normalized_shape", "weight", "bias", "eps", weight=None, bias=None,
                   eps=1e-5).bind(node)
    normalized = cx.static(bound["normalized_shape"])
    normalized = (normalized,) if isinstance(normalized, int) else tuple(normalized)
    if (bound["weight"] is None) != (bound["bias"] is None):
        raise UnsupportedOperator(f"layer_norm at {node.name!r} needs weight and bias together")
    operands = [cx.tensor(bound["input"])]
    if bound["weight"] is not None:
        operands += [cx.tensor(bound["weight"]), cx.tensor(bound["bias"])]
    return cx.emit(node.name, "layer_norm", tuple(operands), normalized_shape=normalized,
                   eps=float(cx.static(bound["eps"])))


_SDPA = Params("query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale", "enable_gqa",
               attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, enable_gqa=False)


@_on_function(F.scaled_dot_product_attention)
def _sdpa(cx: _Scope, node):
    bound = _SDPA.bind(node)
    if cx.static(bound["dropout_p"]) != 0:
        raise UnsupportedOperator(f"sdpa dropout_p at {node.name!r} must be zero")
    if cx.static(bound["enable_gqa"]) is not False:
        raise UnsupportedOperator(f"sdpa enable_gqa at {node.name!r} is not supported")
    causal = cx.static(bound["is_causal"])
    if not isinstance(causal, bool):
        raise UnsupportedOperator(f"sdpa is_causal at {node.name!r} must be a bool")
    operands = [cx.tensor(bound[role]) for role in ("query", "key", "value")]
    if bound["attn_mask"] is not None:
        operands.append(cx.tensor(bound["attn_mask"]))
    return cx.emit(node.name, "sdpa", tuple(operands), is_causal=causal, scale=cx.static(bound["scale"]))


@_on_function(F.conv2d, torch.conv2d)
def _conv2d_fn(cx: _Scope, node):
    bound = Params("input", "weight", "bias", "stride", "padding", "dilation", "groups",
                   bias=None, stride=1, padding=0, dilation=1, groups=1).bind(node)
    operands = [cx.tensor(bound["input"]), cx.tensor(bound["weight"])]
    if bound["bias"] is not None:
        operands.append(cx.tensor(bound["bias"]))
    geometry = {key: cx.static(bound[key]) for key in ("stride", "padding", "dilation", "groups")}
    return cx.emit(node.name, "conv2d", tuple(operands), **geometry)


@_on_function(F.embedding, torch.embedding)
def _embedding_fn(cx: _Scope, node):
    bound = Params("input", "weight").bind(node)
    return cx.emit(node.name, "embedding", (cx.tensor(bound["input"]), cx.tensor(bound["weight"])))


@_on_function(torch.flatten)
def _flatten_fn(cx: _Scope, node):
    bound = Params("input", "start_dim", "end_dim", start_dim=0, end_dim=-1).bind(node)
    x = cx.tensor(bound["input"])
    shape = _flattened(cx.spec(x).shape, cx.static(bound["start_dim"]), cx.static(bound["end_dim"]),
                       f"flatten at {node.name!r}")
    return cx.emit(node.name, "reshape", (x,), shape=shape)


# -- tensor-method rules ----------------------------------------------------------------------

@_on_method("size", "dim", "ndim")
def _size(cx: _Scope, node):
    bound = Params("input", "dim", dim=None).bind(node)
    shape = cx.spec(cx.tensor(bound["input"])).shape
    if bound["dim"] is None:
        return Static(shape if node.target == "size" else len(shape))
    axis = cx.static(bound["dim"])
    if not _is_int(axis):
        raise UnsupportedOperator(f"{node.target} at {node.name!r} needs an int dimension")
    if not -len(shape) <= axis < len(shape):
        raise UnsupportedOperator(f"{node.target} index {axis} out of range for rank {len(shape)} at {node.name!r}")
    return Static(shape[axis])


@_on_method("matmul", "mm")
def _matmul_method(cx: _Scope, node):
    return cx.emit(node.name, "matmul", _matmul_operands(cx, node, node.target))


@_on_method("view", "reshape")
def _reshape_method(cx: _Scope, node):
    if node.kwargs:
        raise UnsupportedOperator(f"{node.target} kwargs at {node.name!r} are not supported")
    if len(node.args) < 2:
        raise UnsupportedOperator(f"{node.target} at {node.name!r} needs a shape")
    x = cx.tensor(node.args[0])
    dims = tuple(cx.static(a) for a in node.args[1:])
    if len(dims) == 1 and isinstance(dims[0], (tuple, list)):
        dims = tuple(dims[0])
    return cx.emit(node.name, "reshape", (x,), shape=_target_shape(dims, cx.spec(x).shape, node.target))


@_on_method("flatten")
def _flatten_method(cx: _Scope, node):
    return _flatten_fn(cx, node)


@_on_method("transpose")
def _transpose_method(cx: _Scope, node):
    return _transpose_fn(cx, node)


@_on_method("t")
def _t_method(cx: _Scope, node):
    x = cx.tensor(Params("input").bind(node)["input"])
    if len(cx.spec(x).shape) != 2:
        raise UnsupportedOperator(f"t() at {node.name!r} requires a rank-2 tensor")
    return cx.emit(node.name, "transpose", (x,), dim0=0, dim1=1)


@_on_method("softmax")
def _softmax_method(cx: _Scope, node):
    bound = Params("input", "dim", "dtype", dtype=None).bind(node)
    return cx.emit(node.name, "softmax", (cx.tensor(bound["input"]),), dim=_softmax_dim(cx, bound, node.name))


# -- module rules ---------------------------------------------------------------------------------

@_on_module(nn.Identity)
def _identity(cx, node, mod, x):
    return x


@_on_module(nn.Linear)
def _linear_module(cx, node, mod, x):
    return cx.linear(node.name, x, mod.weight.detach().clone(), None if mod.bias is None else mod.bias.detach().clone())


@_on_module(nn.LayerNorm)
def _layer_norm_module(cx, node, mod, x):
    operands = (x,)
    if mod.elementwise_affine:
        if mod.weight is None or mod.bias is None:
            raise UnsupportedOperator(f"partially affine LayerNorm at {node.name!r}")
        operands = (x, cx.hoist(f"{node.name}_weight", mod.weight), cx.hoist(f"{node.name}_bias", mod.bias))
    return cx.emit(node.name, "layer_norm", operands, normalized_shape=tuple(mod.normalized_shape), eps=float(mod.eps))


@_on_module(nn.Conv2d)
def _conv2d_module(cx, node, mod, x):
    if mod.padding_mode != "zeros":
        raise UnsupportedOperator(f"Conv2d padding_mode={mod.padding_mode!r} at {node.name!r} is not supported")
    operands = (x, cx.hoist(f"{node.name}_weight", mod.weight))
    if mod.bias is not None:
        operands += (cx.hoist(f"{node.name}_bias", mod.bias),)
    return cx.emit(node.name, "conv2d", operands, stride=mod.stride, padding=mod.padding, dilation=mod.dilation,
                   groups=mod.groups)


def _embedding_plain(mod: nn.Embedding) -> bool:
    return (mod.padding_idx is None and mod.max_norm is None and mod.norm_type == 2.0
            and not mod.scale_grad_by_freq and not mod.sparse)


@_on_module(nn.Embedding)
def _embedding_module(cx, node, mod, x):
    if not _embedding_plain(mod):
        raise UnsupportedOperator(f"Embedding options at {node.name!r} are not supported in inference lowering")
    return cx.emit(node.name, "embedding", (x, cx.hoist(f"{node.name}_weight", mod.weight)))


@_on_module(nn.Flatten)
def _flatten_module(cx, node, mod, x):
    return cx.emit(node.name, "reshape", (x,),
                   shape=_flattened(cx.spec(x).shape, mod.start_dim, mod.end_dim, f"Flatten at {node.name!r}"))


@_on_module(nn.GELU)
def _gelu_module(cx, node, mod, x):
    return cx.emit(node.name, "gelu", (x,), approximate=mod.approximate)


@_on_module(nn.ReLU)
def _relu_module(cx, node, mod, x):
    if mod.inplace:
        raise UnsupportedOperator(f"in-place ReLU at {node.name!r} is not supported")
    return cx.emit(node.name, "relu", (x,))


@_on_module(nn.Softmax)
def _softmax_module(cx, node, mod, x):
    if mod.dim is None:
        raise UnsupportedOperator(f"Softmax at {node.name!r} has no static dim")
    return cx.emit(node.name, "softmax", (x,), dim=mod.dim)


# -- driver --------------------------------------------------------------------------------------

def _refuse_training_state(model: nn.Module) -> None:
    for m in model.modules():
        if m.training and isinstance(m, (nn.modules.dropout._DropoutNd, nn.modules.batchnorm._BatchNorm)):
            raise GraphError(f"module {type(m).__name__} is in training mode; call model.eval() before compiling")
        if isinstance(m, nn.Conv2d) and m.padding_mode != "zeros":
            raise UnsupportedOperator(f"Conv2d padding_mode={m.padding_mode!r} is not supported")
        if isinstance(m, nn.Embedding) and not _embedding_plain(m):
            raise UnsupportedOperator(
                "Embedding options padding_idx/max_norm/norm_type/scale_grad_by_freq/sparse are not supported")


def _submodule(root: nn.Module, path: str) -> Any:
    obj: Any = root
    for part in path.split("."):
        if not isinstance(obj, (nn.Module, torch.Tensor)) or not hasattr(obj, part):
            raise GraphError(f"cannot resolve attribute {path!r}")
        obj = getattr(obj, part)
    return obj


def _lower_call(cx: _Scope, traced: torch.fx.GraphModule, node: torch.fx.Node):
    if node.op == "get_attr":
        value = _submodule(traced, node.target)
        if not isinstance(value, torch.Tensor):
            raise GraphError(f"attribute {node.target!r} is not a tensor")
        return cx.constant(node.name, value.detach().clone().contiguous())
    if node.op == "call_function":
        rule = _FUNCTION_RULES.get(node.target)
        if rule is None:
            raise UnsupportedOperator(f"unsupported function {getattr(node.target, '__name__', node.target)!r} "
                                      f"at {node.name!r}")
        return rule(cx, node)
    if node.op == "call_method":
        rule = _METHOD_RULES.get(node.target)
        if rule is None:
            raise UnsupportedOperator(f"unsupported method {node.target!r} at {node.name!r}")
        return rule(cx, node)
    if node.op == "call_module":
        mod = _submodule(traced, node.target)
        x = cx.tensor(Params("input").bind(node)["input"])
        for kind, rule in _MODULE_RULES:
            if isinstance(mod, kind):
                return rule(cx, node, mod, x)
        raise UnsupportedOperator(f"unsupported module {type(mod).__name__} at {node.name!r}")
    raise UnsupportedOperator(f"unsupported fx node op {node.op!r} at {node.name!r}")


def _outputs(cx: _Scope, result: Any) -> tuple[tuple[str, ...], bool]:
    def produced(r) -> str | None:
        bound = cx.env.get(r.name) if isinstance(r, torch.fx.Node) else None
        return None if bound is None or isinstance(bound, Static) else bound

    if isinstance(result, torch.fx.Node):
        name = produced(result)
        if name is None:
            raise UnsupportedOperator("model outputs must be produced tensors; static values are not supported")
        return (name,), False
    if isinstance(result, tuple):
        names = tuple(produced(r) for r in result)
        if any(n is None for n in names):
            raise UnsupportedOperator("only flat tuples of produced tensors are supported as outputs")
        return names, True
    raise UnsupportedOperator(
        f"unsupported output type {type(result).__name__}; only a tensor or flat tuple of tensors is supported")


def from_torch(model: torch.nn.Module, example_inputs: tuple[torch.Tensor, ...]) -> Graph:
    """Trace ``model`` with torch.fx and lower it to the IR for these example inputs."""
    if not isinstance(model, nn.Module):
        raise GraphError("from_torch expects an nn.Module")
    for i, t in enumerate(example_inputs):
        if not isinstance(t, torch.Tensor):
            raise GraphError(f"example input {i} is not a tensor")
    _refuse_training_state(model)
    try:
        traced = torch.fx.symbolic_trace(model)
    except Exception as e:  # noqa: BLE001 - any tracing failure means the model is not lowerable
        raise UnsupportedOperator(f"symbolic trace failed: {e}") from e
    placeholders = [n for n in traced.graph.nodes if n.op == "placeholder"]
    if len(placeholders) != len(example_inputs):
        raise GraphError(f"model expects {len(placeholders)} inputs, got {len(example_inputs)} example inputs")
    specs = {f"input_{i}": TensorSpec(tuple(t.shape), t.dtype, str(t.device)) for i, t in enumerate(example_inputs)}
    with torch.no_grad():
        cx = _Scope(specs)
        cx.env.update({ph.name: f"input_{i}" for i, ph in enumerate(placeholders)})
        for node in traced.graph.nodes:
            if node.op == "placeholder":
                continue
            if node.op == "output":
                names, as_tuple = _outputs(cx, node.args[0])
                return cx.builder.finish(names, output_is_tuple=as_tuple)
            cx.env[node.name] = _lower_call(cx, traced, node)
    raise GraphError("traced graph has no output node")
