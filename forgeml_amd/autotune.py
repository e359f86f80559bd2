"""Per-node tile selection: a correctness gate first, then timing.

The contract is ForgeML's ``tune_graph`` (src/forgeml/autotune.py:16-103):

* the compiled model runs once, then the graph is walked with torch values,
  so every GEMM node is tuned on the inputs it sees in a real call and
  downstream nodes receive the torch result;
* each candidate launches into a fresh output and must pass the gate
  (``measurement.check_output`` against the torch value) before it may be
  timed; an exception from the launch or the gate rejects it;
* the winner is the lowest median latency, the earliest candidate on ties,
  and is stored in ``compiled.kernel_configs`` of this instance only;
* the report keeps the reference's schema (``scope``, ``timing``,
  ``warmup``, ``repeats``, ``nodes[*]`` with ``winner``, ``config``,
  ``candidates``, ``rejected``, input shapes and strides, dtype, device,
  activation, approximate).

The search space is the tile table built for the node's dtype
(``kernels.candidates``).
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import asdict, dataclass
from typing import TYPE_CHECKING

import torch

from forgeml_amd import kernels
from forgeml_amd.kernels import KernelConfig
from forgeml_amd.measurement import check_output, measure_variants
from forgeml_amd.ops import evaluate

if TYPE_CHECKING:
    from forgeml_amd.compiler import CompiledModel


@dataclass(frozen=True)
class _GemmNode:
    """A GEMM node's operands as a tuning call sees them."""

    a: torch.Tensor
    b: torch.Tensor
    bias: torch.Tensor | None
    activation: str
    approximate: str

    @classmethod
    def of(cls, node, args: tuple[torch.Tensor, ...]) -> "_GemmNode":
        gelu = node.op == "fused_linear_gelu"
        return cls(args[0], args[1], args[2] if len(args) == 3 else None,
                   "gelu" if gelu else "none", node.attrs.get("approximate", "none") if gelu else "none")

    def launcher(self, config: KernelConfig) -> Callable[[], torch.Tensor]:
        # kernels.matmul is looked up at call time, so a replacement installed
        # on the module (tests do this) is what runs.
        return lambda: kernels.matmul(self.a, self.b, self.bias, activation=self.activation,
                                      approximate=self.approximate, config=config)

    def describe(self, args) -> dict:
        return {
            "input_shapes": [list(t.shape) for t in args],
            "input_strides": [list(t.stride()) for t in args],
            "dtype": str(self.a.dtype),
            "device": str(self.a.device),
            "activation": self.activation,
            "approximate": self.approximate,
        }


def _gate(call: _GemmNode, expected: torch.Tensor):
    """Launch every candidate once against ``expected``: (passing, rejected)."""
    passing: dict[str, tuple[KernelConfig, Callable, dict]] = {}
    rejected: dict[str, str] = {}
    for idx, config in enumerate(kernels.candidates(call.a.dtype)):
        label = f"candidate_{idx}"
        launch = call.launcher(config)
        try:
            verdict = check_output(launch(), expected)
        except Exception as exc:  # noqa: BLE001 - a launch or gate failure rejects this candidate only
            rejected[label] = str(exc)
        else:
            passing[label] = (config, launch, verdict)
    return passing, rejected


def _winner(timings: dict[str, dict], order: list[str]) -> str:
    return min(order, key=lambda label: (timings[label]["median_ms"], order.index(label)))


@torch.inference_mode()
def tune_graph(compiled: CompiledModel, inputs: tuple[torch.Tensor, ...], *, warmup: int = 3,
               repeats: int = 10) -> dict:
    """Gate, time and pick a tile for every hip GEMM node of ``compiled``."""
    if warmup < 0 or repeats < 2:
        raise ValueError("autotuning requires warmup >= 0 and repeats >= 2")
    compiled(*inputs)  # the model must run as compiled before any node is tuned
    env = {**compiled.graph.constants, **dict(zip(compiled.graph.inputs, inputs))}
    nodes_report: dict[str, dict] = {}
    picked: dict[str, KernelConfig] = {}
    for node in compiled.graph.nodes:
        args = tuple(env[name] for name in node.inputs)
        reference = evaluate(node.op, args, node.attrs)
        env[node.name] = reference
        if node.op not in kernels.GEMM_OPS or compiled.kernel_plan.get(node.name) != "hip":
            continue
        call = _GemmNode.of(node, args)
        passing, rejected = _gate(call, reference)
        if not passing:
            raise RuntimeError(f"no numerically valid kernel candidate for {node.name!r}")
        timings = measure_variants({label: launch for label, (_, launch, _) in passing.items()},
                                   device=call.a.device, warmup=warmup, repeats=repeats)
        best = _winner(timings, list(passing))
        picked[node.name] = passing[best][0]
        nodes_report[node.name] = {
            "winner": best,
            "config": asdict(passing[best][0]),
            "candidates": {
                label: {"config": asdict(config), "timing": timings[label], "correctness": verdict}
                for label, (config, _, verdict) in passing.items()
            },
            "rejected": rejected,
            **call.describe(args),
        }
    compiled.kernel_configs.update(picked)
    return {
        "scope": "this_compiled_model_instance_only",
        "timing": "synchronized_host_wall_clock_including_output_allocation",
        "warmup": warmup,
        "repeats": repeats,
        "nodes": nodes_report,
    }
