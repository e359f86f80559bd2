"""Per-node tile selection with a correctness gate before any timing.

Follows ForgeML's ``tune_graph`` (src/forgeml/autotune.py:16-103): each GEMM
node planned for the GPU kernel is evaluated once with the torch path for its
expected value; every candidate tile is launched into a fresh output and must
pass ``check_output`` before it may be timed; a launch that raises is
recorded as a rejection; the lowest median wins (first candidate on ties);
downstream nodes receive the torch value as input.  The winners are stored
in ``compiled.kernel_configs`` for this compiled model only (no cache).

The candidate set is the MI355X tile table built for the node's dtype
(``kernels.candidates``), not Triton meta-parameters.
"""

from __future__ import annotations

from dataclasses import asdict
from typing import TYPE_CHECKING

import torch

from forgeml_amd import kernels
from forgeml_amd.measurement import check_output, measure_variants
from forgeml_amd.ops import evaluate

if TYPE_CHECKING:
    from forgeml_amd.compiler import CompiledModel


@torch.inference_mode()
def tune_graph(
    compiled: CompiledModel,
    inputs: tuple[torch.Tensor, ...],
    *,
    warmup: int = 3,
    repeats: int = 10,
) -> dict:
    if warmup < 0 or repeats < 2:
        raise ValueError("autotuning requires warmup >= 0 and repeats >= 2")
    compiled(*inputs)
    values = dict(compiled.graph.constants)
    values.update(zip(compiled.graph.inputs, inputs))
    records: dict = {}
    chosen: dict = {}
    for node in compiled.graph.nodes:
        args = tuple(values[name] for name in node.inputs)
        expected = evaluate(node.op, args, node.attrs)
        if compiled.kernel_plan.get(node.name) == "hip" and node.op in kernels.GEMM_OPS:
            bias = args[2] if len(args) == 3 else None
            activation = "gelu" if node.op == "fused_linear_gelu" else "none"
            approximate = node.attrs.get("approximate", "none") if activation == "gelu" else "none"
            variants, configs, rejected, errors = {}, {}, {}, {}
            for index, config in enumerate(kernels.candidates(args[0].dtype)):
                name = f"candidate_{index}"

                def launch(config=config, args=args, bias=bias, activation=activation, approximate=approximate):
                    return kernels.matmul(
                        args[0], args[1], bias, activation=activation, approximate=approximate, config=config
                    )

                try:
                    errors[name] = check_output(launch(), expected)
                except Exception as exc:  # noqa: BLE001 - any failure rejects the candidate
                    rejected[name] = str(exc)
                    continue
                variants[name] = launch
                configs[name] = config
            if not variants:
                raise RuntimeError(f"no numerically valid kernel candidate for {node.name!r}")
            timings = measure_variants(variants, device=args[0].device, warmup=warmup, repeats=repeats)
            winner = min(timings, key=lambda name: timings[name]["median_ms"])
            chosen[node.name] = configs[winner]
            records[node.name] = {
                "winner": winner,
                "config": asdict(configs[winner]),
                "candidates": {
                    name: {"config": asdict(configs[name]), "timing": timing, "correctness": errors[name]}
                    for name, timing in timings.items()
                },
                "rejected": rejected,
                "input_shapes": [list(arg.shape) for arg in args],
                "input_strides": [list(arg.stride()) for arg in args],
                "dtype": str(args[0].dtype),
                "device": str(args[0].device),
                "activation": activation,
                "approximate": approximate,
            }
        values[node.name] = expected
    compiled.kernel_configs.update(chosen)
    return {
        "scope": "this_compiled_model_instance_only",
        "timing": "synchronized_host_wall_clock_including_output_allocation",
        "warmup": warmup,
        "repeats": repeats,
        "nodes": records,
    }
