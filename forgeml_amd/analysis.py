"""Static operator cost model reported by ``CompiledModel.explain()``.

Counts follow ForgeML's model (src/forgeml/analysis.py:14-105) so explain()
output matches the reference's captures: a GEMM is 2*M*N*K, a bias add is
M*N, and GELU is charged 8 flops per element.  These are bookkeeping figures
for plans, not hardware measurements; kernel rooflines use 2*M*N*K only.
"""

from __future__ import annotations

import math
from collections import Counter

from forgeml_amd.ir import Graph, Node, TensorSpec
from forgeml_amd.memory import VIEW_LIKE_OPS

_ELEMENTWISE_FLOPS = {"add": 1, "mul": 1, "relu": 1, "gelu": 8, "softmax": 5, "layer_norm": 6}


def node_flops(node: Node, inputs: list[TensorSpec]) -> int:
    elements = math.prod(node.spec.shape)
    op = node.op
    if op in ("matmul", "linear", "fused_linear_gelu"):
        (m, k), n = inputs[0].shape, inputs[1].shape[1]
        flops = 2 * m * k * n
        if op != "matmul" and len(inputs) == 3:
            flops += elements
        if op == "fused_linear_gelu":
            flops += 8 * elements
        return flops
    if op in _ELEMENTWISE_FLOPS:
        return _ELEMENTWISE_FLOPS[op] * elements
    if op == "sdpa":
        batch, heads, q_len, head_dim = inputs[0].shape
        kv_len = inputs[1].shape[2]
        pairs = batch * heads * q_len * kv_len
        if node.attrs.get("is_causal"):
            pairs = min(pairs, batch * heads * (q_len * (q_len + 1) // 2))
        return 4 * pairs * head_dim + (6 if len(inputs) == 4 else 5) * pairs
    if op == "conv2d":
        _, _, out_h, out_w = node.spec.shape
        out_c, in_per_group, kh, kw = inputs[1].shape
        flops = 2 * inputs[0].shape[0] * out_h * out_w * out_c * in_per_group * kh * kw
        return flops + (elements if len(inputs) == 3 else 0)
    return 0


def graph_analysis(graph: Graph) -> dict:
    graph.validate()
    specs = graph.specs()
    rows = []
    depth: dict[str, int] = {}
    total_flops = total_bytes = 0
    for node in graph.nodes:
        in_specs = [specs[s] for s in node.inputs]
        flops = node_flops(node, in_specs)
        # Views move no data; their traffic is charged to the consumer.
        logical = 0 if node.op in VIEW_LIKE_OPS else (
            sum(specs[s].nbytes for s in dict.fromkeys(node.inputs)) + node.spec.nbytes
        )
        depth[node.name] = 1 + max((depth.get(s, 0) for s in node.inputs), default=0)
        rows.append(
            {
                "name": node.name,
                "op": node.op,
                "flops": flops,
                "logical_bytes": logical,
                "arithmetic_intensity": flops / max(logical, 1),
                "depth": depth[node.name],
                "output_shape": list(node.spec.shape),
            }
        )
        total_flops += flops
        total_bytes += logical
    return {
        "model": "static_operator_cost_bounds_not_measured_hardware_counters",
        "nodes": len(graph.nodes),
        "op_counts": dict(sorted(Counter(n.op for n in graph.nodes).items())),
        "flops": total_flops,
        "logical_bytes": total_bytes,
        "arithmetic_intensity": total_flops / max(total_bytes, 1),
        "critical_path_ops": max(depth.values(), default=0),
        "input_bytes": sum(s.nbytes for s in graph.inputs.values()),
        "constant_bytes": sum(t.numel() * t.element_size() for t in graph.constants.values()),
        "output_bytes": sum(specs[name].nbytes for name in graph.outputs),
        "dominant_nodes": sorted(rows, key=lambda r: (r["flops"], r["logical_bytes"], r["name"]), reverse=True)[:5],
        "per_node": rows,
    }
