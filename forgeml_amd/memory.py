"""Slot arena planning for compiled graphs.

Same contract as ForgeML's planner (src/forgeml/memory.py:59-138), which the
executor relies on when it writes GEMM results straight into slots:

* view ops (reshape/transpose/narrow) alias their source and extend its live
  range to their own last materialising use (memory.py:72-99);
* every non-output node of an out=-capable op gets a flat 1-D slot of
  ceil(bytes/itemsize) elements of its dtype on its device (memory.py:130-134);
* a slot is reused only when its previous tenant's last use is strictly
  before the new value's first definition, choosing the smallest slot that
  fits (best fit; memory.py:120-129), so a kernel never writes over a live
  operand of its own.
"""

from __future__ import annotations

from dataclasses import dataclass

from forgeml_amd.ir import Graph, TensorSpec

VIEW_LIKE_OPS = frozenset({"reshape", "transpose", "narrow"})

# Ops whose result the executor can write through out= into a planned slot.
OUT_CAPABLE_OPS = frozenset(
    {"matmul", "linear", "add", "mul", "relu", "softmax", "gelu", "embedding", "fused_linear_gelu"}
)


@dataclass(frozen=True)
class Allocation:
    slot: int
    size_bytes: int
    first: int
    last: int


@dataclass
class MemoryPlan:
    allocations: dict[str, Allocation]
    aliases: dict[str, str]
    slot_specs: dict[int, TensorSpec]
    naive_bytes: int
    planned_bytes: int

    def to_dict(self) -> dict:
        return {
            "aliases": dict(self.aliases),
            "allocations": {
                k: {"slot": a.slot, "size_bytes": a.size_bytes, "first": a.first, "last": a.last}
                for k, a in self.allocations.items()
            },
            "slot_specs": {str(k): v.to_dict() for k, v in self.slot_specs.items()},
            "naive_bytes": self.naive_bytes,
            "planned_bytes": self.planned_bytes,
        }


def _live_until(graph: Graph) -> dict[str, int]:
    """Last position at which each node's storage is read, following views."""
    position = {n.name: i for i, n in enumerate(graph.nodes)}
    readers: dict[str, list[int]] = {}
    for node in graph.nodes:
        for src in set(node.inputs):
            if src in position:
                readers.setdefault(src, []).append(position[node.name])
    last: dict[str, int] = {}
    # A view's reads count as reads of its source, so resolve views first:
    # walking the nodes backwards visits every consumer before its producer.
    for node in reversed(graph.nodes):
        end = position[node.name]
        for reader in readers.get(node.name, ()):
            consumer = graph.nodes[reader]
            end = max(end, last[consumer.name] if consumer.op in VIEW_LIKE_OPS else reader)
        last[node.name] = end
    return last


def plan_memory(graph: Graph) -> MemoryPlan:
    graph.validate()
    outputs = set(graph.outputs)
    position = {n.name: i for i, n in enumerate(graph.nodes)}
    last_use = _live_until(graph)
    aliases: dict[str, str] = {}
    allocations: dict[str, Allocation] = {}
    slot_specs: dict[int, TensorSpec] = {}
    slot_free_after: dict[int, int] = {}
    naive = 0
    for node in graph.nodes:
        if node.name in outputs:
            continue
        naive += node.spec.nbytes
        if node.op in VIEW_LIKE_OPS:
            aliases[node.name] = node.inputs[0]
            continue
        if node.op not in OUT_CAPABLE_OPS:
            continue
        first = position[node.name]
        need = node.spec.nbytes
        best, best_capacity = None, None
        for slot, spec in slot_specs.items():
            if slot_free_after[slot] >= first:
                continue
            if spec.dtype != node.spec.dtype or spec.device != node.spec.device:
                continue
            capacity = spec.shape[0] * spec.dtype.itemsize
            if capacity >= need and (best is None or capacity < best_capacity):
                best, best_capacity = slot, capacity
        if best is None:
            best = len(slot_specs)
            elements = -(-need // node.spec.dtype.itemsize)
            slot_specs[best] = TensorSpec((elements,), node.spec.dtype, node.spec.device)
        slot_free_after[best] = last_use[node.name]
        allocations[node.name] = Allocation(best, need, first, last_use[node.name])
    planned = sum(s.shape[0] * s.dtype.itemsize for s in slot_specs.values())
    return MemoryPlan(allocations, aliases, slot_specs, naive, planned)
