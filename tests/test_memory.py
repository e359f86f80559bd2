"""Slot planning rules (src/forgeml/memory.py:59-138)."""

import torch

from forgeml_amd.ir import GraphBuilder, TensorSpec
from forgeml_amd.memory import plan_memory


def spec(*shape):
    return TensorSpec(tuple(shape), torch.float32, "cpu")


def test_strict_reuse_only_after_last_use():
    b = GraphBuilder({"x": spec(4), "z": spec(4)})
    b.add("a", "relu", ("x",))
    b.add("b", "relu", ("a",))
    b.add("c", "relu", ("z",))
    b.add("d", "relu", ("c",))
    b.add("y", "add", ("b", "d"))
    plan = plan_memory(b.finish(("y",)))
    assert plan.allocations["c"].slot == plan.allocations["a"].slot
    assert "y" not in plan.allocations
    allocs = list(plan.allocations.values())
    for i, p in enumerate(allocs):
        for q in allocs[i + 1:]:
            if p.slot == q.slot:
                assert p.last < q.first or q.last < p.first


def test_views_alias_and_extend_lifetime():
    b = GraphBuilder({"x": spec(8), "z": spec(2, 4)})
    b.add("a", "relu", ("x",))
    b.add("r", "reshape", ("a",), shape=(2, 4))
    b.add("c", "relu", ("z",))
    b.add("y", "add", ("r", "c"))
    plan = plan_memory(b.finish(("y",)))
    assert plan.aliases == {"r": "a"}
    assert set(plan.allocations) == {"a", "c"}
    assert plan.allocations["a"].last == 3
    assert plan.allocations["a"].slot != plan.allocations["c"].slot
    assert plan.planned_bytes == 64


def test_naive_and_planned_bytes_and_output_only():
    b = GraphBuilder({"x": spec(8), "z": spec(8)})
    b.add("a", "relu", ("x",))
    b.add("b", "relu", ("a",))
    b.add("c", "relu", ("z",))
    b.add("y", "add", ("b", "c"))
    plan = plan_memory(b.finish(("y",)))
    assert plan.naive_bytes == 96 and plan.planned_bytes == 64
    assert plan.to_dict()["allocations"]["a"]["slot"] == 0
    b2 = GraphBuilder({"x": spec(4)})
    b2.add("y", "relu", ("x",))
    plan2 = plan_memory(b2.finish(("y",)))
    assert plan2.naive_bytes == 0 and plan2.planned_bytes == 0


def test_best_fit_prefers_smallest_free_slot():
    b = GraphBuilder({"x": spec(16), "s": spec(4)})
    b.add("big", "relu", ("x",))          # slot 0, 64 B
    b.add("small", "relu", ("s",))        # slot 1, 16 B
    b.add("u", "add", ("big", "big"))     # frees big; u needs 64 B -> new slot
    b.add("v", "add", ("small", "small"))  # frees small
    b.add("w", "relu", ("s",))            # 16 B: best fit is the 16 B slot
    b.add("y", "add", ("w", "v"))
    b.add("out", "add", ("u", "u"))
    plan = plan_memory(b.finish(("y", "out")))
    assert plan.allocations["w"].slot == plan.allocations["small"].slot
