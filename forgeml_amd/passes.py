"""Graph passes that produce the GEMM nodes the gfx950 kernels execute.

A model must compile to the same graph, node names and memory plan as under
ForgeML's ``optimize`` (src/forgeml/passes.py:410-430), whose published
captures pin them.  So the pipeline, the rewrite rules and the generated
names are ForgeML's:

1. dead-node elimination;
2. constant folding of nodes whose inputs are all constants, views always,
   other ops while input and output stay within 64 MiB;
3. algebraic simplification: identity reshapes and transposes vanish, a
   reshape of a reshape reads the first one's source, an inverse transpose
   pair vanishes;
4. common-subexpression elimination (``add`` / ``mul`` operands unordered);
5. ``canonicalize_linear``: ``matmul`` + 1-D output-width bias ``add`` ->
   ``linear`` (passes.py:164-201);
6. ``fuse_linear_gelu``: ``gelu`` of a ``linear`` / ``matmul`` (or of a
   ``matmul`` + constant bias ``add``) whose result nothing else reads ->
   ``fused_linear_gelu`` under the gelu's name (passes.py:204-265);
7. ``fuse_shared_projections``: ``linear`` nodes with constant weights that
   read the same input -> one wide ``<leader>_shared_<n>`` linear plus
   ``narrow`` views under the members' names (passes.py:268-339): the fused
   QKV projection;
8. ``schedule``: among six greedy topological orders, the one with the
   smallest planned arena, then the lexicographically smallest names
   (passes.py:342-407).

How it is built here: every pass works on a ``_Work`` copy of the graph (an
ordered node list, an alias map that later nodes are read through, and
consumer counts), rewrites in one sweep, and commits a validated ``Graph``
whose constants are pruned to what is still read.
"""

from __future__ import annotations

from collections import Counter
from collections.abc import Callable
from dataclasses import dataclass

import torch

from forgeml_amd.ir import Graph, GraphError, Node, TensorSpec
from forgeml_amd.memory import VIEW_LIKE_OPS, plan_memory
from forgeml_amd.ops import evaluate

FOLD_LIMIT_BYTES = 64 * 1024 * 1024


@dataclass(frozen=True)
class PassRecord:
    name: str
    nodes_before: int
    nodes_after: int


class _Work:
    """A graph being rewritten."""

    def __init__(self, graph: Graph):
        self.source = graph
        self.constants = dict(graph.constants)
        self.nodes: list[Node] = []
        self._alias: dict[str, str] = {}

    # Names read by later nodes go through the alias map.
    def alias(self, name: str, target: str) -> None:
        self._alias[name] = target

    def resolve(self, name: str) -> str:
        seen = name
        while seen in self._alias and self._alias[seen] != seen:
            seen = self._alias[seen]
        return seen

    def keep(self, node: Node) -> Node:
        node = Node(node.name, node.op, tuple(self.resolve(i) for i in node.inputs), dict(node.attrs), node.spec)
        self.nodes.append(node)
        return node

    def commit(self, *, prune_constants: bool = True, outputs: tuple[str, ...] | None = None) -> Graph:
        outs = tuple(self.resolve(o) for o in (self.source.outputs if outputs is None else outputs))
        constants = self.constants
        if prune_constants:
            read = {i for n in self.nodes for i in n.inputs} | set(outs)
            constants = {k: v for k, v in constants.items() if k in read}
        graph = Graph(inputs=dict(self.source.inputs), constants=constants, nodes=list(self.nodes), outputs=outs,
                      output_is_tuple=self.source.output_is_tuple)
        graph.validate()
        return graph


def _readers(graph: Graph) -> Counter:
    """How many node inputs read each name (a node reading a name twice counts twice)."""
    return Counter(i for n in graph.nodes for i in n.inputs)


def _sole_reader(graph: Graph, readers: Counter, name: str) -> bool:
    """The value feeds exactly one input slot and is not a graph output."""
    return readers[name] == 1 and name not in graph.outputs


# -- clean-up passes --------------------------------------------------------------

def eliminate_dead_nodes(graph: Graph) -> Graph:
    """Drop nodes and constants the outputs do not depend on."""
    producer = {n.name: n for n in graph.nodes}
    live: set[str] = set()
    stack = list(graph.outputs)
    while stack:
        name = stack.pop()
        if name in live:
            continue
        live.add(name)
        if name in producer:
            stack.extend(producer[name].inputs)
    work = _Work(graph)
    work.nodes = [n for n in graph.nodes if n.name in live]
    work.constants = {k: v for k, v in graph.constants.items() if k in live}
    return work.commit(prune_constants=False)


def _foldable(node: Node, known: dict[str, torch.Tensor]) -> bool:
    if not all(i in known for i in node.inputs):
        return False
    if node.op in VIEW_LIKE_OPS:
        return True  # a view materialises nothing
    read = sum(known[i].numel() * known[i].element_size() for i in set(node.inputs))
    return node.spec.nbytes <= FOLD_LIMIT_BYTES and read <= FOLD_LIMIT_BYTES


def fold_constants(graph: Graph) -> Graph:
    """Evaluate, once, every node computable from constants (within the size cap)."""
    work = _Work(graph)
    for node in graph.nodes:
        if not _foldable(node, work.constants):
            work.nodes.append(node)
            continue
        try:
            with torch.inference_mode():
                work.constants[node.name] = evaluate(node.op, tuple(work.constants[i] for i in node.inputs),
                                                     dict(node.attrs))
        except Exception as e:  # noqa: BLE001 - report which node could not be folded
            raise GraphError(f"constant folding failed at node {node.name!r}: {e}") from e
    return work.commit()


# Peephole rules of simplify_algebra: given the node (inputs already
# resolved) and the kept producers, return the name it is an alias of, a
# replacement node, or the node itself.
def _simplify_reshape(node: Node, producer: Node | None, specs) -> str | Node:
    if specs[node.inputs[0]].shape == node.spec.shape:
        return node.inputs[0]
    if producer is not None and producer.op == "reshape":
        return Node(node.name, "reshape", producer.inputs, dict(node.attrs), node.spec)
    return node


def _transpose_axes(node: Node, rank: int) -> frozenset:
    return frozenset((node.attrs["dim0"] % rank, node.attrs["dim1"] % rank))


def _simplify_transpose(node: Node, producer: Node | None, specs) -> str | Node:
    rank = len(node.spec.shape)
    axes = _transpose_axes(node, rank)
    if len(axes) == 1:
        return node.inputs[0]
    if producer is not None and producer.op == "transpose" and _transpose_axes(producer, rank) == axes:
        return producer.inputs[0]
    return node


_PEEPHOLES: dict[str, Callable] = {"reshape": _simplify_reshape, "transpose": _simplify_transpose}


def simplify_algebra(graph: Graph) -> Graph:
    specs = graph.specs()
    work = _Work(graph)
    kept: dict[str, Node] = {}
    for original in graph.nodes:
        node = Node(original.name, original.op, tuple(work.resolve(i) for i in original.inputs),
                    dict(original.attrs), original.spec)
        rule = _PEEPHOLES.get(node.op)
        result = node if rule is None else rule(node, kept.get(node.inputs[0]), specs)
        if isinstance(result, str):
            work.alias(node.name, work.resolve(result))
            continue
        kept[result.name] = work.keep(result)
    return eliminate_dead_nodes(work.commit(prune_constants=False))


def _frozen(value):
    if isinstance(value, dict):
        return tuple(sorted((k, _frozen(v)) for k, v in value.items()))
    if isinstance(value, (list, tuple)):
        return tuple(_frozen(v) for v in value)
    return value


_COMMUTATIVE = frozenset({"add", "mul"})


def common_subexpression_elimination(graph: Graph) -> Graph:
    work = _Work(graph)
    first: dict[tuple, str] = {}
    for node in graph.nodes:
        inputs = tuple(work.resolve(i) for i in node.inputs)
        key = (node.op, tuple(sorted(inputs)) if node.op in _COMMUTATIVE else inputs, _frozen(node.attrs), node.spec)
        if key in first:
            work.alias(node.name, first[key])
        else:
            first[key] = node.name
            work.keep(node)
    return work.commit()


# -- the GEMM rewrites -------------------------------------------------------------------

def _replace_and_drop(graph: Graph, replaced: dict[str, Node], dropped: set[str]) -> Graph:
    work = _Work(graph)
    work.nodes = [replaced.get(n.name, n) for n in graph.nodes if n.name not in dropped]
    return work.commit()


def canonicalize_linear(graph: Graph) -> Graph:
    """add(matmul(x, w), b) with b 1-D of the output width -> linear(x, w, b)."""
    producer = {n.name: n for n in graph.nodes}
    readers = _readers(graph)
    specs = graph.specs()
    replaced: dict[str, Node] = {}
    dropped: set[str] = set()
    for node in graph.nodes:
        if node.op != "add":
            continue
        a, b = node.inputs
        for gemm_name, bias in ((a, b), (b, a)):
            gemm = producer.get(gemm_name)
            if gemm is None or gemm.op != "matmul" or not _sole_reader(graph, readers, gemm_name):
                continue
            bias_shape = specs[bias].shape if bias in specs else None
            if bias_shape is None or len(bias_shape) != 1 or bias_shape[0] != gemm.spec.shape[1]:
                continue
            replaced[node.name] = Node(node.name, "linear", gemm.inputs + (bias,), {}, node.spec)
            dropped.add(gemm_name)
            break
    return _replace_and_drop(graph, replaced, dropped)


def _matmul_plus_constant_bias(graph: Graph, producer: dict[str, Node], add: Node):
    """(matmul node, bias name) when ``add`` is matmul + a constant, else None."""
    a, b = add.inputs
    for gemm_name, bias in ((a, b), (b, a)):
        gemm = producer.get(gemm_name)
        if gemm is not None and gemm.op == "matmul" and bias in graph.constants:
            return gemm, bias
    return None


def fuse_linear_gelu(graph: Graph) -> Graph:
    """gelu(linear | matmul) and gelu(matmul + constant bias) -> fused_linear_gelu.

    The fused node keeps the gelu node's name, spec and ``approximate``.
    """
    producer = {n.name: n for n in graph.nodes}
    readers = _readers(graph)
    replaced: dict[str, Node] = {}
    dropped: set[str] = set()

    def fused(gelu: Node, operands: tuple[str, ...]) -> Node:
        return Node(gelu.name, "fused_linear_gelu", operands, {"approximate": gelu.attrs.get("approximate", "none")},
                    gelu.spec)

    for node in graph.nodes:
        if node.op != "gelu" or len(node.inputs) != 1 or node.inputs[0] not in producer:
            continue
        src = producer[node.inputs[0]]
        if not _sole_reader(graph, readers, src.name):
            continue
        if src.op in ("linear", "matmul"):
            replaced[node.name] = fused(node, src.inputs)
            dropped.add(src.name)
            continue
        if src.op != "add":
            continue
        match = _matmul_plus_constant_bias(graph, producer, src)
        if match is None:
            continue
        gemm, bias = match
        bias_value = graph.constants[bias]
        if (not _sole_reader(graph, readers, gemm.name) or bias_value.dim() != 1 or len(gemm.spec.shape) != 2
                or bias_value.shape[0] != gemm.spec.shape[1]):
            continue
        replaced[node.name] = fused(node, (gemm.inputs[0], gemm.inputs[1], bias))
        dropped.update((gemm.name, src.name))
    return _replace_and_drop(graph, replaced, dropped)


class _Namer:
    """``<hint>_<n>`` names from one counter, skipping names already taken."""

    def __init__(self, taken):
        self.taken = set(taken)
        self.serial = 0

    def __call__(self, hint: str) -> str:
        while True:
            self.serial += 1
            name = f"{hint}_{self.serial}"
            if name not in self.taken:
                self.taken.add(name)
                return name


def _projection_groups(graph: Graph) -> list[list[Node]]:
    """Linear nodes with constant parameters grouped by (input, arity), in graph order."""
    groups: dict[tuple[str, int], list[Node]] = {}
    for node in graph.nodes:
        if node.op != "linear" or not all(p in graph.constants for p in node.inputs[1:]):
            continue
        groups.setdefault((node.inputs[0], len(node.inputs)), []).append(node)
    return [members for members in groups.values() if len(members) > 1]


def fuse_shared_projections(graph: Graph) -> Graph:
    """Linears reading the same input with constant weights -> one wide GEMM.

    Members are concatenated along N in graph order into a ``<leader>_shared``
    linear emitted at the leader's position; each member becomes a
    ``narrow`` view of it (so the fused QKV projection is one kernel launch
    with N = 3 * d_model).
    """
    groups = _projection_groups(graph)
    if not groups:
        return _replace_and_drop(graph, {}, set())
    name = _Namer(set(graph.inputs) | set(graph.constants) | {n.name for n in graph.nodes})
    constants = dict(graph.constants)
    specs = graph.specs()
    at_leader: dict[str, list[Node]] = {}
    dropped: set[str] = set()
    for members in groups:
        leader = members[0]
        with_bias = len(leader.inputs) == 3
        parts = [[constants[m.inputs[j]] for m in members] for j in range(1, len(leader.inputs))]
        if any(len({t.dtype for t in part}) > 1 for part in parts):
            continue
        operands = [leader.inputs[0]]
        weight = name(f"{leader.name}_shared_weight")
        constants[weight] = torch.cat(parts[0], dim=1).contiguous()
        operands.append(weight)
        if with_bias:
            bias = name(f"{leader.name}_shared_bias")
            constants[bias] = torch.cat(parts[1])
            operands.append(bias)
        x = specs[leader.inputs[0]]
        widths = [m.spec.shape[1] for m in members]
        wide = name(f"{leader.name}_shared")
        emitted = [Node(wide, "linear", tuple(operands), {}, TensorSpec((x.shape[0], sum(widths)), x.dtype, x.device))]
        starts = [sum(widths[:i]) for i in range(len(members))]
        for member, start, width in zip(members, starts, widths):
            emitted.append(Node(member.name, "narrow", (wide,), {"dim": 1, "start": start, "length": width},
                                member.spec))
            dropped.add(member.name)
        at_leader[leader.name] = emitted
    work = _Work(graph)
    work.constants = constants
    for node in graph.nodes:
        if node.name in at_leader:
            work.nodes.extend(at_leader[node.name])
        elif node.name not in dropped:
            work.nodes.append(node)
    return work.commit(prune_constants=False)


# -- scheduling --------------------------------------------------------------------------

class _ListScheduler:
    """Greedy topological ordering: repeatedly emit the ready node of highest priority.

    A priority sees the node, its position in the input order and ``freed``:
    the bytes of its inputs that no later node reads (graph outputs are never
    freed).
    """

    def __init__(self, graph: Graph):
        self.graph = graph
        self.position = {n.name: i for i, n in enumerate(graph.nodes)}
        self.specs = graph.specs()
        self.readers_of: dict[str, list[str]] = {}
        for node in graph.nodes:
            for src in dict.fromkeys(node.inputs):
                self.readers_of.setdefault(src, []).append(node.name)

    def order(self, priority: Callable[[Node, int, int], tuple]) -> list[Node]:
        graph, position, specs = self.graph, self.position, self.specs
        by_name = {n.name: n for n in graph.nodes}
        unmet = {n.name: len({i for i in n.inputs if i in position}) for n in graph.nodes}
        unread = {name: len(readers) for name, readers in self.readers_of.items() if name in position}
        outputs = set(graph.outputs)

        def freed(node: Node) -> int:
            return sum(specs[i].nbytes for i in set(node.inputs)
                       if i in position and i not in outputs and unread.get(i) == 1)

        ready = [n for n in graph.nodes if unmet[n.name] == 0]
        emitted: list[Node] = []
        while ready:
            best = max(range(len(ready)), key=lambda j: priority(ready[j], position[ready[j].name], freed(ready[j])))
            node = ready.pop(best)
            emitted.append(node)
            for reader in sorted(self.readers_of.get(node.name, ())):
                unmet[reader] -= 1
                if unmet[reader] == 0:
                    ready.append(by_name[reader])
            for i in set(node.inputs):
                if i in unread:
                    unread[i] -= 1
        if len(emitted) != len(graph.nodes):
            raise GraphError("graph contains a cycle")
        return emitted


# The six priorities tried (each ends in a unique position term, so no two
# ready nodes tie): trade freed bytes against the bytes a node allocates at
# three weights, allocate-smallest-first, and the input order and its reverse.
_PRIORITIES: tuple[Callable[[Node, int, int], tuple], ...] = (
    lambda n, pos, freed: (freed - n.spec.nbytes, -pos),
    lambda n, pos, freed: (freed - 2 * n.spec.nbytes, -pos),
    lambda n, pos, freed: (freed - n.spec.nbytes // 2, -pos),
    lambda n, pos, freed: (-n.spec.nbytes, freed, -pos),
    lambda n, pos, freed: (-pos,),
    lambda n, pos, freed: (pos,),
)


def schedule(graph: Graph) -> Graph:
    """Reorder nodes for the smallest planned arena (ties: lexicographic names)."""
    scheduler = _ListScheduler(graph)
    orders: dict[tuple[str, ...], list[Node]] = {}
    for priority in _PRIORITIES:
        order = scheduler.order(priority)
        orders.setdefault(tuple(n.name for n in order), order)

    def arena_bytes(names: tuple[str, ...]) -> int:
        work = _Work(graph)
        work.nodes = orders[names]
        return plan_memory(work.commit(prune_constants=False)).planned_bytes

    best = min(orders, key=lambda names: (arena_bytes(names), names))
    work = _Work(graph)
    work.nodes = orders[best]
    return work.commit(prune_constants=False)


PIPELINE = (
    ("eliminate_dead_nodes", eliminate_dead_nodes),
    ("fold_constants", fold_constants),
    ("eliminate_dead_nodes", eliminate_dead_nodes),
    ("simplify_algebra", simplify_algebra),
    ("common_subexpression_elimination", common_subexpression_elimination),
    ("canonicalize_linear", canonicalize_linear),
    ("fuse_linear_gelu", fuse_linear_gelu),
    ("fuse_shared_projections", fuse_shared_projections),
    ("eliminate_dead_nodes", eliminate_dead_nodes),
    ("schedule", schedule),
)


def optimize(graph: Graph) -> tuple[Graph, list[PassRecord]]:
    """Run the pipeline on a copy of ``graph``; records node counts per pass."""
    graph.validate()
    current = graph.clone()
    records: list[PassRecord] = []
    for name, run in PIPELINE:
        before = len(current.nodes)
        current = run(current)
        current.validate()
        records.append(PassRecord(name, before, len(current.nodes)))
    return current, records
