"""Graph passes that produce the GEMM nodes the gfx950 kernels execute.

The pipeline and every rewrite keep the semantics of ForgeML's
``optimize`` (src/forgeml/passes.py:410-430) so that a model compiles to the
same graph, with the same node names, as under the reference:

1. dead-node elimination (passes.py:33-42)
2. constant folding under a 64 MiB cap (passes.py:45-74)
3. algebraic simplification of reshapes/transposes (passes.py:83-124)
4. common-subexpression elimination (passes.py:135-161)
5. ``canonicalize_linear``: matmul + 1-D bias add -> linear (passes.py:164-201)
6. ``fuse_linear_gelu``: linear/matmul (+ bias add) + gelu -> one
   ``fused_linear_gelu`` node (passes.py:204-265)
7. ``fuse_shared_projections``: linears that share an input and constant
   weights -> one wide linear plus ``narrow`` views (passes.py:268-339), the
   fused QKV projection
8. ``schedule``: the topological order with the smallest planned arena among
   six greedy orders (passes.py:342-407)
"""

from __future__ import annotations

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


def _with_nodes(graph: Graph, nodes: list[Node], constants: dict, outputs=None) -> Graph:
    out = Graph(
        inputs=dict(graph.inputs),
        constants=constants,
        nodes=nodes,
        outputs=tuple(graph.outputs if outputs is None else outputs),
        output_is_tuple=graph.output_is_tuple,
    )
    out.validate()
    return out


def _consumers(graph: Graph) -> dict[str, list[str]]:
    table: dict[str, list[str]] = {}
    for node in graph.nodes:
        for src in node.inputs:
            table.setdefault(src, []).append(node.name)
    return table


def _follow(aliases: dict[str, str], name: str) -> str:
    while aliases.get(name, name) != name:
        name = aliases[name]
    return name


def eliminate_dead_nodes(graph: Graph) -> Graph:
    live = set(graph.outputs)
    kept: list[Node] = []
    for node in reversed(graph.nodes):
        if node.name in live:
            kept.append(node)
            live.update(node.inputs)
    kept.reverse()
    return _with_nodes(graph, kept, {k: v for k, v in graph.constants.items() if k in live})


def fold_constants(graph: Graph) -> Graph:
    constants = dict(graph.constants)
    known = dict(constants)
    nodes: list[Node] = []
    for node in graph.nodes:
        if not all(src in known for src in node.inputs):
            nodes.append(node)
            continue
        # Views materialise nothing; other ops are folded only under the cap,
        # which bounds both compile-time memory and fold compute.
        in_bytes = sum(known[s].numel() * known[s].element_size() for s in dict.fromkeys(node.inputs))
        if node.op not in VIEW_LIKE_OPS and (
            node.spec.nbytes > FOLD_LIMIT_BYTES or in_bytes > FOLD_LIMIT_BYTES
        ):
            nodes.append(node)
            continue
        try:
            with torch.inference_mode():
                value = evaluate(node.op, tuple(known[s] for s in node.inputs), dict(node.attrs))
        except Exception as e:  # noqa: BLE001
            raise GraphError(f"constant folding failed at node {node.name!r}: {e}") from e
        constants[node.name] = value
        known[node.name] = value
    used = {s for n in nodes for s in n.inputs} | set(graph.outputs)
    return _with_nodes(graph, nodes, {k: v for k, v in constants.items() if k in used})


def simplify_algebra(graph: Graph) -> Graph:
    specs = graph.specs()
    aliases: dict[str, str] = {}
    kept: dict[str, Node] = {}
    nodes: list[Node] = []
    for original in graph.nodes:
        inputs = tuple(_follow(aliases, s) for s in original.inputs)
        node = Node(original.name, original.op, inputs, dict(original.attrs), original.spec)
        if node.op == "reshape":
            if specs[node.inputs[0]].shape == node.spec.shape:
                aliases[node.name] = node.inputs[0]  # identity reshape
                continue
            src = kept.get(node.inputs[0])
            if src is not None and src.op == "reshape":  # reshape of reshape
                node = Node(node.name, "reshape", src.inputs, dict(node.attrs), node.spec)
        elif node.op == "transpose":
            rank = len(node.spec.shape)
            dims = frozenset((node.attrs["dim0"] % rank, node.attrs["dim1"] % rank))
            if len(dims) == 1:
                aliases[node.name] = node.inputs[0]  # transpose(d, d)
                continue
            src = kept.get(node.inputs[0])
            if (
                src is not None
                and src.op == "transpose"
                and frozenset((src.attrs["dim0"] % rank, src.attrs["dim1"] % rank)) == dims
            ):
                aliases[node.name] = _follow(aliases, src.inputs[0])  # inverse pair
                continue
        aliases[node.name] = node.name
        kept[node.name] = node
        nodes.append(node)
    outputs = tuple(_follow(aliases, name) for name in graph.outputs)
    rewritten = Graph(
        inputs=dict(graph.inputs),
        constants=dict(graph.constants),
        nodes=nodes,
        outputs=outputs,
        output_is_tuple=graph.output_is_tuple,
    )
    rewritten.validate()
    return eliminate_dead_nodes(rewritten)


def _hashable(value):
    if isinstance(value, (tuple, list)):
        return tuple(_hashable(v) for v in value)
    if isinstance(value, dict):
        return tuple(sorted((k, _hashable(v)) for k, v in value.items()))
    return value


def common_subexpression_elimination(graph: Graph) -> Graph:
    aliases: dict[str, str] = {}
    first_of: dict[tuple, str] = {}
    nodes: list[Node] = []
    for node in graph.nodes:
        inputs = tuple(_follow(aliases, s) for s in node.inputs)
        operands = tuple(sorted(inputs)) if node.op in ("add", "mul") else inputs
        key = (node.op, operands, _hashable(node.attrs), node.spec)
        if key in first_of:
            aliases[node.name] = first_of[key]
            continue
        first_of[key] = node.name
        aliases[node.name] = node.name
        nodes.append(Node(node.name, node.op, inputs, dict(node.attrs), node.spec))
    outputs = tuple(_follow(aliases, name) for name in graph.outputs)
    used = {s for n in nodes for s in n.inputs} | set(outputs)
    return _with_nodes(graph, nodes, {k: v for k, v in graph.constants.items() if k in used}, outputs)


def _only_consumer(graph: Graph, consumers: dict[str, list[str]], name: str) -> bool:
    return name not in graph.outputs and len(consumers.get(name, ())) == 1


def canonicalize_linear(graph: Graph) -> Graph:
    """matmul(x, w) + b with a 1-D output-width b becomes linear(x, w, b)."""
    consumers = _consumers(graph)
    by_name = {n.name: n for n in graph.nodes}
    specs = graph.specs()
    replaced: dict[str, Node] = {}
    dropped: set[str] = set()
    for node in graph.nodes:
        if node.op != "add":
            continue
        x, y = node.inputs
        for mm_name, bias in ((x, y), (y, x)):
            mm = by_name.get(mm_name)
            bias_spec = specs.get(bias)
            if mm is None or mm.op != "matmul" or not _only_consumer(graph, consumers, mm.name):
                continue
            if bias_spec is None or len(bias_spec.shape) != 1 or bias_spec.shape[0] != mm.spec.shape[1]:
                continue
            replaced[node.name] = Node(node.name, "linear", mm.inputs + (bias,), {}, node.spec)
            dropped.add(mm.name)
            break
    nodes = [replaced.get(n.name, n) for n in graph.nodes if n.name not in dropped]
    used = {s for n in nodes for s in n.inputs}
    return _with_nodes(
        graph, nodes, {k: v for k, v in graph.constants.items() if k in used or k in graph.outputs}
    )


def fuse_linear_gelu(graph: Graph) -> Graph:
    """gelu(linear|matmul) and gelu(matmul + const bias) become fused_linear_gelu.

    The fused node keeps the gelu node's name, spec and ``approximate``.
    """
    consumers = _consumers(graph)
    by_name = {n.name: n for n in graph.nodes}
    replaced: dict[str, Node] = {}
    dropped: set[str] = set()
    for node in graph.nodes:
        if node.op != "gelu" or len(node.inputs) != 1:
            continue
        approximate = node.attrs.get("approximate", "none")
        producer = by_name.get(node.inputs[0])
        if producer is None:
            continue
        if producer.op in ("linear", "matmul"):
            if _only_consumer(graph, consumers, producer.name):
                replaced[node.name] = Node(
                    node.name, "fused_linear_gelu", producer.inputs, {"approximate": approximate}, node.spec
                )
                dropped.add(producer.name)
            continue
        if producer.op != "add" or not _only_consumer(graph, consumers, producer.name):
            continue
        match = None
        for mm_name, bias in ((producer.inputs[0], producer.inputs[1]), (producer.inputs[1], producer.inputs[0])):
            mm = by_name.get(mm_name)
            if mm is not None and mm.op == "matmul" and bias in graph.constants:
                match = (mm, bias)
                break
        if match is None:
            continue
        mm, bias = match
        if not _only_consumer(graph, consumers, mm.name):
            continue
        bias_t = graph.constants[bias]
        if bias_t.dim() != 1 or bias_t.shape[0] != mm.spec.shape[1] or len(mm.spec.shape) != 2:
            continue
        replaced[node.name] = Node(
            node.name,
            "fused_linear_gelu",
            (mm.inputs[0], mm.inputs[1], bias),
            {"approximate": approximate},
            node.spec,
        )
        dropped.update((mm.name, producer.name))
    if not replaced:
        return _with_nodes(graph, list(graph.nodes), dict(graph.constants))
    nodes = [replaced.get(n.name, n) for n in graph.nodes if n.name not in dropped]
    used = {s for n in nodes for s in n.inputs}
    return _with_nodes(
        graph, nodes, {k: v for k, v in graph.constants.items() if k in used or k in graph.outputs}
    )


def fuse_shared_projections(graph: Graph) -> Graph:
    """Linears reading the same input with constant weights become one wide GEMM.

    Members are concatenated along N in graph order into a ``<leader>_shared``
    linear; each member becomes a ``narrow`` view of it (so the fused QKV
    projection is one kernel launch with N = 3 * d_model).
    """
    position = {n.name: i for i, n in enumerate(graph.nodes)}
    specs = graph.specs()
    groups: dict[tuple[str, int], list[Node]] = {}
    for node in graph.nodes:
        if node.op != "linear" or node.inputs[1] not in graph.constants:
            continue
        if len(node.inputs) == 3 and node.inputs[2] not in graph.constants:
            continue
        groups.setdefault((node.inputs[0], len(node.inputs)), []).append(node)
    groups = {k: v for k, v in groups.items() if len(v) >= 2}
    if not groups:
        return _with_nodes(graph, list(graph.nodes), dict(graph.constants))
    taken = set(graph.inputs) | set(graph.constants) | set(position)
    constants = dict(graph.constants)
    serial = 0

    def fresh(hint: str) -> str:
        nonlocal serial
        while True:
            serial += 1
            name = f"{hint}_{serial}"
            if name not in taken:
                taken.add(name)
                return name

    emitted_at: dict[str, list[Node]] = {}
    dropped: set[str] = set()
    for members in groups.values():
        members.sort(key=lambda n: position[n.name])
        leader = members[0]
        has_bias = len(leader.inputs) == 3
        if len({constants[m.inputs[1]].dtype for m in members}) != 1:
            continue
        if has_bias and len({constants[m.inputs[2]].dtype for m in members}) > 1:
            continue
        x_spec = specs[leader.inputs[0]]
        weight = fresh(f"{leader.name}_shared_weight")
        constants[weight] = torch.cat([constants[m.inputs[1]] for m in members], dim=1).contiguous()
        inputs = [leader.inputs[0], weight]
        if has_bias:
            bias = fresh(f"{leader.name}_shared_bias")
            constants[bias] = torch.cat([constants[m.inputs[2]] for m in members])
            inputs.append(bias)
        width = sum(m.spec.shape[1] for m in members)
        wide = fresh(f"{leader.name}_shared")
        out = [Node(wide, "linear", tuple(inputs), {}, TensorSpec((x_spec.shape[0], width), x_spec.dtype, x_spec.device))]
        offset = 0
        for m in members:
            out.append(Node(m.name, "narrow", (wide,), {"dim": 1, "start": offset, "length": m.spec.shape[1]}, m.spec))
            offset += m.spec.shape[1]
            dropped.add(m.name)
        emitted_at[leader.name] = out
    nodes: list[Node] = []
    for node in graph.nodes:
        if node.name in emitted_at:
            nodes.extend(emitted_at[node.name])
        elif node.name not in dropped:
            nodes.append(node)
    return _with_nodes(graph, nodes, constants)


def _greedy_order(graph: Graph, score) -> list[Node]:
    """Topological order picking, among ready nodes, the max of score()."""
    outputs = set(graph.outputs)
    position = {n.name: i for i, n in enumerate(graph.nodes)}
    by_name = {n.name: n for n in graph.nodes}
    users: dict[str, set[str]] = {}
    waiting: dict[str, set[str]] = {}
    for node in graph.nodes:
        for src in set(node.inputs):
            users.setdefault(src, set()).add(node.name)
        waiting[node.name] = {s for s in node.inputs if s in position}
    specs = graph.specs()
    pending_users = {k: len(v) for k, v in users.items() if k in position}

    def freed(node: Node) -> int:
        # Bytes whose last reader is this node (outputs are never freed).
        return sum(
            specs[s].nbytes
            for s in set(node.inputs)
            if s in position and s not in outputs and pending_users.get(s, 0) == 1
        )

    ready = [n for n in graph.nodes if not waiting[n.name]]
    order: list[Node] = []
    while ready:
        pick = max(ready, key=lambda n: score(n, position[n.name], freed(n)))
        ready.remove(pick)
        order.append(pick)
        for user in sorted(users.get(pick.name, ())):
            waiting[user].discard(pick.name)
            if not waiting[user]:
                ready.append(by_name[user])
        for s in set(pick.inputs):
            if s in pending_users:
                pending_users[s] -= 1
    if len(order) != len(graph.nodes):
        raise GraphError("graph contains a cycle")
    return order


_SCHEDULE_SCORES = (
    lambda node, pos, freed: (freed - node.spec.nbytes, -pos),
    lambda node, pos, freed: (freed - 2 * node.spec.nbytes, -pos),
    lambda node, pos, freed: (freed - node.spec.nbytes // 2, -pos),
    lambda node, pos, freed: (-node.spec.nbytes, freed, -pos),
    lambda node, pos, freed: (-pos,),
    lambda node, pos, freed: (pos,),
)


def schedule(graph: Graph) -> Graph:
    """Reorder nodes for the smallest planned arena (ties: lexicographic names)."""
    candidates: list[list[Node]] = []
    seen: set[tuple[str, ...]] = set()
    for score in _SCHEDULE_SCORES:
        order = _greedy_order(graph, score)
        names = tuple(n.name for n in order)
        if names not in seen:
            seen.add(names)
            candidates.append(order)

    def cost(order: list[Node]):
        planned = plan_memory(_with_nodes(graph, order, dict(graph.constants))).planned_bytes
        return planned, tuple(n.name for n in order)

    return _with_nodes(graph, min(candidates, key=cost), dict(graph.constants))


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
    graph.validate()
    work = graph.clone()
    records: list[PassRecord] = []
    for name, fn in PIPELINE:
        before = len(work.nodes)
        work = fn(work)
        work.validate()
        records.append(PassRecord(name, before, len(work.nodes)))
    return work, records
