"""``compile()`` and the slot-arena executor ``CompiledModel``.

Behaviour follows ForgeML's executor (src/forgeml/compiler.py:19-264):

* the slot arena is allocated once per compiled model and reused on every
  call, so a call is not reentrant (compiler.py:37-42);
* each node gets a closure chosen at build time (compiler.py:66-127):
  internal GEMM nodes planned for ``"hip"`` write straight into their slot
  view, output nodes get a fresh tensor, view ops borrow their source;
* reassigning ``kernel_plan`` rebuilds the closures (compiler.py:55-64);
* the GPU kernel is looked up as ``kernels.matmul`` at call time, so a test
  can replace it on the module (compiler.py:186-206);
* there is no silent fallback: a failing kernel launch raises.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field

import torch
import torch.nn.functional as F

from forgeml_amd import kernels
from forgeml_amd.analysis import graph_analysis
from forgeml_amd.frontend import from_torch
from forgeml_amd.ir import Graph, GraphError
from forgeml_amd.kernels import DEFAULT_CONFIG, KernelConfig
from forgeml_amd.memory import OUT_CAPABLE_OPS, VIEW_LIKE_OPS, MemoryPlan, plan_memory
from forgeml_amd.ops import evaluate
from forgeml_amd.passes import PassRecord
from forgeml_amd.passes import optimize as optimize_graph

BACKENDS = ("torch", "hip", "auto")


def _slot_writer(node, view: torch.Tensor):
    """Torch-backend closure that writes node's result into its slot view."""
    op = node.op
    if op == "matmul":
        return lambda args: torch.matmul(args[0], args[1], out=view)
    if op == "linear":
        if len(node.inputs) == 3:
            return lambda args: torch.addmm(args[2], args[0], args[1], out=view)
        return lambda args: torch.mm(args[0], args[1], out=view)
    if op == "add":
        return lambda args: torch.add(args[0], args[1], out=view)
    if op == "mul":
        return lambda args: torch.mul(args[0], args[1], out=view)
    if op == "relu":
        return lambda args: torch.clamp_min(args[0], 0, out=view)
    if op == "softmax":
        dim = node.attrs["dim"]
        return lambda args: torch.softmax(args[0], dim=dim, out=view)
    if op == "gelu":
        approx = node.attrs.get("approximate", "none")
        return lambda args: F.gelu(args[0], approximate=approx, out=view)
    if op == "embedding":
        return lambda args: torch.ops.aten.embedding.out(args[1], args[0], -1, False, False, out=view)
    if op == "fused_linear_gelu":
        approx = node.attrs.get("approximate", "none")

        def run_fused(args):
            # The reference's CPU path: GEMM into the slot, then GELU in place.
            if len(args) == 3:
                torch.addmm(args[2], args[0], args[1], out=view)
            else:
                torch.mm(args[0], args[1], out=view)
            torch.ops.aten.gelu_.default(view, approximate=approx)
            return view

        return run_fused
    raise GraphError(f"no slot writer for op {op!r}")


@dataclass
class CompiledModel:
    graph: Graph
    original_graph: Graph
    memory_plan: MemoryPlan
    passes: list[PassRecord]
    backend: str
    kernel_plan: dict[str, str] = field(default_factory=dict)
    kernel_configs: dict[str, KernelConfig] = field(default_factory=dict)

    def __post_init__(self) -> None:
        uses: dict[str, int] = {}
        for node in self.graph.nodes:
            for src in node.inputs:
                uses[src] = uses.get(src, 0) + 1
        self._uses_template = uses
        self._outputs = frozenset(self.graph.outputs)
        self._produced = {node.name for node in self.graph.nodes}
        # One arena per compiled model, reused by every call (not reentrant).
        self._slots: dict[int, torch.Tensor] = {
            slot: torch.empty(spec.shape, dtype=spec.dtype, device=spec.device)
            for slot, spec in self.memory_plan.slot_specs.items()
        }
        self._views: dict[str, torch.Tensor] = {}
        for node in self.graph.nodes:
            alloc = self.memory_plan.allocations.get(node.name)
            if alloc is not None:
                n = alloc.size_bytes // node.spec.dtype.itemsize
                self._views[node.name] = self._slots[alloc.slot][:n].view(node.spec.shape)
        self._kernel_layout_constants()
        self._build_steps()

    def _build_steps(self) -> None:
        """Closures per node, with hip GEMMs fused with the residual add after them."""
        object.__setattr__(self, "fused_residuals", self._plan_residual_fusions())
        fused_adds = {add: carried for add, _view, _r, carried in self.fused_residuals.values()}
        steps = []
        for node in self.graph.nodes:
            inputs = tuple(node.inputs)
            if node.name in self.fused_residuals:
                add_name, _view, residual, _carried = self.fused_residuals[node.name]
                run = self._make_fused_residual_step(node, add_name)
                inputs = inputs + (residual,)
            elif node.name in fused_adds:
                # The add was done in the GEMM's epilogue: pass its result on.
                pos = node.inputs.index(fused_adds[node.name])
                run = (lambda p: (lambda args: args[p]))(pos)
            else:
                run = self._make_step(node)
            steps.append((node, run, inputs))
        object.__setattr__(self, "_steps", steps)

    def _plan_residual_fusions(self) -> dict[str, tuple[str, str | None, str, str]]:
        """GEMM nodes whose result only feeds an ``add`` (optionally through one
        reshape) immediately after them in the schedule.

        The reference runs the GEMM, then the add as a second kernel
        (src/forgeml/compiler.py:93-98); here the GEMM's epilogue adds the other
        operand and writes the add's destination directly, and the add node
        passes that result on.  Conditions: the GEMM is hip-planned and not a
        graph output; the chain is adjacent in the schedule, so nothing runs in
        between; shapes match without broadcasting; and the add's slot (if it
        has one) holds none of the GEMM's inputs or the other operand, so the
        early write clobbers nothing.  Returns gemm -> (add, reshape or None,
        residual, the add's input that carries the GEMM result).
        """
        nodes = self.graph.nodes
        index = {n.name: i for i, n in enumerate(nodes)}
        producer = {n.name: n for n in nodes}
        consumers: dict[str, list] = {}
        for n in nodes:
            for src in n.inputs:
                consumers.setdefault(src, []).append(n)
        specs = self.graph.specs()

        def root_slot(name: str):
            while name in producer and producer[name].op in VIEW_LIKE_OPS:
                name = producer[name].inputs[0]
            alloc = self.memory_plan.allocations.get(name)
            return None if alloc is None else alloc.slot

        fusions = {}
        for i, node in enumerate(nodes):
            if node.op not in kernels.GEMM_OPS or self.kernel_plan.get(node.name) != "hip":
                continue
            if node.name in self._outputs or len(consumers.get(node.name, [])) != 1:
                continue
            view, nxt, carried = None, consumers[node.name][0], node.name
            if nxt.op == "reshape":
                if index[nxt.name] != i + 1 or nxt.name in self._outputs or len(consumers.get(nxt.name, [])) != 1:
                    continue
                view, carried, nxt = nxt, nxt.name, consumers[nxt.name][0]
            if nxt.op != "add" or index[nxt.name] != i + (2 if view else 1) or len(nxt.inputs) != 2:
                continue
            others = [x for x in nxt.inputs if x != carried]
            if len(others) != 1:
                continue
            residual = others[0]
            dtype = node.spec.dtype
            if (
                tuple(specs[residual].shape) != tuple(nxt.spec.shape)
                or tuple(specs[carried].shape) != tuple(nxt.spec.shape)
                or specs[residual].dtype != dtype
                or nxt.spec.dtype != dtype
            ):
                continue
            dest = root_slot(nxt.name) if nxt.name not in self._outputs else None
            if dest is not None and any(root_slot(x) == dest for x in (*node.inputs, residual)):
                continue
            fusions[node.name] = (nxt.name, None if view is None else view.name, residual, carried)
        return fusions

    def _make_fused_residual_step(self, node, add_name: str):
        add_node = next(n for n in self.graph.nodes if n.name == add_name)
        to_output = add_name in self._outputs
        slot_view = None if to_output else self._views[add_name]
        m, n = node.spec.shape
        spec = add_node.spec

        def run(args):
            *gemm_args, residual = args
            if to_output:
                dest = torch.empty(spec.shape, dtype=spec.dtype, device=gemm_args[0].device)
            else:
                dest = slot_view
            return self._run_hip(node, tuple(gemm_args), dest.view(m, n), residual=residual.reshape(m, n))

        return run

    def _kernel_layout_constants(self) -> None:
        """Store GEMM weights of hip-planned nodes K-contiguous.

        A ``[K, N]`` weight constant becomes the same logical tensor with
        strides ``(1, K)`` (the ``nn.Linear`` layout), which the gfx950 kernels
        stream by DMA straight into LDS; the row-major copy would need the
        transposing register loader.  Values, shape, dtype and device are
        unchanged, so torch ops on the constant are unaffected.
        """
        consts = self.graph.constants
        for node in self.graph.nodes:
            if self.kernel_plan.get(node.name) != "hip" or node.op not in kernels.GEMM_OPS:
                continue
            name = node.inputs[1]
            w = consts.get(name)
            if w is None or w.dim() != 2 or not w.is_contiguous() or w.shape[0] == 1 or w.shape[1] == 1:
                continue
            consts[name] = w.t().contiguous().t()

    def __setattr__(self, name, value):
        object.__setattr__(self, name, value)
        # A new kernel plan changes dispatch, so rebuild the step closures.
        if name == "kernel_plan" and "_views" in self.__dict__:
            self._kernel_layout_constants()
            self._build_steps()

    def _make_step(self, node):
        on_hip = self.kernel_plan.get(node.name) == "hip"
        is_output = node.name in self._outputs
        if node.op in VIEW_LIKE_OPS:
            if on_hip:
                raise GraphError(f"no hip kernel for op {node.op!r}")
            if is_output:
                return lambda args: self._evaluate(node, args).clone()
            return lambda args: self._evaluate(node, args)
        if on_hip and node.op == "layer_norm":
            attrs = node.attrs
            return lambda args: kernels.layer_norm(
                args[0], attrs["normalized_shape"], *(args[1:] if len(args) == 3 else (None, None)), eps=attrs["eps"]
            )
        if on_hip and node.op == "sdpa":
            causal, scale = node.attrs["is_causal"], node.attrs.get("scale")
            return lambda args: kernels.attention(args[0], args[1], args[2], is_causal=causal, scale=scale)
        if on_hip:
            view = None if is_output else self._views.get(node.name)
            return lambda args: self._run_hip(node, args, view)
        if is_output or node.op not in OUT_CAPABLE_OPS:
            # Outputs own fresh storage; ops without out= are refcounted.
            return lambda args: self._evaluate(node, args)
        return _slot_writer(node, self._views[node.name])

    def autotune(self, *inputs: torch.Tensor, warmup: int = 3, repeats: int = 10) -> dict:
        from forgeml_amd.autotune import tune_graph

        return tune_graph(self, inputs, warmup=warmup, repeats=repeats)

    def kernel_source(self) -> str:
        return kernels.kernel_source()

    def _check_inputs(self, inputs) -> dict[str, torch.Tensor]:
        names = list(self.graph.inputs)
        if len(inputs) != len(names):
            raise GraphError(f"expected {len(names)} inputs, got {len(inputs)}")
        values: dict[str, torch.Tensor] = {}
        for name, t in zip(names, inputs):
            if not isinstance(t, torch.Tensor):
                raise GraphError("inputs must be torch.Tensor")
            spec = self.graph.inputs[name]
            if tuple(t.shape) != spec.shape:
                raise GraphError(f"input {name!r} shape {tuple(t.shape)} != expected {spec.shape}")
            if t.dtype != spec.dtype:
                raise GraphError(f"input {name!r} dtype {t.dtype} != expected {spec.dtype}")
            if str(t.device) != spec.device:
                raise GraphError(f"input {name!r} device {t.device} != expected {spec.device}")
            values[name] = t
        return values

    def __call__(self, *inputs: torch.Tensor):
        values = self._check_inputs(inputs)
        values.update(self.graph.constants)
        outputs = self._outputs
        remaining = dict(self._uses_template)
        with torch.inference_mode():
            for node, run, inputs in self._steps:
                values[node.name] = run(tuple(values[i] for i in inputs))
                for src in node.inputs:
                    if src in remaining:
                        remaining[src] -= 1
                        if remaining[src] == 0 and src not in outputs:
                            values.pop(src, None)
            result = []
            for name in self.graph.outputs:
                if name not in values:
                    raise GraphError(f"output {name!r} was not produced")
                # Outputs naming an input or constant are cloned (no aliasing).
                result.append(values[name] if name in self._produced else values[name].clone())
        return tuple(result) if self.graph.output_is_tuple else result[0]

    @staticmethod
    def _evaluate(node, args: tuple[torch.Tensor, ...]) -> torch.Tensor:
        try:
            return evaluate(node.op, args, node.attrs)
        except GraphError:
            raise
        except Exception as e:  # noqa: BLE001
            raise GraphError(f"node {node.name!r} ({node.op}) execution failed: {e}") from e

    def _run_hip(self, node, args: tuple[torch.Tensor, ...], out: torch.Tensor | None,
                 residual: torch.Tensor | None = None) -> torch.Tensor:
        config = self.kernel_configs.get(node.name, DEFAULT_CONFIG)
        bias = args[2] if len(args) == 3 else None
        # The residual keyword is passed only when fused, so a replacement
        # kernels.matmul with the reference's signature keeps working otherwise.
        extra = {} if residual is None else {"residual": residual}
        if node.op == "matmul":
            return kernels.matmul(args[0], args[1], config=config, out=out, **extra)
        if node.op == "linear":
            return kernels.matmul(args[0], args[1], bias, config=config, out=out, **extra)
        if node.op == "fused_linear_gelu":
            return kernels.matmul(
                args[0], args[1], bias, activation="gelu",
                approximate=node.attrs.get("approximate", "none"), config=config, out=out, **extra,
            )
        raise GraphError(f"no hip kernel for op {node.op!r}")

    def capture_graph(self, *example_inputs: torch.Tensor, warmup: int = 2) -> "GraphedModel":
        """Capture one call into a HIP graph for these input shapes (see GraphedModel)."""
        return GraphedModel(self, example_inputs, warmup=warmup)

    def explain(self) -> dict:
        analysis = graph_analysis(self.graph)
        original = graph_analysis(self.original_graph)
        return {
            "backend": self.backend,
            "original_nodes": len(self.original_graph.nodes),
            "optimized_nodes": len(self.graph.nodes),
            "passes": [
                {"name": p.name, "nodes_before": p.nodes_before, "nodes_after": p.nodes_after} for p in self.passes
            ],
            "memory_plan": self.memory_plan.to_dict(),
            "graph": self.graph.to_dict(),
            "kernel_plan": dict(self.kernel_plan),
            "kernel_configs": {k: asdict(v) for k, v in self.kernel_configs.items()},
            "analysis": analysis,
            "original_analysis": original,
            "optimization_delta": {
                "nodes": len(self.original_graph.nodes) - len(self.graph.nodes),
                "flops": original["flops"] - analysis["flops"],
                "logical_bytes": original["logical_bytes"] - analysis["logical_bytes"],
                "critical_path_ops": original["critical_path_ops"] - analysis["critical_path_ops"],
                "planned_bytes": self.memory_plan.naive_bytes - self.memory_plan.planned_bytes,
            },
        }


class GraphedModel:
    """A CompiledModel call captured once into a HIP graph and replayed.

    The per-node host work of ``CompiledModel.__call__`` (closures, kernel
    argument validation, launches; src/forgeml/compiler.py:158-164) is paid
    once at capture; a call then copies the inputs into the graph's static
    input buffers and replays every kernel of the model as one graph launch.
    The slot arena, the weights and the graph's own memory pool stay
    resident.  Outputs are the graph's static output tensors: the next call
    overwrites them, so clone what must be kept.  Like the compiled model, a
    graphed model is not reentrant.

    Shapes, dtypes and devices are fixed by the example inputs.  Capture runs
    ``warmup`` eager calls first, on a side stream, so the kernels' one-time
    set-up (library load, LDS limits) happens outside the graph.
    """

    def __init__(self, compiled: CompiledModel, example_inputs, *, warmup: int = 2):
        inputs = compiled._check_inputs(tuple(example_inputs))
        devices = {t.device for t in inputs.values()}
        if len(devices) != 1 or next(iter(devices)).type != "cuda":
            raise GraphError("graph capture needs every input on one GPU")
        self.compiled = compiled
        self.device = next(iter(devices))
        self._static_inputs = [t.clone() for t in inputs.values()]
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                compiled(*self._static_inputs)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.device(self.device), torch.cuda.graph(self.graph):
            self._static_output = compiled(*self._static_inputs)
        torch.cuda.synchronize(self.device)

    def __call__(self, *inputs: torch.Tensor):
        values = self.compiled._check_inputs(inputs)
        for dst, src in zip(self._static_inputs, values.values()):
            if src.data_ptr() != dst.data_ptr():
                dst.copy_(src)
        self.graph.replay()
        return self._static_output

    @property
    def static_inputs(self) -> list[torch.Tensor]:
        """The graph's input buffers: writing them directly skips the copy."""
        return self._static_inputs


def compile(
    model: torch.nn.Module | Graph,
    example_inputs: tuple[torch.Tensor, ...] = (),
    *,
    backend: str = "torch",
    optimize: bool = True,
) -> CompiledModel:
    """Lower, optimise, plan and bind a model (src/forgeml/compiler.py:240-264)."""
    if backend not in BACKENDS:
        raise GraphError(f"unsupported backend {backend!r}; expected 'torch', 'hip', or 'auto'")
    if isinstance(model, Graph):
        model.validate()
        graph = model.clone()
    elif isinstance(model, torch.nn.Module):
        graph = from_torch(model, example_inputs)
    else:
        raise GraphError("compile expects an nn.Module or a Graph")
    original = graph.clone()
    if optimize:
        graph, records = optimize_graph(graph)
    else:
        graph.validate()
        records = []
    plan = plan_memory(graph)
    kernel_plan = kernels.select_kernels(graph, backend)
    return CompiledModel(graph, original, plan, records, backend, kernel_plan=kernel_plan)
