"""forgeml_amd — ForgeML's compiled-linear path, native to AMD Instinct MI355X.

The host side (IR, passes, memory planner, executor, autotuner) keeps
ForgeML's API; the fused GEMM + bias + GELU/ReLU kernels are hand-written
for gfx950 (CDNA4 MFMA) and called through a C ABI (include/forgeml_hip.h).
"""

from forgeml_amd.analysis import graph_analysis
from forgeml_amd.compiler import CompiledModel, GraphedModel, compile
from forgeml_amd.frontend import from_torch
from forgeml_amd.ir import Graph, GraphBuilder, GraphError, TensorSpec
from forgeml_amd.neural import TransformerBlock

__all__ = [
    "CompiledModel",
    "Graph",
    "GraphBuilder",
    "GraphedModel",
    "GraphError",
    "TensorSpec",
    "TransformerBlock",
    "compile",
    "from_torch",
    "graph_analysis",
]
