"""Extract the structural goldens held in ForgeML's published captures.

Reads the reference's own result files (benchmarks/results/compiler-cpu.json
and neural-cpu.json) and keeps, per workload and variant, the data that a
compile of the same model must reproduce: the optimized/unoptimized graph,
memory plan, pass records, kernel plan and static analysis.  Timings and
environment fields are dropped.  Run once in a container that has the
reference checkout; the output is committed as forgeml_captures.json.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

REFERENCE = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent / "forgeml_captures.json"

KEEP = ("graph", "memory_plan", "passes", "kernel_plan", "optimized_nodes", "original_nodes", "optimization_delta")
ANALYSIS = ("flops", "logical_bytes", "critical_path_ops", "op_counts", "nodes", "input_bytes",
            "constant_bytes", "output_bytes", "per_node")


def _variant(v: dict) -> dict:
    out = {k: v[k] for k in KEEP}
    out["analysis"] = {k: v["analysis"][k] for k in ANALYSIS}
    out["original_analysis"] = {k: v["original_analysis"][k] for k in ANALYSIS}
    return out


def main() -> None:
    goldens = {"source": "benchmarks/results/compiler-cpu.json, benchmarks/results/neural-cpu.json", "workloads": []}
    compiler = json.loads((REFERENCE / "benchmarks/results/compiler-cpu.json").read_text())
    for w in compiler["workloads"]:
        goldens["workloads"].append({
            "suite": "mlp",
            "name": w["name"],
            "batch": w["batch"], "width": w["width"], "hidden": w["hidden"], "output": w["output"],
            "residual": w["name"].startswith("residual"),
            "unoptimized": _variant(w["unoptimized"]),
            "optimized": _variant(w["optimized"]),
        })
    neural = json.loads((REFERENCE / "benchmarks/results/neural-cpu.json").read_text())
    for w in neural["workloads"]:
        if not w["name"].startswith("transformer_block"):
            continue  # the vision-text workload is outside the linear path
        goldens["workloads"].append({
            "suite": "transformer_block",
            "name": w["name"],
            "input_shape": w["unoptimized"]["graph"]["inputs"]["input_0"]["shape"],
            "unoptimized": _variant(w["unoptimized"]),
            "optimized": _variant(w["optimized"]),
        })
    OUT.write_text(json.dumps(goldens, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(goldens['workloads'])} workloads)")


if __name__ == "__main__":
    main()
