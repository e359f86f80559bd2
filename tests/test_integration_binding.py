"""The ctypes binding a ForgeML maintainer would add (the `src/forgeml/_hip.py`
block of INTEGRATION.md), executed against this build's library on the CPU:
it loads, its argtypes match the exported symbols, and the reference's
KernelConfig values map to library config ids (no kernel is launched).
"""

import re
from dataclasses import dataclass
from pathlib import Path

import pytest
import torch

from forgeml_amd import _native, kernels
from forgeml_amd.ir import GraphError

DOC = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


@dataclass(frozen=True)
class RefKernelConfig:
    """The reference's KernelConfig fields and defaults (src/forgeml/kernels.py:12-18)."""

    block_m: int = 32
    block_n: int = 64
    block_k: int = 32
    num_warps: int = 4
    num_stages: int = 2


@pytest.fixture(scope="module")
def binding():
    _native.load()
    blocks = re.findall(r"```python\n(# src/forgeml/_hip\.py\n.*?)```", DOC.read_text(), flags=re.S)
    assert len(blocks) == 1, "INTEGRATION.md must hold one src/forgeml/_hip.py block"
    source = blocks[0].replace('ctypes.CDLL("libforgeml_hip.so")', f'ctypes.CDLL("{_native.LIBRARY_PATH}")')
    source = source.replace("from forgeml.ir import GraphError", "from forgeml_amd.ir import GraphError")
    namespace: dict = {}
    exec(compile(source, "INTEGRATION.md:_hip.py", "exec"), namespace)
    return namespace


def test_reference_configs_map_to_library_ids(binding):
    config_id = binding["_config_id"]
    # The reference's 64x64 tile with 4 warps is built for both dtype classes.
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        cid = config_id(RefKernelConfig(64, 64, 32, 4, 3), dtype)
        assert cid == kernels.config_id(kernels.KernelConfig(64, 64, 32 if dtype == torch.float32 else 64, 4, 4),
                                        dtype)
    # DEFAULT_CONFIG and tiles with no built counterpart take the shape heuristic.
    for cfg in (RefKernelConfig(), RefKernelConfig(16, 32, 32, 4, 2), RefKernelConfig(32, 128, 32, 8, 3)):
        assert config_id(cfg, torch.float32) == binding["CONFIG_AUTO"]


def test_plan_errors_are_raised(binding):
    # A negative stride: forgeml_hip_gemm_plan refuses it, and the binding raises.
    lib = binding["_lib"]
    plan = (binding["_I64"] * 4)()
    rc = lib.forgeml_hip_gemm_plan(256, 8, 1, 256, -1, 1, 8, 8, 8, 0, -1, plan)
    assert rc == binding["EINVAL"]
    with pytest.raises(GraphError, match="forgeml_hip_gemm_plan failed"):
        binding["_check"](rc, "forgeml_hip_gemm_plan")
    with pytest.raises(RuntimeError, match="forgeml_hip_gemm failed"):
        binding["_check"](-3, "forgeml_hip_gemm")
