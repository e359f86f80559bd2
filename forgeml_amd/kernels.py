"""Kernel boundary: the fused GEMM + bias + activation entry point.

``matmul`` is the drop-in for ForgeML's ``kernels.matmul``
(src/forgeml/kernels.py:52-116): same signature, same validation order and
``GraphError`` messages, same ownership rules (the caller owns every buffer;
``out`` may be a planner slot view; ``out`` must not share storage with an
input).  Where the reference launches its Triton kernel
(src/forgeml/kernels.py:206-209 -> src/forgeml/_triton.py:65-93) this calls
the hand-written gfx950 kernels through the C ABI on the current HIP stream.

Tile configurations are compiled ahead of time, so ``KernelConfig`` names an
entry of the library's MI355X tile table instead of Triton meta-parameters
(src/forgeml/kernels.py:12-32).  ``DEFAULT_CONFIG`` selects a tile by shape.
"""

from __future__ import annotations

import ctypes
import importlib.resources
from dataclasses import dataclass

import torch

from forgeml_amd import _native
from forgeml_amd.ir import Graph, GraphError


@dataclass(frozen=True)
class KernelConfig:
    """One MI355X tile configuration, or all-None for the shape heuristic.

    block_m x block_n is the output tile of one workgroup, block_k the K
    elements staged per LDS buffer (128 bytes: 32 fp32 or 64 bf16/fp16),
    num_waves the 64-lane wavefronts per workgroup and num_stages the LDS
    buffers in the software pipeline.
    """

    block_m: int | None = None
    block_n: int | None = None
    block_k: int | None = None
    num_waves: int | None = None
    num_stages: int | None = None

    @property
    def is_auto(self) -> bool:
        return (self.block_m is None and self.block_n is None and self.block_k is None and self.num_waves is None
                and self.num_stages is None)


DEFAULT_CONFIG = KernelConfig()

# The library's tile table, in config-id order (forgeml_amd/csrc/tile_table.hpp).
# A CPU test checks it against forgeml_hip_config_info.
# (block_m, block_n, waves, LDS stages); the 64x64 tiles keep up to four stages
# in flight when both operands are K-contiguous (two on grids of more than two
# workgroups per CU, where more resident workgroups hide latency better).
_FP32_TILES = ((128, 128, 4, 2), (64, 64, 4, 4), (256, 256, 8, 2))
_H16_TILES = ((256, 256, 4, 2), (128, 128, 4, 2), (64, 64, 4, 4), (256, 256, 8, 2))
# The few-row kernels come last: up to 64 rows, 16 columns per workgroup, 8
# waves splitting K in chunks of 16 fp32 / 32 16-bit elements, up to 4 chunks
# in flight per wave.  They run only K-contiguous A and B.
SKINNY_FP32 = KernelConfig(64, 16, 16, 8, 4)
SKINNY_H16 = KernelConfig(64, 16, 32, 8, 4)
CANDIDATES: tuple[KernelConfig, ...] = tuple(
    [KernelConfig(bm, bn, 32, w, st) for bm, bn, w, st in _FP32_TILES]
    + [KernelConfig(bm, bn, 64, w, st) for bm, bn, w, st in _H16_TILES]
    + [SKINNY_FP32, SKINNY_H16]
)
# dtype class of each candidate: 0 = fp32, 1 = bf16/fp16.
_CANDIDATE_CLASS = tuple([0] * len(_FP32_TILES) + [1] * len(_H16_TILES) + [0, 1])
_CONFIG_IDS = {cfg: i for i, cfg in enumerate(CANDIDATES)}

_DTYPES = {torch.float16, torch.bfloat16, torch.float32}
_DTYPE_CODES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16, torch.float16: _native.DTYPE_F16}
_ACTIVATIONS = ("none", "gelu", "relu")
GEMM_OPS = ("matmul", "linear", "fused_linear_gelu")
TARGET_ARCH = "gfx950"


def candidates(dtype: torch.dtype) -> tuple[KernelConfig, ...]:
    """Tile configurations built for ``dtype`` (the autotuner's search space)."""
    dclass = 0 if dtype == torch.float32 else 1
    return tuple(c for c, k in zip(CANDIDATES, _CANDIDATE_CLASS) if k == dclass)


_ARCH_BY_INDEX: dict[int, str] = {}
_CUDA_SEEN = False  # torch.cuda.is_available() has returned True in this process


def _cuda_ready() -> bool:
    """torch.cuda.is_available(), asked until it first returns True (it reads the environment each call)."""
    global _CUDA_SEEN
    if not _CUDA_SEEN:
        _CUDA_SEEN = torch.cuda.is_available()
    return _CUDA_SEEN


def _arch_of_index(index: int) -> str:
    arch = _ARCH_BY_INDEX.get(index)
    if arch is None:
        props = torch.cuda.get_device_properties(index)
        arch = _ARCH_BY_INDEX[index] = str(getattr(props, "gcnArchName", "")).split(":")[0]
    return arch


def _device_arch(device: torch.device) -> str:
    """gfx name of a GPU (e.g. "gfx950"), looked up once per device index."""
    return _arch_of_index(device.index if device.index is not None else torch.cuda.current_device())


# hipStream_t of torch's current stream on a GPU: torch's raw-stream query
# where the build has it (one call, no Stream object), else the public API.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(index: int) -> int:
    if _RAW_STREAM is not None:
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(index).cuda_stream


def _gpu_ok(device: torch.device | None = None) -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        return _device_arch(device or torch.device("cuda", torch.cuda.current_device())) == TARGET_ARCH
    except (RuntimeError, AssertionError):
        return False


def available() -> bool:
    """True when a gfx950 GPU is visible and the kernel library loads."""
    if not _gpu_ok():
        return False
    try:
        _native.load()
    except _native.NativeLibraryError:
        return False
    return True


def _check_config(config: KernelConfig, dtype: torch.dtype) -> int:
    if not isinstance(config, KernelConfig):
        raise GraphError(f"config must be a KernelConfig, got {type(config).__name__}")
    if config.is_auto:
        return _native.CONFIG_AUTO
    cid = _CONFIG_IDS.get(config)
    if cid is None or _CANDIDATE_CLASS[cid] != (0 if dtype == torch.float32 else 1):
        built = candidates(dtype)
        raise GraphError(f"config {config} is not a built MI355X tile for {dtype}; choose one of {list(built)}")
    return cid


def config_id(config: KernelConfig, dtype: torch.dtype) -> int:
    """Library config id of ``config`` for ``dtype`` (-1 = shape heuristic)."""
    return _check_config(config, dtype)


def resolve_config(m: int, n: int, k: int, dtype: torch.dtype, config: KernelConfig = DEFAULT_CONFIG) -> KernelConfig:
    """The concrete tile ``config`` runs with for an (m, n, k) GEMM."""
    cid = _check_config(config, dtype)
    if cid == _native.CONFIG_AUTO:
        cid = _native.load().forgeml_hip_select_config(m, n, k, _DTYPE_CODES[dtype])
        if cid < 0:
            raise GraphError(f"select_config failed: {_native.last_error()}")
    return CANDIDATES[cid]


def _act_code(activation: str, approximate: str) -> int:
    if activation == "gelu":
        return _native.ACT_GELU_ERF if approximate == "none" else _native.ACT_GELU_TANH
    if activation == "relu":
        return _native.ACT_RELU
    return _native.ACT_NONE


def launch(
    a: torch.Tensor,
    b: torch.Tensor,
    bias: torch.Tensor | None,
    out: torch.Tensor,
    *,
    act: int,
    config_id: int,
    workspace: torch.Tensor | None = None,
    stream: int | None = None,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Unchecked launch of the fused kernel (arguments already validated)."""
    lib = _native.load()
    m, k = a.shape
    n = b.shape[1]
    dtype = _DTYPE_CODES[a.dtype]
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    if stream is None:
        stream = _stream_handle(a.get_device())
    bias_ptr, sbi = (None, 0) if bias is None else (bias.data_ptr(), bias.stride(0))
    if residual is None:
        rc = lib.forgeml_hip_gemm(
            a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0), b.stride(1), bias_ptr, sbi,
            out.data_ptr(), m, n, k, dtype, act, config_id, ws_ptr, ws_bytes, ctypes.c_void_p(stream),
        )
    else:
        rc = lib.forgeml_hip_gemm_add(
            a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0), b.stride(1), bias_ptr, sbi,
            residual.data_ptr(), residual.stride(0), residual.stride(1),
            out.data_ptr(), m, n, k, dtype, act, config_id, ws_ptr, ws_bytes, ctypes.c_void_p(stream),
        )
    if rc != _native.OK:
        msg = f"forgeml_hip_gemm failed ({rc}): {_native.last_error()}"
        raise GraphError(msg) if rc in (_native.EINVAL, _native.ECONFIG) else RuntimeError(msg)
    return out


def workspace_for(m: int, n: int, k: int, dtype: torch.dtype, cid: int, device: torch.device) -> torch.Tensor | None:
    """A workspace large enough for any operand layout of this shape (None if none splits K)."""
    nbytes = _native.load().forgeml_hip_gemm_workspace_size(m, n, k, _DTYPE_CODES[dtype], cid)
    if nbytes < 0:
        raise GraphError(f"workspace_size failed: {_native.last_error()}")
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


KIND_NAMES = ("tiled", "few-row")


# forgeml_hip_gemm_plan results by operand geometry: what a plan depends on
# (shapes, element strides, dtype, config and the operands' 16-byte
# alignment), so repeated calls, such as a compiled model's, skip the C call.
_PLAN_CACHE: dict[tuple, tuple[int, int, int, int]] = {}
_PLAN_CACHE_MAX = 4096


def _plan_ids(a: torch.Tensor, b: torch.Tensor, cid: int) -> tuple[int, int, int, int]:
    """(config id, K slices, workspace bytes, kernel kind) of a GEMM, refused as GraphError."""
    m, k = a.shape
    n = b.shape[1]
    a_ptr, b_ptr = a.data_ptr(), b.data_ptr()
    sa, sb = a.stride(), b.stride()
    key = (m, n, k, sa, sb, a_ptr & 15, b_ptr & 15, a.dtype, cid)
    ids = _PLAN_CACHE.get(key)
    if ids is None:
        out = (ctypes.c_int64 * 4)()
        rc = _native.load().forgeml_hip_gemm_plan(
            a_ptr, sa[0], sa[1], b_ptr, sb[0], sb[1], m, n, k, _DTYPE_CODES[a.dtype], cid, out,
        )
        if rc != _native.OK:
            raise GraphError(f"forgeml_hip_gemm_plan failed ({rc}): {_native.last_error()}")
        ids = (int(out[0]), int(out[1]), int(out[2]), int(out[3]))
        if len(_PLAN_CACHE) >= _PLAN_CACHE_MAX:
            _PLAN_CACHE.clear()
        _PLAN_CACHE[key] = ids
    return ids


def plan(a: torch.Tensor, b: torch.Tensor, config: KernelConfig = DEFAULT_CONFIG) -> dict:
    """What ``matmul(a, b, config=config)`` runs: config, K slices, workspace bytes, kernel kind."""
    cid, splits, ws_bytes, kind = _plan_ids(a, b, _check_config(config, a.dtype))
    return {
        "config": CANDIDATES[cid],
        "config_id": cid,
        "k_splits": splits,
        "workspace_bytes": ws_bytes,
        "kernel": KIND_NAMES[kind],
    }


def matmul(
    a: torch.Tensor,
    b: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    activation: str = "none",
    approximate: str = "none",
    config: KernelConfig = DEFAULT_CONFIG,
    out: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """out = act(rnd(rnd(a @ b) + bias)) on the gfx950 kernels.

    ``activation`` is "none", "gelu" (``approximate`` "none" = erf, "tanh")
    or "relu" (clamp_min(x, 0), the executor's relu slot writer fused into
    the epilogue).  ``residual`` (keyword only, not in the reference's
    signature) adds an [M, N] tensor to the rounded activation in the same
    epilogue, as the reference's following ``add`` node would; it may be
    ``out`` itself.  ``workspace`` (keyword only, not in the reference's
    signature): a uint8 GPU buffer for split-K partial sums, at least
    ``plan(a, b, config)["workspace_bytes"]`` (or ``workspace_for``) bytes and
    16-byte aligned; when given, no per-call plan is made and the library
    refuses one that is too small.  Without it the call plans and allocates
    what the split needs.  Launches on ``torch.cuda.current_stream()`` of
    ``a``'s device and returns ``out`` (allocated when None).
    """
    if not _cuda_ready():
        raise GraphError("hip matmul requires a ROCm GPU visible to torch (torch.cuda)")
    _native.load()
    if not isinstance(a, torch.Tensor) or not isinstance(b, torch.Tensor):
        raise GraphError("matmul inputs must be tensors")
    # Devices compared by index (get_device() builds no torch.device object).
    if not a.is_cuda or not b.is_cuda or a.get_device() != b.get_device():
        raise GraphError("matmul inputs must be GPU tensors on the same device")
    dev = a.get_device()
    if a.dtype not in _DTYPES or a.dtype != b.dtype:
        raise GraphError(f"matmul dtype {a.dtype} not supported or mismatched")
    if a.dim() != 2 or b.dim() != 2:
        raise GraphError("matmul requires rank-2 inputs")
    m, k = a.shape
    k2, n = b.shape
    if k != k2 or m <= 0 or n <= 0 or k <= 0:
        raise GraphError(f"matmul incompatible shapes {a.shape} x {b.shape}")
    if activation not in _ACTIVATIONS:
        raise GraphError(f"activation must be one of {_ACTIVATIONS}, got {activation!r}")
    if approximate not in ("none", "tanh"):
        raise GraphError(f"approximate must be 'none' or 'tanh', got {approximate!r}")
    if activation != "gelu" and approximate != "none":
        raise GraphError("approximate only applies when activation='gelu'")
    if bias is not None and (
        not isinstance(bias, torch.Tensor)
        or not bias.is_cuda
        or bias.get_device() != dev
        or bias.dtype != a.dtype
        or bias.dim() != 1
        or bias.shape[0] != n
    ):
        raise GraphError("bias must be a 1-D GPU tensor of output width matching dtype/device")
    if residual is not None and (
        not isinstance(residual, torch.Tensor)
        or not residual.is_cuda
        or residual.get_device() != dev
        or residual.dtype != a.dtype
        or tuple(residual.shape) != (m, n)
    ):
        raise GraphError("residual must be a GPU tensor of shape (M, N) matching dtype/device")
    cid = _check_config(config, a.dtype)
    if _arch_of_index(dev) != TARGET_ARCH:
        raise GraphError(f"the HIP kernels are built for {TARGET_ARCH}; device {a.device} is {_arch_of_index(dev)}")
    if out is None:
        out = torch.empty((m, n), dtype=a.dtype, device=a.device)
    else:
        if (
            not isinstance(out, torch.Tensor)
            or tuple(out.shape) != (m, n)
            or out.dtype != a.dtype
            or not out.is_cuda
            or out.get_device() != dev
            or not out.is_contiguous()
        ):
            raise GraphError("out must be a contiguous tensor of shape (M, N) matching dtype/device")
        out_ptr = out.untyped_storage().data_ptr()
        for src in (a, b, bias):
            if src is not None and src.untyped_storage().data_ptr() == out_ptr:
                raise GraphError("out must not share storage with inputs")
        if (
            residual is not None
            and residual.untyped_storage().data_ptr() == out_ptr
            and (residual.data_ptr() != out.data_ptr() or residual.stride() != out.stride())
        ):
            raise GraphError("residual must be out itself or not share its storage")
    if workspace is not None and (
        not isinstance(workspace, torch.Tensor) or not workspace.is_cuda or workspace.get_device() != dev
        or workspace.dtype != torch.uint8 or not workspace.is_contiguous()
    ):
        raise GraphError("workspace must be a contiguous uint8 GPU tensor on the inputs' device")
    ws = workspace
    if ws is None:
        nbytes = _plan_ids(a, b, cid)[2]
        ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    act = _act_code(activation, approximate)
    # The library's per-device set-up (the LDS limit of large tiles) applies
    # to the calling thread's current HIP device: make it the operands'
    # device for the call when it is another one.
    if dev == torch.cuda.current_device():
        return launch(a, b, bias, out, act=act, config_id=cid, workspace=ws, residual=residual)
    with torch.cuda.device(dev):
        return launch(a, b, bias, out, act=act, config_id=cid, workspace=ws, residual=residual)


# -- the transformer block's other hot ops ----------------------------------------

BLOCK_OPS = ("layer_norm", "sdpa")
_ATTENTION_DIMS = (32, 64, 96, 128)


def _block_op_supported(node, specs) -> bool:
    """Whether the HIP kernel runs this layer_norm / sdpa node's specs."""
    if node.op == "layer_norm":
        return node.spec.dtype in _DTYPES
    if node.op == "sdpa":
        q, k = specs[node.inputs[0]], specs[node.inputs[1]]
        return (len(node.inputs) == 3 and q.dtype == torch.float32 and q.shape[-1] in _ATTENTION_DIMS
                and k.shape[-1] == q.shape[-1])
    return False


def layer_norm(x: torch.Tensor, normalized_shape, weight: torch.Tensor | None = None,
               bias: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """F.layer_norm over the trailing ``normalized_shape`` dims on the gfx950 kernel."""
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)
    normalized_shape = tuple(normalized_shape)
    if not x.is_cuda or x.dtype not in _DTYPES:
        raise GraphError("hip layer_norm needs a GPU tensor of fp32, bf16 or fp16")
    if tuple(x.shape[-len(normalized_shape):]) != normalized_shape:
        raise GraphError(f"layer_norm shape {tuple(x.shape)} does not end with {normalized_shape}")
    if (weight is None) != (bias is None):
        raise GraphError("hip layer_norm takes both weight and bias or neither")
    cols = 1
    for d in normalized_shape:
        cols *= d
    xc = x.contiguous()
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    w = None if weight is None else weight.contiguous()
    b = None if bias is None else bias.contiguous()
    rows = xc.numel() // cols
    rc = _native.load().forgeml_hip_layer_norm(
        xc.data_ptr(), cols, None if w is None else w.data_ptr(), None if b is None else b.data_ptr(), y.data_ptr(),
        rows, cols, float(eps), _DTYPE_CODES[x.dtype], ctypes.c_void_p(_stream_handle(x.get_device())),
    )
    if rc != _native.OK:
        raise RuntimeError(f"forgeml_hip_layer_norm failed ({rc}): {_native.last_error()}")
    return y


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, is_causal: bool = False,
              scale: float | None = None) -> torch.Tensor:
    """F.scaled_dot_product_attention (no mask, no dropout) on the gfx950 kernel, fp32.

    The result has shape [B, H, Lq, D] and is stored [B, Lq, H, D] (returned as
    its transposed view), the layout the block's following transpose + reshape
    reads without a copy.
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise GraphError("hip attention needs rank-4 GPU tensors [batch, heads, sequence, dim]")
    if not (q.dtype == k.dtype == v.dtype == torch.float32):
        raise GraphError("hip attention is built for fp32")
    bsz, heads, lq, dim = q.shape
    lk = k.shape[2]
    if k.shape != (bsz, heads, lk, dim) or v.shape != k.shape or dim not in _ATTENTION_DIMS:
        raise GraphError(f"hip attention shapes {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)} not supported")
    qkv = []
    for t in (q, k, v):
        if t.stride(3) != 1 or t.stride(2) < dim or t.data_ptr() % 16 or any(s % 4 for s in t.stride()[:3]):
            # The kernel reads rows of D contiguous, 16-byte aligned floats at
            # least D apart (a broadcast sequence dimension is not).  A fresh
            # allocation: contiguous() would hand back a contiguous tensor
            # whose storage offset leaves it misaligned.
            t = t.clone(memory_format=torch.contiguous_format)
        qkv.append(t)
    out = torch.empty(bsz, lq, heads, dim, dtype=q.dtype, device=q.device).transpose(1, 2)
    strides = [(ctypes.c_int64 * 4)(*t.stride()) for t in (*qkv, out)]
    sc = float(scale) if scale is not None else dim ** -0.5
    rc = _native.load().forgeml_hip_attention(
        qkv[0].data_ptr(), strides[0], qkv[1].data_ptr(), strides[1], qkv[2].data_ptr(), strides[2],
        out.data_ptr(), strides[3], bsz, heads, lq, lk, dim, int(bool(is_causal)), sc, _native.DTYPE_F32,
        ctypes.c_void_p(_stream_handle(q.get_device())),
    )
    if rc != _native.OK:
        raise RuntimeError(f"forgeml_hip_attention failed ({rc}): {_native.last_error()}")
    return out


def select_kernels(graph: Graph, backend: str) -> dict[str, str]:
    """Per-node backend plan: "hip" for GEMM nodes on a gfx950 GPU, and for the
    transformer block's layer_norm / sdpa nodes the HIP kernels support; else "torch"."""
    if backend == "torch":
        return {n.name: "torch" for n in graph.nodes}
    if backend not in ("auto", "hip"):
        raise GraphError(f"unsupported backend {backend!r}; expected 'torch', 'hip', or 'auto'")
    can = available()
    specs = graph.specs()
    if backend == "hip":
        if not can:
            raise GraphError("backend 'hip' requires a gfx950 GPU and the built kernel library")
        if not all(torch.device(s.device).type == "cuda" for s in graph.inputs.values()):
            raise GraphError("backend 'hip' requires GPU graph inputs")
    plan = {}
    for node in graph.nodes:
        on_gpu = all(torch.device(specs[i].device).type == "cuda" for i in node.inputs)
        if can and node.op in GEMM_OPS and node.spec.dtype in _DTYPES and (backend == "hip" or on_gpu):
            plan[node.name] = "hip"
        elif can and on_gpu and node.op in BLOCK_OPS and _block_op_supported(node, specs):
            plan[node.name] = "hip"
        else:
            plan[node.name] = "torch"
    return plan


# Every kernel a compiled model can launch: the tiled fused GEMM, the few-row
# GEMM, the split-K reduce (in gemm_kernels.hpp), and LayerNorm / attention.
KERNEL_SOURCES = ("gemm_kernels.hpp", "skinny_kernels.hpp", "block_kernels.hip")


def kernel_source() -> str:
    """Source text of the HIP kernels a compiled model can run, each file
    under a ``// ===== csrc/<name> =====`` line (the reference returns its
    Triton module's source)."""
    root = importlib.resources.files("forgeml_amd").joinpath("csrc")
    return "\n".join(f"// ===== csrc/{name} =====\n{root.joinpath(name).read_text()}" for name in KERNEL_SOURCES)
