"""forgeml_hip_gemm_noalloc, called through the C ABI, against forgeml_hip_gemm
with a caller workspace on the same operands: the same kernels run, so the
results are bit-identical.  Two calls in a row share the GPU's scratch
array, the second on a smaller problem, and the second's result must not
depend on what the first left there."""

from __future__ import annotations

import ctypes

import pytest
import torch

from forgeml_amd import _native, kernels
from oracle.fused_linear import reference_cpu, tolerance
from tests.cases import case_seed, gemm_inputs, to_gpu

pytestmark = pytest.mark.gpu


def _say(*parts):
    print("case:", *parts, flush=True)


def _abi_args(a, b, bias):
    bias_ptr, sbi = (None, 0) if bias is None else (bias.data_ptr(), bias.stride(0))
    return (a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0), b.stride(1), bias_ptr, sbi)


def _run_noalloc(a, b, bias, act):
    lib = _native.load()
    m, k = a.shape
    n = b.shape[1]
    out = torch.empty(m, n, dtype=a.dtype, device=a.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(a.device).cuda_stream)
    rc = lib.forgeml_hip_gemm_noalloc(*_abi_args(a, b, bias), out.data_ptr(), m, n, k, kernels._DTYPE_CODES[a.dtype],
                                      act, -1, stream)
    assert rc == _native.OK, _native.last_error()
    return out


def _run_with_workspace(a, b, bias, act):
    lib = _native.load()
    m, k = a.shape
    n = b.shape[1]
    info = kernels.plan(a, b)
    ws = torch.empty(max(info["workspace_bytes"], 16), dtype=torch.uint8, device=a.device)
    out = torch.empty(m, n, dtype=a.dtype, device=a.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(a.device).cuda_stream)
    rc = lib.forgeml_hip_gemm(*_abi_args(a, b, bias), out.data_ptr(), m, n, k, kernels._DTYPE_CODES[a.dtype], act,
                              -1, ws.data_ptr(), ws.numel(), stream)
    assert rc == _native.OK, _native.last_error()
    return out, info


# (M, N, K, B layout, dtype): two split-K problems, the second smaller, then
# one that does not split K.
_CASES = [(5, 640, 3000, "nn", torch.float32), (3, 200, 2049, "nn", torch.float32),
          (9, 768, 4096, "nn", torch.bfloat16), (2, 96, 1536, "nn", torch.bfloat16),
          (300, 200, 136, "nt", torch.float32)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_workspace_entry_point(gpu, dtype):
    cases = [c for c in _CASES if c[4] == dtype] + [_CASES[-1]]
    splits = []
    for m, n, k, layout, dt in cases:
        seed = case_seed("noalloc", m, n, k, dt)
        a, b, bias = gemm_inputs(m, n, k, dt, seed=seed, b_layout=layout)
        a_d, b_d, bias_d = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
        for act in (_native.ACT_NONE, _native.ACT_GELU_ERF):
            got = _run_noalloc(a_d, b_d, bias_d, act)
            want, info = _run_with_workspace(a_d, b_d, bias_d, act)
            _say("noalloc", m, n, k, layout, dt, "act", act, "splits", info["k_splits"], "seed", seed)
            splits.append(info["k_splits"])
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"noalloc differs from the workspace entry point at {m}x{n}x{k} {dt}"
            rtol, atol = tolerance(dt, k)
            expected = reference_cpu(a, b, bias, "gelu" if act else "none")
            torch.testing.assert_close(got.cpu().float(), expected.float(), rtol=rtol, atol=atol)
    # The first two problems split K (so they used the scratch array), the last does not.
    assert splits[0] > 1 and splits[2] > 1 and splits[-1] == 1, splits


def test_noalloc_refuses_beyond_its_scratch(gpu):
    lib = _native.load()
    limit = lib.forgeml_hip_noalloc_scratch_bytes()
    assert limit == 32 << 20
    # 2048 x 1920 outputs on the 256x256 fp32 tile are 64 tiles, so K is
    # split 8 ways: 8 planes of 2048 x 1920 fp32 need 125.8 MB, past the array.
    m, n, k = 2048, 1920, 4096
    out = (ctypes.c_int64 * 4)()
    a = torch.empty(m, k, device=gpu)
    b = torch.empty(k, n, device=gpu)  # [K, N] row-major
    cid = kernels.config_id(kernels.candidates(torch.float32)[2], torch.float32)  # 256x256
    rc = lib.forgeml_hip_gemm_plan(a.data_ptr(), k, 1, b.data_ptr(), n, 1, m, n, k, _native.DTYPE_F32, cid, out)
    assert rc == _native.OK and out[2] > limit, list(out)
    c = torch.empty(m, n, device=gpu)
    _say("noalloc refusal", m, n, k, "needs", out[2])
    rc = lib.forgeml_hip_gemm_noalloc(a.data_ptr(), k, 1, b.data_ptr(), n, 1, None, 0, c.data_ptr(), m, n, k,
                                      _native.DTYPE_F32, 0, cid, None)
    assert rc == _native.EWORKSPACE and "scratch" in _native.last_error()
