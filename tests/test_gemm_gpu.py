"""GPU parity of the gfx950 fused GEMM kernels against ForgeML's CPU path.

Every case compares ``forgeml_amd.kernels.matmul`` (C ABI -> HIP kernel)
with ``oracle.fused_linear.reference_cpu`` (torch addmm/mm + GELU on the
CPU, src/forgeml/ops.py:28-53) on the same seeded inputs, under the gate of
``oracle.fused_linear.tolerance``: fp32 rtol 1e-4 / atol 1e-5*sqrt(K), bf16
rtol 2e-2 / atol 5e-2, fp16 1e-2 / 1e-2; non-finite output always fails.

16-bit outputs are also held to the kernel's epilogue contract at ulp level
(``oracle.fused_linear.contract_ulp_check``): every element within one ulp of
act(rnd(rnd(sum) + bias)) for one of the two roundings of the fp64 sum the
fp32 accumulation can reach, and at least 99 % of elements exactly equal to
the rounding of the fp64 sum.  That gate sees a wrong GELU form, a skipped
rounding step or a truncating conversion, which the tolerance gate does not.
"""

from __future__ import annotations

import pytest
import torch

from forgeml_amd import kernels
from forgeml_amd.ir import GraphError
from oracle.fused_linear import contract_ulp_check, kernel_contract, reference_cpu, tolerance
from tests.cases import case_seed, gemm_inputs, to_gpu

pytestmark = pytest.mark.gpu


def _say(*parts):
    print("case:", *parts, flush=True)


def _gate(got: torch.Tensor, expected: torch.Tensor, k: int, what: str):
    got = got.detach().cpu()
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    rtol, atol = tolerance(expected.dtype, k)
    torch.testing.assert_close(got.float(), expected.float(), rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def _built_for(a_d, b_d, config) -> bool:
    """Whether ``config`` runs these operands; when not, the boundary must refuse it."""
    try:
        kernels.plan(a_d, b_d, config)
    except GraphError as e:
        assert "not built for this operand layout" in str(e), str(e)
        return False
    return True


def _contract(got, a, b, bias, activation, approximate, what, acc=None):
    report = contract_ulp_check(got, a, b, bias, activation, approximate, acc=acc)
    assert report["bad"] == 0 and report["exact_frac"] >= 0.99, f"{what}: contract {report}"


# -- the reference's own GPU kernel tests (tests/test_kernels.py:101-161) ------

_DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("dtype", _DTYPES)
@pytest.mark.parametrize("m,n,k", [(1, 17, 9), (31, 65, 33), (64, 64, 64)])
def test_matmul_small_shapes(gpu, dtype, m, n, k):
    g = torch.Generator().manual_seed(case_seed("small", m, n, k, dtype))
    a = torch.randn(m, k, generator=g).to(dtype)
    b = torch.randn(k, n, generator=g).to(dtype)
    _say("matmul", m, n, k, dtype)
    got = kernels.matmul(a.to(gpu), b.to(gpu))
    # tests/test_kernels.py:110 expects torch.matmul(a.float(), b.float()).to(dtype)
    expected = torch.matmul(a.float(), b.float()).to(dtype)
    ref_rtol, ref_atol = {torch.float32: (1e-4, 1e-4), torch.float16: (1e-2, 1e-2), torch.bfloat16: (5e-2, 5e-2)}[dtype]
    torch.testing.assert_close(got.cpu().float(), expected.float(), rtol=ref_rtol, atol=ref_atol)
    _gate(got, reference_cpu(a, b), k, "vs CPU path")


@pytest.mark.parametrize("dtype", _DTYPES)
@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_bias_gelu(gpu, dtype, approximate):
    g = torch.Generator().manual_seed(case_seed("bias_gelu", dtype, approximate))
    a = torch.randn(16, 32, generator=g).to(dtype)
    b = torch.randn(32, 24, generator=g).to(dtype)
    bias = torch.randn(24, generator=g).to(dtype)
    _say("bias_gelu", dtype, approximate)
    got = kernels.matmul(a.to(gpu), b.to(gpu), bias.to(gpu), activation="gelu", approximate=approximate).cpu()
    # tests/test_kernels.py:124-126: gelu((a.float() @ b.float()).to(dtype) + bias)
    expected = torch.nn.functional.gelu((a.float() @ b.float()).to(dtype) + bias, approximate=approximate)
    ref_rtol, ref_atol = {torch.float32: (1e-4, 1e-4), torch.float16: (1e-2, 1e-2), torch.bfloat16: (5e-2, 5e-2)}[dtype]
    torch.testing.assert_close(got.float(), expected.float(), rtol=ref_rtol, atol=ref_atol)
    _gate(got, reference_cpu(a, b, bias, "gelu", approximate), 32, "vs CPU path")
    # The kernel's epilogue order is exactly the reference kernel's contract.
    contract = kernel_contract(a, b, bias, "gelu", approximate)
    torch.testing.assert_close(got.float(), contract.float(), rtol=tolerance(dtype, 32)[0], atol=1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_strided_bias(gpu, approximate):
    g = torch.Generator().manual_seed(case_seed("strided_bias", approximate))
    a = torch.randn(16, 32, generator=g)
    b = torch.randn(32, 24, generator=g)
    bias_full = torch.randn(48, generator=g)
    _say("strided_bias", approximate)
    got = kernels.matmul(a.to(gpu), b.to(gpu), bias_full.to(gpu)[::2], activation="gelu", approximate=approximate)
    _gate(got, reference_cpu(a, b, bias_full[::2], "gelu", approximate), 32, "strided bias")


def test_noncontiguous_inputs(gpu):
    g = torch.Generator().manual_seed(case_seed("noncontig"))
    a = torch.randn(32, 16, generator=g)
    b = torch.randn(24, 32, generator=g)
    _say("noncontiguous")
    got = kernels.matmul(a.to(gpu).t(), b.to(gpu).t())
    _gate(got, reference_cpu(a.t(), b.t()), 32, "transposed A and B")


def test_out_buffer_and_overlap_reject(gpu):
    a = torch.randn(16, 16, device=gpu)
    b = torch.randn(16, 16, device=gpu)
    out = torch.empty(16, 16, device=gpu)
    _say("out buffer")
    got = kernels.matmul(a, b, out=out)
    assert got.data_ptr() == out.data_ptr()
    _gate(out, reference_cpu(a.cpu(), b.cpu()), 16, "out=")
    with pytest.raises(GraphError, match="storage"):
        kernels.matmul(a, b, out=a)


def test_relu_epilogue(gpu):
    a, b, bias = gemm_inputs(96, 200, 136, torch.float32, seed=case_seed("relu"))
    _say("relu epilogue")
    got = kernels.matmul(to_gpu(a, gpu), to_gpu(b, gpu), bias.to(gpu), activation="relu")
    _gate(got, reference_cpu(a, b, bias, "relu"), 136, "relu")


# -- ragged and edge-masked sweep (M x N x K x dtype, +-bias, +-GELU) ----------

_SWEEP_M = [1, 7, 33, 257, 1000]
_SWEEP_N = [768, 3072, 3000]
_SWEEP_K = [768, 1024, 1531]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k", _SWEEP_K)
@pytest.mark.parametrize("n", _SWEEP_N)
@pytest.mark.parametrize("m", _SWEEP_M)
def test_ragged_sweep(gpu, m, n, k, dtype):
    seed = case_seed("sweep", m, n, k, dtype)
    a, b_nt, bias = gemm_inputs(m, n, k, dtype, seed=seed, b_layout="nt")
    a_d = a.to(gpu)
    layouts = {"nt": to_gpu(b_nt, gpu), "nn": b_nt.contiguous().to(gpu)}
    bias_d = bias.to(gpu)
    acc = a.double() @ b_nt.double() if dtype != torch.float32 else None
    for with_bias in (False, True):
        for activation in ("none", "gelu"):
            expected = reference_cpu(a, b_nt, bias if with_bias else None, activation)
            for name, b_d in layouts.items():
                what = f"M={m} N={n} K={k} {dtype} B={name} bias={with_bias} act={activation} seed={seed}"
                _say(what)
                got = kernels.matmul(a_d, b_d, bias_d if with_bias else None, activation=activation)
                _gate(got, expected, k, what)
                if acc is not None:
                    _contract(got, a, b_nt, bias if with_bias else None, activation, "none", what, acc=acc)


# -- every tile configuration x operand layout ---------------------------------

def _layouts(m, n, k, dtype, seed):
    """(name, make_a, make_b) covering the K-, MN-contiguous and generic load paths.

    The makers build the operand on a device so that strided views keep
    their strides there.
    """
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(m, k, generator=g) * k ** -0.25).to(dtype)
    w = (torch.randn(n, k, generator=g) * k ** -0.25).to(dtype)
    a_pad = torch.zeros(m, 2 * k, dtype=dtype)
    a_pad[:, ::2] = a
    row_major_a = lambda dev: a.to(dev)                          # stride (K, 1)
    col_major_a = lambda dev: a.t().contiguous().to(dev).t()     # stride (1, M)
    strided_a = lambda dev: a_pad.to(dev)[:, ::2]                # stride (2K, 2): generic path
    b_nt = lambda dev: w.to(dev).t()                             # B = W^T, stride (1, K)
    b_kn = lambda dev: w.t().contiguous().to(dev)                # B [K,N], stride (N, 1)
    return a, w, [
        ("K,K", row_major_a, b_nt),
        ("K,MN", row_major_a, b_kn),
        ("MN,K", col_major_a, b_nt),
        ("MN,MN", col_major_a, b_kn),
        ("G,G", strided_a, b_nt),
    ]


@pytest.mark.parametrize("dtype", _DTYPES)
def test_every_config_and_layout(gpu, dtype):
    m, n, k = 392, 328, 520  # multiples of 8, not of any tile: edge tiles everywhere
    seed = case_seed("configs", dtype)
    a, w, layouts = _layouts(m, n, k, dtype, seed)
    g = torch.Generator().manual_seed(seed + 1)
    bias = (torch.rand(n, generator=g) * 0.2 - 0.1).to(dtype)
    expected = reference_cpu(a, w.t(), bias, "gelu")
    acc = a.double() @ w.t().double()
    for config in kernels.candidates(dtype):
        for name, make_a, make_b in layouts:
            what = f"{dtype} config={config} layout={name} seed={seed}"
            _say(what)
            a_d, b_d = make_a(gpu), make_b(gpu)
            if config in (kernels.SKINNY_FP32, kernels.SKINNY_H16):
                # The few-row kernel takes at most 64 rows: an explicit request is refused.
                with pytest.raises(GraphError, match="few-row"):
                    kernels.matmul(a_d, b_d, bias.to(gpu), activation="gelu", config=config)
                continue
            if not _built_for(a_d, b_d, config):
                with pytest.raises(GraphError, match="not built"):
                    kernels.matmul(a_d, b_d, bias.to(gpu), activation="gelu", config=config)
                continue
            got = kernels.matmul(a_d, b_d, bias.to(gpu), activation="gelu", config=config)
            _gate(got, expected, k, what)
            if dtype != torch.float32:
                _contract(got, a, w.t(), bias, "gelu", "none", what, acc=acc)


# -- rows not 16-byte aligned, and split K ----------------------------------------
#
# Odd K (fp32 rows 4-byte aligned: dword DMA; 16-bit rows 2-byte aligned:
# element loads) and K = 2 mod 8 (16-bit rows 4-byte aligned: dword DMA),
# with B as W^T or as contiguous [K,N].  The small grids (a few 64x64 or
# 128x128 tiles) split K over workgroups and reduce through the workspace.

@pytest.mark.parametrize("dtype", _DTYPES)
@pytest.mark.parametrize("m,n,k", [(392, 328, 521), (392, 328, 522), (1000, 1024, 522), (3, 200, 2049)])
def test_unaligned_k_layouts(gpu, dtype, m, n, k):
    seed = case_seed("unaligned", m, n, k, dtype)
    a, b_nt, bias = gemm_inputs(m, n, k, dtype, seed=seed, b_layout="nt")
    expected = reference_cpu(a, b_nt, bias, "gelu")
    a_d, bias_d = a.to(gpu), bias.to(gpu)
    layouts = {"nt": to_gpu(b_nt, gpu), "nn": b_nt.contiguous().to(gpu)}
    tiled = tuple(c for c in kernels.candidates(dtype) if c not in (kernels.SKINNY_FP32, kernels.SKINNY_H16))
    for config in (kernels.DEFAULT_CONFIG,) + tiled:
        for name, b_d in layouts.items():
            what = f"M={m} N={n} K={k} {dtype} B={name} config={config} seed={seed}"
            _say(what)
            if not _built_for(a_d, b_d, config):
                with pytest.raises(GraphError, match="not built"):
                    kernels.matmul(a_d, b_d, bias_d, activation="gelu", config=config)
                continue
            got = kernels.matmul(a_d, b_d, bias_d, activation="gelu", config=config)
            _gate(got, expected, k, what)


@pytest.mark.parametrize("dtype", _DTYPES)
def test_split_k_epilogues(gpu, dtype):
    m, n, k = 5, 640, 3000
    seed = case_seed("split_k", dtype)
    # B stored [K, N]: the tiled kernels run it (the few-row kernel takes W^T).
    a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed, b_layout="nn")
    ws = kernels.workspace_for(m, n, k, dtype, -1, gpu)
    assert ws is not None, "this skinny shape is expected to split K"
    a_d, b_d, bias_d = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
    for with_bias in (False, True):
        for activation, approximate in (("none", "none"), ("gelu", "none"), ("gelu", "tanh"), ("relu", "none")):
            what = f"split-K {dtype} bias={with_bias} act={activation}/{approximate} seed={seed}"
            _say(what)
            got = kernels.matmul(a_d, b_d, bias_d if with_bias else None, activation=activation,
                                 approximate=approximate)
            _gate(got, reference_cpu(a, b, bias if with_bias else None, activation, approximate), k, what)
    # The slices are summed in a fixed order: repeated calls are bit-identical.
    first = kernels.matmul(a_d, b_d, bias_d, activation="gelu")
    assert torch.equal(first, kernels.matmul(a_d, b_d, bias_d, activation="gelu"))


def test_split_k_workspace_is_checked(gpu):
    m, n, k = 1, 768, 4096
    a, b, _ = gemm_inputs(m, n, k, torch.float32, seed=case_seed("ws_check"), bias=False, b_layout="nn")
    a_d, b_d = a.to(gpu), to_gpu(b, gpu)
    out = torch.empty(m, n, device=gpu)
    _say("split-K workspace check")
    with pytest.raises(RuntimeError, match="workspace"):
        kernels.launch(a_d, b_d, None, out, act=0, config_id=-1, workspace=None)
    ws = kernels.workspace_for(m, n, k, torch.float32, -1, gpu)
    kernels.launch(a_d, b_d, None, out, act=0, config_id=-1, workspace=ws)
    _gate(out, reference_cpu(a, b), k, "split-K explicit workspace")
    # matmul with a caller's workspace: no per-call plan, the same result; a
    # workspace too small is refused by the library before any launch.
    got = kernels.matmul(a_d, b_d, workspace=ws)
    assert torch.equal(got, out)
    with pytest.raises(RuntimeError, match="workspace"):
        kernels.matmul(a_d, b_d, workspace=ws[:16])
    with pytest.raises(GraphError, match="workspace"):
        kernels.matmul(a_d, b_d, workspace=ws.view(torch.float32))


# -- the 64x64 tile's two LDS rings ----------------------------------------------

@pytest.mark.parametrize("dtype", _DTYPES)
def test_small_tile_rings(gpu, dtype):
    """The 64x64 tile rings through four LDS stages on grids of at most 512
    workgroups and two on larger ones, for 16-byte and 4-byte K-contiguous rows."""
    cfg = next(c for c in kernels.candidates(dtype) if (c.block_m, c.block_n) == (64, 64))
    odd_k = 1025 if dtype == torch.float32 else 1026  # 4-byte rows
    for m, n, k in ((1000, 3072, 1024), (1000, 3072, odd_k), (200, 640, 1024), (200, 640, odd_k)):
        seed = case_seed("rings", m, n, k, dtype)
        a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed)
        a_d, b_d, bias_d = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
        info = kernels.plan(a_d, b_d, cfg)
        wgs = -(-m // 64) * -(-n // 64) * info["k_splits"]
        what = f"64x64 M={m} N={n} K={k} {dtype} workgroups={wgs} seed={seed}"
        _say(what)
        got = kernels.matmul(a_d, b_d, bias_d, activation="gelu", config=cfg)
        rows = _row_sample(m, 96, seed)
        expected = reference_cpu(a[rows], b, bias, "gelu")
        _gate(got.cpu()[rows], expected, k, what)
        if dtype != torch.float32:
            _contract(got.cpu()[rows], a[rows], b, bias, "gelu", "none", what)


# -- the few-row kernel (M <= 64, K-contiguous A and B) -------------------------
#
# K values cover 16-byte rows (768), 4-byte rows (odd fp32 K 1531; 16-bit
# K = 2 mod 8: 1002, 2050) and 2-byte rows (odd 16-bit K 1531, 2001), and both
# ring depths (2 chunks in flight up to 6 chunks per wave: 16-bit K <= 1536,
# fp32 K <= 768; else 4); M covers 1..4 row blocks of 16 and N edges of the
# 16-column workgroups.

@pytest.mark.parametrize("dtype", _DTYPES)
@pytest.mark.parametrize("k", [8, 768, 1002, 1531, 2001, 2050])
def test_few_row_kernel(gpu, dtype, k):
    config = kernels.SKINNY_FP32 if dtype == torch.float32 else kernels.SKINNY_H16
    for m in (1, 5, 16, 17, 33, 64):
        for n in (16, 40, 3000):
            seed = case_seed("few_row", m, n, k, dtype)
            a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed)
            a_d, b_d, bias_d = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
            for activation, approximate in (("gelu", "none"), ("gelu", "tanh"), ("none", "none"), ("relu", "none")):
                what = f"few-row M={m} N={n} K={k} {dtype} act={activation}/{approximate} seed={seed}"
                _say(what)
                got = kernels.matmul(a_d, b_d, bias_d, activation=activation, approximate=approximate, config=config)
                _gate(got, reference_cpu(a, b, bias, activation, approximate), k, what)
            got = kernels.matmul(a_d, b_d, config=config)
            _gate(got, reference_cpu(a, b), k, f"few-row M={m} N={n} K={k} {dtype} no bias, explicit config")


def _at_offset(t: torch.Tensor, device, elems: int) -> torch.Tensor:
    """A copy of 2-D ``t`` on ``device`` whose storage starts ``elems`` elements
    past an allocation (so its base is not 16-byte aligned), same strides."""
    flat = torch.zeros(t.numel() + elems + 8, dtype=t.dtype, device=device)
    view = flat[elems:elems + t.numel()].view(t.shape)
    view.copy_(t.to(device))
    return view


@pytest.mark.parametrize("dtype", _DTYPES)
def test_few_row_kernel_misaligned_bases(gpu, dtype):
    """Operands whose base addresses and rows sit at every element offset of a
    16-byte block (odd and even K), on the few-row kernel's dword-aligned
    loads: the last row of each buffer ends inside a 16-byte block, where the
    tail lanes realign an aligned block instead."""
    cfg = kernels.SKINNY_FP32 if dtype == torch.float32 else kernels.SKINNY_H16
    esz = torch.tensor([], dtype=dtype).element_size()
    for k in (1531, 1002, 37, 2001):
        for m, n in ((1, 3000), (5, 40), (33, 200)):
            seed = case_seed("few_row_misaligned", m, n, k, dtype)
            a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed)
            expected = reference_cpu(a, b, bias, "gelu")
            for off_a, off_b in ((1, 3), (16 // esz - 1, 2), (2, 16 // esz - 1), (0, 1)):
                a_d = _at_offset(a, gpu, off_a)
                w_d = _at_offset(b.t().contiguous(), gpu, off_b)  # W [N, K] row-major; B = W^T
                b_d = w_d.t()
                what = f"few-row misaligned M={m} N={n} K={k} {dtype} offsets=({off_a},{off_b}) seed={seed}"
                _say(what)
                plan = kernels.plan(a_d, b_d, cfg)
                assert plan["kernel"] == "few-row", plan
                got = kernels.matmul(a_d, b_d, bias.to(gpu), activation="gelu", config=cfg)
                _gate(got, expected, k, what)
                if dtype != torch.float32:
                    _contract(got, a, b, bias, "gelu", "none", what)


def test_few_row_kernel_strided_rows_and_determinism(gpu):
    # A rows padded to a longer stride, bias strided: still K-contiguous.
    m, n, k = 24, 200, 520
    g = torch.Generator().manual_seed(case_seed("few_row_strided"))
    a_full = torch.randn(m, k + 40, generator=g) * k ** -0.25
    w = torch.randn(n, k, generator=g) * k ** -0.25
    bias_full = torch.rand(2 * n, generator=g) * 0.2 - 0.1
    a = a_full[:, :k]
    expected = reference_cpu(a, w.t(), bias_full[::2], "gelu")
    a_d = a_full.to(gpu)[:, :k]
    b_d = w.to(gpu).t()
    bias_d = bias_full.to(gpu)[::2]
    _say("few-row strided rows")
    cfg = kernels.SKINNY_FP32
    assert kernels.plan(a_d, b_d, cfg)["kernel"] == "few-row"
    got = kernels.matmul(a_d, b_d, bias_d, activation="gelu", config=cfg)
    _gate(got, expected, k, "few-row strided rows")
    assert torch.equal(got, kernels.matmul(a_d, b_d, bias_d, activation="gelu", config=cfg))
    # Chosen by the shape heuristic for one row and a short K.
    a1 = a_d[:1]
    assert kernels.plan(a1, b_d)["kernel"] == "few-row"
    _gate(kernels.matmul(a1, b_d, bias_d, activation="gelu"), reference_cpu(a[:1], w.t(), bias_full[::2], "gelu"), k,
          "few-row auto")


# -- residual add in the epilogue (forgeml_hip_gemm_add) --------------------------

def _with_residual(expected: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
    # The reference's add node after the GEMM: torch add in the dtype.
    return expected + r.to(expected.dtype)


@pytest.mark.parametrize("dtype", _DTYPES)
def test_residual_add_every_kernel(gpu, dtype):
    # (M, N, K, B layout): a tiled launch, a split-K launch, a few-row launch.
    cases = [(300, 200, 136, "nt"), (5, 640, 3000, "nn"), (7, 3072, 512, "nt")]
    for m, n, k, layout in cases:
        seed = case_seed("residual", m, n, k, dtype)
        a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed, b_layout=layout)
        g = torch.Generator().manual_seed(seed + 1)
        r = torch.randn(m, n, generator=g).to(dtype)
        a_d, b_d, bias_d = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
        kind = kernels.plan(a_d, b_d)
        for activation in ("none", "gelu"):
            what = f"residual M={m} N={n} K={k} {dtype} {kind['kernel']} splits={kind['k_splits']} act={activation}"
            _say(what)
            expected = _with_residual(reference_cpu(a, b, bias, activation), r)
            got = kernels.matmul(a_d, b_d, bias_d, activation=activation, residual=r.to(gpu))
            _gate(got, expected, k, what)
            # The fused add is the GEMM's own output followed by torch's add:
            # the same bits.
            unfused = kernels.matmul(a_d, b_d, bias_d, activation=activation) + r.to(gpu)
            assert torch.equal(got, unfused), f"{what}: fused residual differs from GEMM + add"
            # In place: the residual is the output buffer itself.
            out = r.to(gpu)
            kernels.matmul(a_d, b_d, bias_d, activation=activation, residual=out, out=out)
            _gate(out, expected, k, what + " in place")
        # A residual with other strides (a transposed view).
        rt = r.t().contiguous().to(gpu).t()
        got = kernels.matmul(a_d, b_d, bias_d, residual=rt)
        _gate(got, _with_residual(reference_cpu(a, b, bias), r), k, f"residual strided M={m} N={n} {dtype}")


def test_residual_argument_checks(gpu):
    a = torch.randn(8, 16, device=gpu)
    b = torch.randn(16, 32, device=gpu)
    with pytest.raises(GraphError, match="residual"):
        kernels.matmul(a, b, residual=torch.randn(8, 31, device=gpu))
    with pytest.raises(GraphError, match="residual"):
        kernels.matmul(a, b, residual=torch.randn(8, 32, device=gpu, dtype=torch.bfloat16))
    base = torch.empty(16, 32, device=gpu)
    with pytest.raises(GraphError, match="residual"):
        kernels.matmul(a, b, out=base[:8], residual=base[4:12])


def test_deterministic(gpu):
    a, b, bias = gemm_inputs(512, 768, 1024, torch.bfloat16, seed=case_seed("det"))
    a, b, bias = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
    _say("determinism")
    first = kernels.matmul(a, b, bias, activation="gelu")
    second = kernels.matmul(a, b, bias, activation="gelu")
    assert torch.equal(first, second)


# -- full-size configurations: sampled rows are exact parity cases -------------

def _row_sample(m: int, count: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    rows = torch.randperm(m, generator=g)[: count - 2]
    return torch.cat([torch.tensor([0, m - 1]), rows]).sort().values


def test_fp32_4096_cube_nt(gpu):
    """fp32 M=N=K=4096, B = W^T (nn.Linear weight), bias, exact-erf GELU."""
    m = n = k = 4096
    seed = case_seed("c2", m)
    a, b, bias = gemm_inputs(m, n, k, torch.float32, seed=seed, b_layout="nt")
    _say("fp32 4096^3 NT bias+gelu", seed)
    got = kernels.matmul(to_gpu(a, gpu), to_gpu(b, gpu), bias.to(gpu), activation="gelu").cpu()
    assert torch.isfinite(got).all()
    rows = _row_sample(m, 64, seed)
    expected = reference_cpu(a[rows], b, bias, "gelu")
    _gate(got[rows], expected, k, "fp32 4096^3 sampled rows")


def test_bf16_decoder_mlp(gpu):
    """bf16 M=8192: [4096->14336]+GELU, then [14336->4096]+bias (fp32 accumulate)."""
    m, d, f = 8192, 4096, 14336
    seed = case_seed("c5", m, d, f)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(f, d, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(d, f, generator=g) * 0.02).to(torch.bfloat16)
    b2 = (torch.rand(d, generator=g) * 0.2 - 0.1).to(torch.bfloat16)
    _say("bf16 decoder MLP", seed)
    h = kernels.matmul(x.to(gpu), to_gpu(w1.t(), gpu), activation="gelu")
    y = kernels.matmul(h, to_gpu(w2.t(), gpu), b2.to(gpu))
    rows = _row_sample(m, 32, seed)
    h_rows = h[rows.to(gpu)].cpu()
    _gate(h_rows, reference_cpu(x[rows], w1.t(), None, "gelu"), d, "up GEMM sampled rows")
    _contract(h_rows, x[rows], w1.t(), None, "gelu", "none", "up GEMM sampled rows")
    # The down GEMM is checked on the kernel's own H rows (same inputs).
    y_rows = y[rows.to(gpu)].cpu()
    _gate(y_rows, reference_cpu(h_rows, w2.t(), b2), f, "down GEMM sampled rows")
    _contract(y_rows, h_rows, w2.t(), b2, "none", "none", "down GEMM sampled rows")
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_gelu_tail_contract(gpu, dtype, approximate):
    """Pre-activations spanning [-10, 4] (the GELU tail, where x Phi(x) is
    small) through the tiled, few-row and split-K epilogues: C = A[:, 0]
    exactly, B selecting column 0 of A."""
    for m, n, k, layout in ((4096, 64, 8, "nt"), (64, 48, 8, "nt"), (5, 640, 3000, "nn")):
        vals = torch.linspace(-10.0, 4.0, m)
        a = torch.zeros(m, k)
        a[:, 0] = vals
        w = torch.zeros(n, k)
        w[:, 0] = 1.0
        a, w = a.to(dtype), w.to(dtype)
        b = w.t() if layout == "nt" else w.t().contiguous()
        a_d, b_d = a.to(gpu), to_gpu(b, gpu)
        kind = kernels.plan(a_d, b_d)
        what = f"GELU tail {dtype} {approximate} M={m} N={n} K={k} {kind['kernel']} splits={kind['k_splits']}"
        _say(what)
        got = kernels.matmul(a_d, b_d, activation="gelu", approximate=approximate).cpu()
        _contract(got, a, b, None, "gelu", approximate, what)


# -- the 8-wave 256x256 16-bit tile at edges, K tails and split K -------------

def _eight_wave_config(dtype):
    (cfg,) = [c for c in kernels.candidates(dtype) if (c.block_m, c.block_n, c.num_waves) == (256, 256, 8)]
    return cfg


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(392, 328, 520), (256, 256, 64), (1000, 3000, 1536), (512, 512, 8192), (300, 700, 72),
                                   (4096, 2048, 1000)])
def test_eight_wave_tile(gpu, dtype, m, n, k):
    """The 8-wave 256x256 tiles (16-bit and fp32): edge tiles in M and N, K
    tails shorter than a stage, one-stage K, and a grid small enough to split
    K; every epilogue, 16-bit outputs also held to the contract."""
    cfg = _eight_wave_config(dtype)
    seed = case_seed("eight_wave", m, n, k, dtype)
    a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed, b_layout="nt")
    a_d, b_d, bias_d = a.to(gpu), to_gpu(b, gpu), bias.to(gpu)
    info = kernels.plan(a_d, b_d, cfg)
    acc = a.double() @ b.double()
    for with_bias in (False, True):
        for activation, approximate in (("none", "none"), ("gelu", "none"), ("gelu", "tanh"), ("relu", "none")):
            what = (f"8-wave {m}x{n}x{k} {dtype} splits={info['k_splits']} bias={with_bias} "
                    f"act={activation}/{approximate} seed={seed}")
            _say(what)
            bb, bb_d = (bias, bias_d) if with_bias else (None, None)
            got = kernels.matmul(a_d, b_d, bb_d, activation=activation, approximate=approximate, config=cfg)
            _gate(got, reference_cpu(a, b, bb, activation, approximate), k, what)
            if dtype != torch.float32:
                _contract(got, a, b, bb, activation, approximate, what, acc=acc)
    # residual after the activation, into a fresh output and in place
    g = torch.Generator().manual_seed(seed + 1)
    r = torch.randn(m, n, generator=g).to(dtype)
    expected = reference_cpu(a, b, bias, "gelu") + r
    got = kernels.matmul(a_d, b_d, bias_d, activation="gelu", residual=r.to(gpu), config=cfg)
    _gate(got, expected, k, f"8-wave residual {m}x{n}x{k}")
    assert torch.equal(got, kernels.matmul(a_d, b_d, bias_d, activation="gelu", config=cfg) + r.to(gpu))
    out = r.to(gpu)
    kernels.matmul(a_d, b_d, bias_d, activation="gelu", residual=out, out=out, config=cfg)
    _gate(out, expected, k, f"8-wave residual in place {m}x{n}x{k}")
    # deterministic
    assert torch.equal(kernels.matmul(a_d, b_d, bias_d, config=cfg), kernels.matmul(a_d, b_d, bias_d, config=cfg))


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_bf16_gelu_table_equals_arithmetic_form(gpu, approximate):
    """The 8-wave tile's GELU table against the per-element form of the 64x64
    tile, on every bf16 bit pattern as a pre-activation (C = A[:, 0], exact:
    K = 8 and B one-hot), alone, after a bias per column and before a
    residual: the same bits everywhere (NaN where NaN)."""
    dtype = torch.bfloat16
    m, n, k = 65536, 256, 8
    a = torch.zeros(m, k, dtype=dtype)
    a[:, 0] = torch.arange(m, dtype=torch.int32).to(torch.int16).view(dtype)
    w = torch.zeros(n, k, dtype=dtype)
    w[:, 0] = 1.0
    g = torch.Generator().manual_seed(case_seed("gelu_table", approximate))
    bias = (torch.randn(n, generator=g) * 4).to(dtype)
    r = torch.randn(m, n, generator=g).to(dtype)
    a_d, b_d = a.to(gpu), w.to(gpu).t()
    (arith,) = [c for c in kernels.candidates(dtype) if (c.block_m, c.block_n) == (64, 64)]
    table = _eight_wave_config(dtype)
    for bias_d, res_d in ((None, None), (bias.to(gpu), None), (bias.to(gpu), r.to(gpu))):
        what = f"GELU table {approximate} bias={bias_d is not None} residual={res_d is not None}"
        _say(what)
        outs = [kernels.matmul(a_d, b_d, bias_d, activation="gelu", approximate=approximate, residual=res_d,
                               config=cfg).cpu() for cfg in (table, arith)]
        got, want = (o.view(torch.int16) for o in outs)
        nan = outs[1].isnan()
        assert torch.equal(outs[0].isnan(), nan), what
        diff = (got != want) & ~nan
        assert not diff.any(), f"{what}: {int(diff.sum())} outputs differ, first at {diff.nonzero()[0].tolist()}"


# -- seeded random problems through the few-row kernel ----------------------------

def test_few_row_kernel_random_problems(gpu):
    """200 seeded random problems on the few-row kernel: M in 1..64, N in 1..300,
    K in 1..2600, every dtype, operand bases at random element offsets, every
    epilogue; against the CPU path (and the contract for 16-bit outputs)."""
    g = torch.Generator().manual_seed(case_seed("few_row_random"))
    acts = (("gelu", "none"), ("gelu", "tanh"), ("none", "none"), ("relu", "none"))
    for i in range(200):
        m = int(torch.randint(1, 65, (1,), generator=g))
        n = int(torch.randint(1, 301, (1,), generator=g))
        k = int(torch.randint(1, 2601, (1,), generator=g))
        dtype = _DTYPES[int(torch.randint(0, 3, (1,), generator=g))]
        activation, approximate = acts[int(torch.randint(0, 4, (1,), generator=g))]
        off_a, off_b = (int(v) for v in torch.randint(0, 8, (2,), generator=g))
        seed = case_seed("few_row_random", i)
        a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed)
        cfg = kernels.SKINNY_FP32 if dtype == torch.float32 else kernels.SKINNY_H16
        a_d = _at_offset(a, gpu, off_a)
        b_d = _at_offset(b.t().contiguous(), gpu, off_b).t()
        what = (f"few-row random #{i} M={m} N={n} K={k} {dtype} {activation}/{approximate} "
                f"offsets=({off_a},{off_b}) seed={seed}")
        _say(what)
        assert kernels.plan(a_d, b_d, cfg)["kernel"] == "few-row", what
        got = kernels.matmul(a_d, b_d, bias.to(gpu), activation=activation, approximate=approximate, config=cfg)
        _gate(got, reference_cpu(a, b, bias, activation, approximate), k, what)
        if dtype != torch.float32:
            _contract(got.cpu(), a, b, bias, activation, approximate, what)


def test_tiled_kernels_random_problems(gpu):
    """120 seeded random problems on a random built tile: M, N in 1..2000, K in
    1..3000, every dtype, B as W^T or stored [K, N], A row-major or transposed,
    every epilogue; checked on sampled rows (a tile the layout does not build
    must be refused with ECONFIG)."""
    g = torch.Generator().manual_seed(case_seed("tiled_random"))
    acts = (("gelu", "none"), ("gelu", "tanh"), ("none", "none"), ("relu", "none"))
    for i in range(120):
        m, n = (int(v) for v in torch.randint(1, 2001, (2,), generator=g))
        k = int(torch.randint(1, 3001, (1,), generator=g))
        dtype = _DTYPES[int(torch.randint(0, 3, (1,), generator=g))]
        tiles = [c for c in kernels.candidates(dtype) if c.block_n != 16]
        cfg = tiles[int(torch.randint(0, len(tiles), (1,), generator=g))]
        layout = ("nt", "nn")[int(torch.randint(0, 2, (1,), generator=g))]
        a_t = bool(torch.randint(0, 2, (1,), generator=g))
        activation, approximate = acts[int(torch.randint(0, 4, (1,), generator=g))]
        seed = case_seed("tiled_random", i)
        a, b, bias = gemm_inputs(m, n, k, dtype, seed=seed, b_layout=layout)
        a_d = a.t().contiguous().to(gpu).t() if a_t else a.to(gpu)
        b_d = to_gpu(b, gpu)
        what = (f"tiled random #{i} M={m} N={n} K={k} {dtype} tile={cfg.block_m}x{cfg.block_n}x{cfg.num_waves} "
                f"B={layout} A^T={a_t} {activation}/{approximate} seed={seed}")
        _say(what)
        if not _built_for(a_d, b_d, cfg):
            continue
        got = kernels.matmul(a_d, b_d, bias.to(gpu), activation=activation, approximate=approximate, config=cfg)
        rows = _row_sample(m, min(m, 48), seed) if m > 2 else torch.arange(m)
        expected = reference_cpu(a[rows], b, bias, activation, approximate)
        _gate(got.cpu()[rows], expected, k, what)
        if dtype != torch.float32:
            _contract(got.cpu()[rows], a[rows], b, bias, activation, approximate, what)
