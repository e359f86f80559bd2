"""The C ABI library: it loads without a GPU, exports every symbol the header
declares, and its tile table agrees with the Python KernelConfig table.
No kernel is launched here."""

import ctypes
import re

import pytest
import torch

from forgeml_amd import _native, kernels
from forgeml_amd.ir import GraphError


def _declared_symbols() -> list[str]:
    text = _native.HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(forgeml_hip_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert _declared_symbols() == sorted(_native.SIGNATURES)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.load()
    for name in _declared_symbols():
        assert getattr(lib, name, None) is not None, name
    assert lib.forgeml_hip_abi_version() == _native.ABI_VERSION
    assert len(_native.hip_runtimes_mapped()) <= 1


def test_config_table_matches_python_candidates():
    table = _native.config_table()
    assert len(table) == len(kernels.CANDIDATES)
    for info, cfg in zip(table, kernels.CANDIDATES):
        dclass, bm, bn, bk, waves, stages, split, lds = info
        assert (bm, bn, bk, waves, stages) == (cfg.block_m, cfg.block_n, cfg.block_k, cfg.num_waves, cfg.num_stages)
        assert cfg in kernels.candidates(torch.float32 if dclass == 0 else torch.bfloat16)
        if cfg in (kernels.SKINNY_FP32, kernels.SKINNY_H16):
            # Few-row kernel: chunks of one 16-byte vector per lane, 4 lane groups.
            assert bk * (4 if dclass == 0 else 2) == 64 and split == 1 and lds == 8 * 4 * 64 * 16
        else:
            assert bk * (4 if dclass == 0 else 2) == 128 and split == 16
            # The 8-wave 16-bit 256x256 tile also holds the bf16 GELU table (2 signs x 20 binades x 128 values).
            lut = 2 * 20 * 128 * 2 if dclass == 1 and bm * bn >= 256 * 256 and waves == 8 else 0
            assert lds == stages * (bm + bn) * 128 + lut and lds <= 160 * 1024


def test_host_side_errors_without_launching():
    lib = _native.load()
    assert lib.forgeml_hip_select_config(0, 4, 4, _native.DTYPE_F32) == _native.EINVAL
    assert lib.forgeml_hip_select_config(4, 4, 4, 7) == _native.EINVAL
    assert lib.forgeml_hip_gemm_workspace_size(4, 4, 4, _native.DTYPE_F32, 99) == _native.ECONFIG
    rc = lib.forgeml_hip_gemm(None, 0, 0, None, 0, 0, None, 0, None, 4, 4, 4, 0, 0, -1, None, 0, None)
    assert rc == _native.EINVAL and "non-NULL" in _native.last_error()
    dummy = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    rc = lib.forgeml_hip_gemm(dummy, 4, 1, dummy, 4, 1, None, 0, dummy, 4, 4, 4, _native.DTYPE_BF16, 0, 0,
                              None, 0, None)
    assert rc == _native.ECONFIG and "not built for dtype" in _native.last_error()
    rc = lib.forgeml_hip_gemm(dummy, 4, 1, dummy, 4, 1, None, 0, dummy, 4, 4, 4, 0, 9, -1, None, 0, None)
    assert rc == _native.EINVAL and "activation" in _native.last_error()
    rc = lib.forgeml_hip_gemm(dummy, -4, 1, dummy, 4, 1, None, 0, dummy, 4, 4, 4, 0, 0, -1, None, 0, None)
    assert rc == _native.EINVAL


def test_heuristic_picks_built_tiles():
    lib = _native.load()
    for dtype, code in ((torch.float32, _native.DTYPE_F32), (torch.bfloat16, _native.DTYPE_BF16)):
        for m, n, k in ((1, 768, 768), (64, 2048, 512), (4096, 4096, 4096), (8192, 14336, 4096)):
            cid = lib.forgeml_hip_select_config(m, n, k, code)
            assert kernels.CANDIDATES[cid] in kernels.candidates(dtype)


def test_matmul_boundary_validation_on_cpu():
    a = torch.randn(4, 4)
    if not torch.cuda.is_available():
        with pytest.raises(GraphError, match="GPU"):
            kernels.matmul(a, a)
    with pytest.raises(GraphError):
        kernels._check_config(kernels.KernelConfig(block_m=8), torch.float32)
    with pytest.raises(GraphError):
        kernels._check_config(kernels.candidates(torch.bfloat16)[0], torch.float32)
    assert kernels._check_config(kernels.DEFAULT_CONFIG, torch.float32) == _native.CONFIG_AUTO
    source = kernels.kernel_source()
    for kernel in ("fused_gemm_kernel", "splitk_reduce_kernel", "skinny_gemm_kernel", "layer_norm_kernel",
                   "attention_kernel", "__global__"):
        assert kernel in source, kernel
    for name in kernels.KERNEL_SOURCES:
        assert f"// ===== csrc/{name} =====" in source


def test_split_k_workspace_size():
    lib = _native.load()
    f32 = _native.DTYPE_F32
    # Few output tiles and a long K: the K reduction is split over workgroups
    # and each slice needs an fp32 M x N plane.
    for m, n, k in [(1, 768, 4096), (33, 3072, 1531), (7, 768, 768)]:
        for dtype in (f32, _native.DTYPE_BF16):
            ws = lib.forgeml_hip_gemm_workspace_size(m, n, k, dtype, -1)
            plane = m * n * 4
            assert ws > 0 and ws % plane == 0 and 2 <= ws // plane <= 16, (m, n, k, dtype, ws)
    # Enough tiles to fill the GPU, or too little K to split: no workspace.
    assert lib.forgeml_hip_gemm_workspace_size(4096, 4096, 4096, f32, -1) == 0
    assert lib.forgeml_hip_gemm_workspace_size(1, 768, 64, f32, -1) == 0
    # An explicit small tile on a small grid splits too; the largest tile on a
    # grid that fills the GPU does not.
    small = next(i for i, info in enumerate(_native.config_table()) if info[0] == 0 and info[1] == 64)
    assert lib.forgeml_hip_gemm_workspace_size(64, 64, 8192, f32, small) > 0
    assert lib.forgeml_hip_gemm_workspace_size(8192, 8192, 8192, f32, small) == 0
    # A 16-bit config id for an fp32 problem is rejected.
    h16 = next(i for i, info in enumerate(_native.config_table()) if info[0] == 1)
    assert lib.forgeml_hip_gemm_workspace_size(64, 64, 8192, f32, h16) == _native.ECONFIG


def test_split_k_needs_workspace():
    lib = _native.load()
    dummy = ctypes.c_void_p(16)  # never dereferenced: the workspace check fails before any launch
    m, n, k = 1, 768, 4096
    need = lib.forgeml_hip_gemm_workspace_size(m, n, k, _native.DTYPE_F32, -1)
    assert need > 0
    # B stored [K, N] (N-contiguous): the tiled kernels run it, splitting K.
    # The plan must confirm the split before any dummy-pointer call: without
    # it the workspace check would not stop the launch.
    out = (ctypes.c_int64 * 4)()
    assert lib.forgeml_hip_gemm_plan(dummy, k, 1, dummy, n, 1, m, n, k, _native.DTYPE_F32, -1, out) == _native.OK
    assert out[1] > 1 and out[2] > 0, "this layout no longer splits K: the calls below would launch"
    rc = lib.forgeml_hip_gemm(dummy, k, 1, dummy, n, 1, None, 0, dummy, m, n, k, 0, 1, -1, None, 0, None)
    assert rc == _native.EWORKSPACE and "workspace" in _native.last_error()
    rc = lib.forgeml_hip_gemm(dummy, k, 1, dummy, n, 1, None, 0, dummy, m, n, k, 0, 1, -1, dummy, need - 4, None)
    assert rc == _native.EWORKSPACE
    rc = lib.forgeml_hip_gemm(dummy, k, 1, dummy, n, 1, None, 0, dummy, m, n, k, 0, 1, -1, ctypes.c_void_p(20), need,
                              None)
    assert rc == _native.EWORKSPACE and "aligned" in _native.last_error()


def test_few_row_kernel_selection():
    lib = _native.load()
    table = _native.config_table()
    skinny = [i for i, info in enumerate(table) if info[2] == 16]
    assert len(skinny) == 2 and {table[i][0] for i in skinny} == {0, 1}
    for dtype in (_native.DTYPE_F32, _native.DTYPE_BF16):
        # Few rows and enough column groups: the few-row kernel, up to 32
        # chunks of K per wave for one row block, 24 up to 48 rows, 8 at 64.
        assert lib.forgeml_hip_select_config(1, 3072, 1024, dtype) in skinny
        assert lib.forgeml_hip_select_config(48, 3072, 1024, dtype) in skinny
        assert lib.forgeml_hip_select_config(1, 3000, 4096, dtype) in skinny
        assert lib.forgeml_hip_select_config(33, 3000, 1531, dtype) in skinny
        assert lib.forgeml_hip_select_config(17, 3000, 3000, dtype) in skinny
        # More than 64 rows, a long K, or too few column groups: the tiled kernels.
        assert lib.forgeml_hip_select_config(65, 3072, 1024, dtype) not in skinny
        assert lib.forgeml_hip_select_config(64, 4096, 4096, dtype) not in skinny
        assert lib.forgeml_hip_select_config(64, 512, 2048, dtype) not in skinny
        assert lib.forgeml_hip_select_config(1, 256, 16384, dtype) not in skinny
        assert lib.forgeml_hip_select_config(33, 3000, 16384, dtype) not in skinny
    # The few-row kernel needs K-contiguous A and B and at most 64 rows.
    dummy = ctypes.c_void_p(16)
    f32_skinny = next(i for i in skinny if table[i][0] == 0)
    rc = lib.forgeml_hip_gemm(dummy, 64, 1, dummy, 64, 1, None, 0, dummy, 8, 64, 64, 0, 0, f32_skinny, None, 0, None)
    assert rc == _native.ECONFIG and "few-row" in _native.last_error()
    rc = lib.forgeml_hip_gemm(dummy, 64, 1, dummy, 1, 64, None, 0, dummy, 65, 64, 64, 0, 0, f32_skinny, None, 0, None)
    assert rc == _native.ECONFIG


def test_gemm_plan_reports_what_runs():
    lib = _native.load()
    out = (ctypes.c_int64 * 4)()
    dummy = ctypes.c_void_p(256)  # only its alignment is looked at
    f32 = _native.DTYPE_F32

    def plan(m, n, k, sam, sak, sbk, sbn, dtype=f32, cid=-1, a=dummy, b=dummy):
        rc = lib.forgeml_hip_gemm_plan(a, sam, sak, b, sbk, sbn, m, n, k, dtype, cid, out)
        return rc, list(out)

    # One row, B = W^T with 16-byte rows: the few-row kernel, no split.
    rc, (cid, splits, ws, kind) = plan(1, 3072, 1024, 1024, 1, 1, 1024)
    assert rc == 0 and kind == 1 and splits == 1 and ws == 0
    # The same with B stored [K, N]: a tiled kernel splitting K over a workspace.
    rc, (cid, splits, ws, kind) = plan(1, 768, 4096, 4096, 1, 768, 1)
    assert rc == 0 and kind == 0 and splits > 1 and ws == splits * 1 * 768 * 4
    assert ws <= lib.forgeml_hip_gemm_workspace_size(1, 768, 4096, f32, -1)
    # A large square GEMM: the shape heuristic's tile, no split.
    rc, (cid, splits, ws, kind) = plan(4096, 4096, 4096, 4096, 1, 1, 4096)
    assert rc == 0 and kind == 0 and splits == 1 and ws == 0
    assert cid == lib.forgeml_hip_select_config(4096, 4096, 4096, f32)
    # Odd fp32 K and 33 rows: 4-byte rows on the few-row kernel.
    rc, (cid, splits, ws, kind) = plan(33, 3000, 1531, 1531, 1, 1, 1531)
    assert rc == 0 and kind == 1 and splits == 1 and ws == 0
    # Errors are the launch's errors.
    rc, _ = plan(8, 64, 64, 64, 1, -1, 1)  # negative stride
    assert rc == _native.EINVAL
    assert lib.forgeml_hip_gemm_plan(dummy, 4, 1, dummy, 1, 4, 4, 4, 4, f32, -1, None) == _native.EINVAL


def test_cached_plans_match_the_library():
    """kernels.plan answers from a cache keyed by operand geometry: every answer equals a
    fresh forgeml_hip_gemm_plan call, including operands that differ only in alignment
    (16-byte, 4-byte and 2-byte bases of the same shape plan different loaders)."""
    lib = _native.load()
    out = (ctypes.c_int64 * 4)()
    kernels._PLAN_CACHE.clear()
    for dtype, k in ((torch.float32, 1024), (torch.float32, 1531), (torch.bfloat16, 1536), (torch.bfloat16, 1531)):
        base = torch.zeros(64 * 1536 + 16, dtype=dtype)
        for off in (0, 1, 2, 4):
            a = base[off:off + 33 * k].view(33, k)
            w = torch.zeros(3000, k, dtype=dtype)
            for b in (w.t(), w.t().contiguous()):
                for config in (kernels.DEFAULT_CONFIG, *kernels.candidates(dtype)):
                    try:
                        got = kernels.plan(a, b, config)
                    except GraphError:
                        got = None
                    rc = lib.forgeml_hip_gemm_plan(a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0),
                                                   b.stride(1), 33, 3000, k, kernels._DTYPE_CODES[dtype],
                                                   kernels.config_id(config, dtype), out)
                    if rc != _native.OK:
                        assert got is None, (dtype, k, off, config)
                        continue
                    assert got is not None and (got["config_id"], got["k_splits"], got["workspace_bytes"]) == \
                        (out[0], out[1], out[2]), (dtype, k, off, config)
                    assert kernels.plan(a, b, config) == got  # the cached answer is stable
    assert kernels._PLAN_CACHE


def test_block_kernel_argument_errors():
    lib = _native.load()
    dummy = ctypes.c_void_p(256)
    f32 = _native.DTYPE_F32
    assert lib.forgeml_hip_layer_norm(None, 8, None, None, dummy, 4, 8, 1e-5, f32, None) == _native.EINVAL
    assert lib.forgeml_hip_layer_norm(dummy, 8, dummy, None, dummy, 4, 8, 1e-5, f32, None) == _native.EINVAL
    assert lib.forgeml_hip_layer_norm(dummy, 4, None, None, dummy, 4, 8, 1e-5, f32, None) == _native.EINVAL  # stride < cols
    assert lib.forgeml_hip_layer_norm(dummy, 8, None, None, dummy, 4, 8, 0.0, f32, None) == _native.EINVAL
    st = (ctypes.c_int64 * 4)(4096, 64 * 64, 64, 1)
    args = (dummy, st, dummy, st, dummy, st, dummy, st)
    # head dim 48 is not built; fp16 is not built; a non-unit dim stride is refused
    assert lib.forgeml_hip_attention(*args, 1, 1, 64, 64, 48, 1, 0.125, f32, None) == _native.EINVAL
    assert "head dim" in _native.last_error()
    assert lib.forgeml_hip_attention(*args, 1, 1, 64, 64, 64, 1, 0.125, _native.DTYPE_F16, None) == _native.EINVAL
    # k and v rows closer than the head dim (overlapping rows) are refused
    close = (ctypes.c_int64 * 4)(4096, 64 * 64, 32, 1)
    assert lib.forgeml_hip_attention(dummy, st, dummy, close, dummy, st, dummy, st, 1, 1, 64, 64, 64, 1, 0.125, f32,
                                     None) == _native.EINVAL
    assert "apart" in _native.last_error()
    bad = (ctypes.c_int64 * 4)(4096, 64 * 64, 64, 2)
    assert lib.forgeml_hip_attention(dummy, bad, dummy, st, dummy, st, dummy, st, 1, 1, 64, 64, 64, 1, 0.125, f32,
                                     None) == _native.EINVAL


def test_launch_size_limits():
    """A dispatch covers fewer than 2^32 work-items: shapes past that are
    refused with the config asked for, and AUTO plans a config that fits
    (host-side planning only: nothing is launched)."""
    lib = _native.load()
    out = (ctypes.c_int64 * 4)()

    def plan(m, n, k, ld, dtype, cid):
        rc = lib.forgeml_hip_gemm_plan(ctypes.c_void_p(1 << 40), ld, 1, ctypes.c_void_p(1 << 41), 1, ld, m, n, k,
                                       dtype, cid, out)
        return rc, tuple(out)

    f32, bf16 = _native.DTYPE_F32, _native.DTYPE_BF16
    tile64 = kernels.config_id(kernels.candidates(torch.float32)[1], torch.float32)
    # 2^18 x 2^18 outputs: 2^24 workgroups of 256 threads on the 64x64 tile.
    assert plan(1 << 18, 1 << 18, 64, 64, f32, tile64)[0] == _native.EINVAL
    assert "work-items" in _native.last_error()
    rc, (cid, _, _, _) = plan(1 << 18, 1 << 18, 64, 64, f32, -1)
    assert rc == _native.OK and kernels.CANDIDATES[cid].block_m >= 128
    # 2^27 columns on the few-row kernel: 2^23 workgroups of 512 threads.
    few_row = kernels.config_id(kernels.SKINNY_H16, torch.bfloat16)
    assert plan(16, 1 << 27, 16, 16, bf16, few_row)[0] == _native.EINVAL
    rc, (cid, _, _, kind) = plan(16, 1 << 27, 16, 16, bf16, -1)
    assert rc == _native.OK and kind == 0
    assert lib.forgeml_hip_select_config(16, 1 << 27, 16, bf16) == cid
    rc, (_, _, _, kind) = plan(16, 1 << 25, 16, 16, bf16, few_row)
    assert rc == _native.OK and kind == 1
    # 16-bit odd K: element loads, built for the 64x64 tile only.  2^18 x 2^18
    # outputs need 2^32 work-items there, so AUTO refuses with a clear error;
    # half the rows fit.
    rc, _ = plan(1 << 18, 1 << 18, 15, 15, bf16, -1)
    assert rc == _native.EINVAL and "every tile" in _native.last_error()
    rc, (cid, _, _, _) = plan(1 << 17, 1 << 18, 15, 15, bf16, -1)
    assert rc == _native.OK and kernels.CANDIDATES[cid].block_m == 64
    # select_config skips tiles past the bound (fp32 64x64 would need 2^32).
    cid = lib.forgeml_hip_select_config(1 << 18, 1 << 18, 64, f32)
    assert cid >= 0 and kernels.CANDIDATES[cid].block_m >= 128
    # Attention: one 256-thread workgroup per query block.
    dummy = ctypes.c_void_p(256)
    st = (ctypes.c_int64 * 4)(1 << 20, 512 * 32, 32, 1)
    args = (dummy, st, dummy, st, dummy, st, dummy, st)
    assert lib.forgeml_hip_attention(*args, 1 << 20, 16, 512, 512, 32, 0, 0.125, f32, None) == _native.EINVAL
    assert "query blocks" in _native.last_error()


def test_tiles_refuse_layouts_they_are_not_built_for():
    """16-bit tiles above 64x64 are not built for element loads (an odd K),
    the 8-wave 16-bit tile only for two K-contiguous operands with 16-byte
    rows, and the 8-wave fp32 tile not for element loads of both operands:
    an explicit request is refused with ECONFIG; AUTO plans a built tile
    (host-side planning only: nothing is launched)."""
    lib = _native.load()
    out = (ctypes.c_int64 * 4)()
    dummy = ctypes.c_void_p(256)
    bf16 = _native.DTYPE_BF16
    ids = {(cfg.block_m, cfg.num_waves): kernels.config_id(cfg, torch.bfloat16)
           for cfg in kernels.candidates(torch.bfloat16) if cfg.block_n == cfg.block_m}

    def plan(k, sbk, sbn, cid):
        # A row-major [M, K]; B with strides (sbk, sbn); M = N = 1024.
        return lib.forgeml_hip_gemm_plan(dummy, k, 1, dummy, sbk, sbn, 1024, 1024, k, bf16, cid, out)

    for (bm, waves), cid in ids.items():
        # Odd K: 16-bit rows only 2-byte aligned, element loads for A.
        refused = bm > 64
        assert (plan(1531, 1, 1531, cid) == _native.ECONFIG) == refused, (bm, waves)
        if refused:
            assert "not built for this operand layout" in _native.last_error()
        # B stored [K, N]: the transposing loader.
        assert (plan(1024, 1024, 1, cid) == _native.ECONFIG) == (waves > 4), (bm, waves)
        # Both K-contiguous with 16-byte rows: every tile.
        assert plan(1024, 1, 1024, cid) == _native.OK
    # AUTO picks a built tile for the odd-K layout.
    assert plan(1531, 1, 1531, -1) == _native.OK and kernels.CANDIDATES[out[0]].block_m == 64
    # fp32: the 8-wave 256x256 tile takes no element loads of both operands
    # (4-byte rows of an odd K above 128x128); AUTO plans another tile.
    f32 = _native.DTYPE_F32
    cid = kernels.config_id(next(c for c in kernels.candidates(torch.float32) if c.num_waves == 8), torch.float32)
    big = lambda k, c: lib.forgeml_hip_gemm_plan(dummy, k, 1, dummy, 1, k, 4096, 4096, k, f32, c, out)  # noqa: E731
    assert big(4095, cid) == _native.ECONFIG and "not built for this operand layout" in _native.last_error()
    assert big(4096, cid) == _native.OK
    assert big(4095, -1) == _native.OK and out[0] != cid


def _gfx950_kernel_metadata(path):
    """The amdhsa.kernels metadata of every gfx950 code object the library
    embeds: clang offload bundles (one per translation unit) hold ELF code
    objects whose AMDGPU note (type 32) is a msgpack map."""
    import struct

    msgpack = pytest.importorskip("msgpack")
    data = path.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    kernels_md = []
    start = data.find(magic)
    while start >= 0:
        (count,) = struct.unpack_from("<Q", data, start + len(magic))
        pos = start + len(magic) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, pos)
            triple = data[pos + 24:pos + 24 + tlen].decode()
            pos += 24 + tlen
            if not triple.endswith("gfx950") or size == 0:
                continue
            elf = data[start + off:start + off + size]
            assert elf[:4] == b"\x7fELF", triple
            shoff, = struct.unpack_from("<Q", elf, 0x28)
            shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
            for s in range(shnum):
                sh = shoff + s * shentsize
                if struct.unpack_from("<I", elf, sh + 4)[0] != 7:  # SHT_NOTE
                    continue
                noff, nsize = struct.unpack_from("<QQ", elf, sh + 0x18)
                p = noff
                while p < noff + nsize:
                    namesz, descsz, ntype = struct.unpack_from("<III", elf, p)
                    name = elf[p + 12:p + 12 + namesz].rstrip(b"\0")
                    desc = p + 12 + ((namesz + 3) & ~3)
                    if name == b"AMDGPU" and ntype == 32:
                        kernels_md += msgpack.unpackb(elf[desc:desc + descsz], raw=False, strict_map_key=False)["amdhsa.kernels"]
                    p = desc + ((descsz + 3) & ~3)
        start = data.find(magic, start + 1)
    return kernels_md


def test_no_kernel_uses_scratch():
    """Register spills go to per-lane scratch memory, a slow path the tiles are
    sized to avoid (the 4-wave 256x256 tile's accumulators fill the AGPRs, and
    two epilogue changes once pushed it to 1 KB of scratch per lane).  Read the
    built library's own gfx950 code-object metadata and require none."""
    if not _native.LIBRARY_PATH.exists():
        pytest.skip("library not built")
    md = _gfx950_kernel_metadata(_native.LIBRARY_PATH)
    names = [k[".name"] for k in md]
    assert any("fused_gemm_kernel" in n for n in names) and any("attention_kernel" in n for n in names)
    spilled = [(k[".name"], k.get(".private_segment_fixed_size"), k.get(".vgpr_spill_count"))
               for k in md if k.get(".private_segment_fixed_size", 0) or k.get(".vgpr_spill_count", 0)]
    assert not spilled, spilled
