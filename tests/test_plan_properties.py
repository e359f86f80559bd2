"""Property tests of the native launch planner over random shapes, operand
layouts and alignments (host code only: no kernel is launched, and the
operand addresses are only looked at for their alignment).

Invariants, for every problem the planner accepts:
  * the config belongs to the dtype's table and the kind matches it;
  * the few-row kernel is chosen only for M <= 64 with both operands
    K-contiguous;
  * K is split only for tiled launches with few output tiles, into at most
    16 slices of at least 4 stages each, every slice non-empty, and the
    workspace is exactly one fp32 M x N plane per slice;
  * forgeml_hip_gemm_workspace_size is an upper bound over layouts;
  * planning with the chosen config id again gives the same plan.
"""

import ctypes

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from forgeml_amd import _native, kernels

DTYPES = [(_native.DTYPE_F32, 4), (_native.DTYPE_BF16, 2), (_native.DTYPE_F16, 2)]
MAX_SPLIT = 16
MIN_SLICE_STAGES = 4
STAGE_BYTES = 128  # bytes of K per pipeline stage


@st.composite
def problems(draw):
    m = draw(st.integers(1, 3000))
    n = draw(st.integers(1, 3000))
    k = draw(st.integers(1, 12000))
    dtype, esz = draw(st.sampled_from(DTYPES))
    pad = draw(st.integers(0, 9))
    a_layout = draw(st.sampled_from(["row", "col", "strided"]))
    b_layout = draw(st.sampled_from(["wt", "kn", "strided"]))
    if a_layout == "row":
        sam, sak = k + pad, 1
    elif a_layout == "col":
        sam, sak = 1, m + pad
    else:
        sam, sak = 2 * (k + pad), 2
    if b_layout == "wt":  # W^T view of an nn.Linear weight [N, K]
        sbk, sbn = 1, k + pad
    elif b_layout == "kn":
        sbk, sbn = n + pad, 1
    else:
        sbk, sbn = 2, 2 * (k + pad)
    # Base addresses: 256-byte aligned plus a whole number of elements.
    a_addr = 4096 + esz * draw(st.integers(0, 7))
    b_addr = (1 << 20) + esz * draw(st.integers(0, 7))
    return m, n, k, dtype, esz, sam, sak, sbk, sbn, a_addr, b_addr


def _plan(lib, p, cid=-1):
    m, n, k, dtype, _, sam, sak, sbk, sbn, a_addr, b_addr = p
    out = (ctypes.c_int64 * 4)()
    rc = lib.forgeml_hip_gemm_plan(ctypes.c_void_p(a_addr), sam, sak, ctypes.c_void_p(b_addr), sbk, sbn,
                                   m, n, k, dtype, cid, out)
    return rc, tuple(out)


@pytest.fixture(scope="module")
def lib():
    return _native.load()


@settings(max_examples=400, deadline=None, derandomize=True, database=None)
@given(p=problems())
def test_plan_invariants(lib, p):
    m, n, k, dtype, esz, sam, sak, sbk, sbn, _, _ = p
    rc, (cid, splits, ws, kind) = _plan(lib, p)
    assert rc == _native.OK, _native.last_error()
    table = _native.config_table()
    assert 0 <= cid < len(table)
    dclass, bm, bn = table[cid][0], table[cid][1], table[cid][2]
    assert dclass == (0 if dtype == _native.DTYPE_F32 else 1)
    skinny = kernels.CANDIDATES[cid] in (kernels.SKINNY_FP32, kernels.SKINNY_H16)
    assert kind == (1 if skinny else 0)
    if kind == 1:
        assert m <= 64 and sak == 1 and sbk == 1
    nk = -(-k * esz // STAGE_BYTES)
    assert 1 <= splits <= MAX_SPLIT
    if splits > 1:
        tiles = -(-m // bm) * -(-n // bn)
        assert kind == 0 and tiles < 128
        assert splits <= nk // MIN_SLICE_STAGES
        slice_ = -(-nk // splits)
        assert (splits - 1) * slice_ < nk  # the last slice is not empty
        assert ws == splits * m * n * 4
    else:
        assert ws == 0
    assert ws <= lib.forgeml_hip_gemm_workspace_size(m, n, k, dtype, -1)
    # The chosen config, asked for explicitly, plans the same launch.
    assert _plan(lib, p, cid) == (rc, (cid, splits, ws, kind))


@settings(max_examples=300, deadline=None, derandomize=True, database=None)
@given(m=st.integers(1, 8192), n=st.integers(1, 8192), kv=st.integers(1, 2048),
       dt=st.sampled_from(DTYPES))
def test_select_config_matches_the_plan_for_aligned_k_contiguous_operands(lib, m, n, kv, dt):
    """forgeml_hip_select_config is what AUTO resolves to when both operands are
    K-contiguous with 16-byte aligned rows (include/forgeml_hip.h): K a whole
    number of 16-byte vectors."""
    dtype, esz = dt
    k = kv * (16 // esz)
    ld = k
    cid = lib.forgeml_hip_select_config(m, n, k, dtype)
    assert 0 <= cid < len(kernels.CANDIDATES)
    assert _native.config_table()[cid][0] == (0 if dtype == _native.DTYPE_F32 else 1)
    rc, (planned, _, _, _) = _plan(lib, (m, n, k, dtype, esz, ld, 1, 1, ld, 4096, 1 << 20))
    assert rc == _native.OK and planned == cid
    assert cid == lib.forgeml_hip_select_config(m, n, k, dtype)  # deterministic


def test_auto_plans_a_built_tile_for_every_layout(lib):
    """FORGEML_CONFIG_AUTO plans a config the launch accepts for every operand layout pair,
    every residue of M and K mod 8, row padding and base offset: the shape heuristic offers
    only tiles built for the operand combination the layout runs on them (a transposed A
    with 4-byte B rows steps down to element loads, which 16-bit tiles above 64x64 lack)."""
    failures = []
    for dtype, esz in DTYPES:
        for m, n in ((1584, 109), (1585, 1000), (1736, 2134), (2808, 1919)):
            for k in (1228, 1662, 4096, 4100, 4101):
                for pad in (0, 1, 2):
                    for a_layout in ("row", "col", "strided"):
                        for b_layout in ("wt", "kn", "strided"):
                            for a_off in (0, 1):
                                sam, sak = {"row": (k + pad, 1), "col": (1, m + pad), "strided": (2 * (k + pad), 2)}[a_layout]
                                sbk, sbn = {"wt": (1, k + pad), "kn": (n + pad, 1), "strided": (2, 2 * (k + pad))}[b_layout]
                                p = (m, n, k, dtype, esz, sam, sak, sbk, sbn, 4096 + esz * a_off, 1 << 20)
                                rc, (cid, _, _, _) = _plan(lib, p)
                                if rc != _native.OK:
                                    failures.append((p, _native.last_error()))
                                    continue
                                rc2, _ = _plan(lib, p, cid)  # the chosen config is accepted as such
                                if rc2 != _native.OK:
                                    failures.append((p, cid, _native.last_error()))
    assert not failures, failures[:5]
