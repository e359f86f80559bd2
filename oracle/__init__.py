"""Oracle for the fused linear path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed
CPU baseline.  The product (``forgeml_amd``) never calls it: GPU GEMMs run
on the gfx950 kernels or raise.

Contents:

* ``fused_linear.reference_cpu`` — ForgeML's own CPU path for a
  linear / fused_linear_gelu node: ``torch.addmm`` (or ``torch.mm``) on the
  CPU followed by ``F.gelu`` (src/forgeml/ops.py:28-31, 48-53;
  src/forgeml/compiler.py:115-126).  This is what parity is judged against.
* ``fused_linear.kernel_contract`` — the rounding contract of the reference
  kernel's epilogue (src/forgeml/_triton.py:43-57), with fp64 accumulation.
* ``fused_linear.brute_force`` — fp64 triple loop in plain C
  (``gemm_ref.c``), an implementation independent of torch used to pin the
  two functions above.
* ``fused_linear.tolerance`` — the gate's rtol/atol per dtype and K.

ForgeML is pure Python with no C/C++ sources, so there is nothing to build
into ``oracle/_ref``; its arithmetic lives in torch (CPU) and Triton (never
run on hardware), and is pinned here by known values, closed forms, fp64
brute force and the reference tests' own expected-value formulas.
"""
