// tile_table.hpp — the MI355X tile configurations this library is built with.
//
// Tiles are listed as X(...) below.  fp32 stages are 32 K elements and
// 16-bit stages 64 K elements (128 bytes per LDS row either way).  Config ids
// number the fp32 list first, then the 16-bit list; the Python KernelConfig
// table (forgeml_amd/kernels.py) lists them in the same order.
#pragma once

// X(block_m, block_n, waves_m, waves_n, occ, eff, solo_eff): besides the
// shape, the shape heuristic's cost model uses the workgroups that share a
// CU (occ), the tile's relative throughput when the CU holds that many (eff,
// percent) and when it holds only one (solo_eff).  The efficiencies are
// fitted to measured times of every tile over square and rectangular shapes
// with K = 768..4096 on MI355X (K-contiguous operands).
#define FORGEML_F32_TILES(X)       \
  X(128, 128, 2, 2, 2, 100, 88)    \
  X(64, 64, 2, 2, 2, 90, 90)       \
  X(256, 256, 2, 4, 1, 100, 100)

#define FORGEML_H16_TILES(X)       \
  X(256, 256, 2, 2, 1, 91, 91)     \
  X(128, 128, 2, 2, 2, 87, 80)     \
  X(64, 64, 2, 2, 2, 62, 62)       \
  X(256, 256, 2, 4, 1, 100, 100)
