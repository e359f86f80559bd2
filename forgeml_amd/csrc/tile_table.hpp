// tile_table.hpp — the MI355X tile configurations this library is built with.
//
// X(block_m, block_n, waves_m, waves_n).  fp32 stages are 32 K elements and
// 16-bit stages 64 K elements (128 bytes per LDS row either way).  Config ids
// number the fp32 list first, then the 16-bit list; the Python KernelConfig
// table (forgeml_amd/kernels.py) lists them in the same order.
#pragma once

#define FORGEML_F32_TILES(X) \
  X(128, 128, 2, 2)          \
  X(64, 64, 2, 2)            \
  X(256, 128, 4, 2)

#define FORGEML_H16_TILES(X) \
  X(256, 256, 2, 2)          \
  X(128, 128, 2, 2)          \
  X(64, 64, 2, 2)            \
  X(256, 256, 2, 4)
