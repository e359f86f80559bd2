// fused_gemm_bf16.hip — instantiates the bf16 fused GEMM kernels of every tile
// configuration and the few-row kernels (one translation unit per dtype so they build in parallel).
#include "gemm_launch.hpp"
#include "tile_table.hpp"

namespace forgeml {
#define FORGEML_INSTANTIATE(bm, bn, wm, wn, ...) \
  template int launch_tile<DT_BF16, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t);
FORGEML_H16_TILES(FORGEML_INSTANTIATE)
#undef FORGEML_INSTANTIATE
template int launch_skinny<DT_BF16>(const GemmArgs&, int, hipStream_t);
}  // namespace forgeml
