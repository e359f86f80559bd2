// fused_gemm_f32.hip — instantiates the f32 fused GEMM kernels of every tile
// configuration and the few-row kernels (one translation unit per dtype so they build in parallel).
#include "gemm_launch.hpp"
#include "tile_table.hpp"

namespace forgeml {
#define FORGEML_INSTANTIATE(bm, bn, wm, wn, ...) \
  template int launch_tile<DT_F32, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t);
FORGEML_F32_TILES(FORGEML_INSTANTIATE)
#undef FORGEML_INSTANTIATE
template int launch_skinny<DT_F32>(const GemmArgs&, int, hipStream_t);
}  // namespace forgeml
