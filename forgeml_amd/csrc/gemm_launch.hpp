// gemm_launch.hpp — host-side launch of one fused GEMM tile configuration.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

#include "gemm_kernels.hpp"

namespace forgeml {

// Operand-layout combinations a tile configuration is built for (A mode, B mode).
enum : int {
  COMBO_K_K = 0,   // A K-contiguous, B K-contiguous (B = W^T view of an nn.Linear weight)
  COMBO_K_MN = 1,  // A K-contiguous, B N-contiguous (B = contiguous [K,N])
  COMBO_MN_K = 2,
  COMBO_MN_MN = 3,
  COMBO_G_G = 4,   // any strides
  NUM_COMBOS = 5,
};

// Sets the thread-local error text; returns `code`.
int set_error(int code, const char* fmt, ...);

constexpr int kMaxDevices = 64;

template <int DT, int BM, int BN, int WM, int WN, int AMODE, int BMODE>
int launch_one(const GemmArgs& p, hipStream_t stream) {
  constexpr int NT = WM * WN * 64;
  constexpr int LDS = 2 * (BM + BN) * kRowBytes;
  const void* fn = reinterpret_cast<const void*>(&fused_gemm_kernel<DT, BM, BN, WM, WN, AMODE, BMODE>);
  if constexpr (LDS > 65536) {
    // Above 64 KiB the dynamic LDS limit must be raised once per device
    // (gfx950 has 160 KiB of LDS per CU).
    static std::atomic<int> ready[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
      return set_error(-3, "hipGetDevice failed or device index out of range");
    if (ready[dev].load(std::memory_order_acquire) == 0) {
      hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
      if (e != hipSuccess)
        return set_error(-3, "hipFuncSetAttribute(%d bytes LDS): %s", LDS, hipGetErrorString(e));
      ready[dev].store(1, std::memory_order_release);
    }
  }
  hipLaunchKernelGGL((fused_gemm_kernel<DT, BM, BN, WM, WN, AMODE, BMODE>),
                     dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(NT), LDS, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(-3, "kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

template <int DT, int BM, int BN, int WM, int WN>
int launch_tile(const GemmArgs& p, int combo, hipStream_t stream) {
  switch (combo) {
    case COMBO_K_K: return launch_one<DT, BM, BN, WM, WN, MODE_K, MODE_K>(p, stream);
    case COMBO_K_MN: return launch_one<DT, BM, BN, WM, WN, MODE_K, MODE_MN>(p, stream);
    case COMBO_MN_K: return launch_one<DT, BM, BN, WM, WN, MODE_MN, MODE_K>(p, stream);
    case COMBO_MN_MN: return launch_one<DT, BM, BN, WM, WN, MODE_MN, MODE_MN>(p, stream);
    default: return launch_one<DT, BM, BN, WM, WN, MODE_G, MODE_G>(p, stream);
  }
}

using TileLauncher = int (*)(const GemmArgs&, int, hipStream_t);

// Tile table, defined in fused_gemm_abi.hip.
struct TileConfig {
  int dclass;  // 0 = fp32, 1 = 16-bit
  int bm, bn, wm, wn;
  TileLauncher launch[3];  // indexed by DT_*; null where not built
};

}  // namespace forgeml
