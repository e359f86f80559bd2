// gemm_launch.hpp — host-side launch of one fused GEMM tile configuration.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

#include "gemm_kernels.hpp"
#include "skinny_kernels.hpp"

namespace forgeml {

// Operand-layout combinations a tile configuration is built for (A mode, B mode).
enum : int {
  COMBO_K_K = 0,   // A K-contiguous, B K-contiguous (B = W^T view of an nn.Linear weight)
  COMBO_K_MN = 1,  // A K-contiguous, B N-contiguous (B = contiguous [K,N])
  COMBO_MN_K = 2,
  COMBO_MN_MN = 3,
  COMBO_G_G = 4,   // any strides
  // Built for tiles of at most 128x128 (kSmallTileArea); larger tiles use G_G.
  COMBO_K4_K4 = 5,  // both K-contiguous with rows only 4-byte aligned (odd fp32 K)
  COMBO_K4_MN = 6,  // A as above, B N-contiguous
  COMBO_G_MN = 7,   // A any strides (e.g. an odd 16-bit K), B N-contiguous
  NUM_COMBOS = 8,
};

constexpr int kSmallTileArea = 128 * 128;

// Whether a tile is built for an operand combination.  16-bit element loads
// (COMBO_G_*) stage 32 packed values per thread, and tiles above 64x64 then
// run out of registers beside their accumulators and spill to scratch; the
// 8-wave 16-bit tile's budget fits only the DMA loaders of two K-contiguous
// operands, and the 8-wave fp32 tile's everything but element loads of both
// operands.  Those pairs are not built, and the planner refuses a request
// for one; the shape heuristic never chooses them.
constexpr bool combo_supported(int dclass, int bm, int bn, int waves, int combo) {
  if (dclass == 1 && waves > 4 && combo != COMBO_K_K) return false;
  if (dclass == 0 && waves > 4 && combo == COMBO_G_G) return false;
  if (dclass == 1 && bm * bn > 64 * 64 && (combo == COMBO_G_G || combo == COMBO_G_MN)) return false;
  return true;
}

// Sets the thread-local error text; returns `code`.
int set_error(int code, const char* fmt, ...);

constexpr int kMaxDevices = 64;

// The split-K epilogue kernel over the workspace planes of one GEMM.
template <int DT>
int launch_reduce(const GemmArgs& p, hipStream_t stream) {
  ReduceArgs r;
  r.ws = p.ws;
  r.bias = p.bias;
  r.c = p.c;
  r.sbi = p.sbi;
  r.res = p.res;
  r.srm = p.srm;
  r.srn = p.srn;
  r.mn = (int64_t)p.m * p.n;
  r.n = p.n;
  r.splits = p.splits;
  r.has_bias = p.has_bias;
  r.vec = r.mn % 4 == 0 && ((uintptr_t)p.ws & 15) == 0 && ((uintptr_t)p.c & 15) == 0;
  const dim3 grid((unsigned)((r.mn + 1023) / 1024)), block(256);
  switch (p.act) {
    case ACT_GELU_ERF: hipLaunchKernelGGL((splitk_reduce_kernel<DT, ACT_GELU_ERF>), grid, block, 0, stream, r); break;
    case ACT_GELU_TANH: hipLaunchKernelGGL((splitk_reduce_kernel<DT, ACT_GELU_TANH>), grid, block, 0, stream, r); break;
    case ACT_RELU: hipLaunchKernelGGL((splitk_reduce_kernel<DT, ACT_RELU>), grid, block, 0, stream, r); break;
    default: hipLaunchKernelGGL((splitk_reduce_kernel<DT, ACT_NONE>), grid, block, 0, stream, r); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(-3, "split-K reduce launch failed: %s", hipGetErrorString(e));
  return 0;
}

template <int DT, int BM, int BN, int WM, int WN, int AMODE, int BMODE, int S>
int launch_ring(const GemmArgs& p, hipStream_t stream) {
  constexpr int NT = WM * WN * 64;
  constexpr int LDS = S * (BM + BN) * kRowBytes + (gelu_lut_tile<DT, BM, BN, WM * WN>() ? kLutBytes : 0);
  const void* fn = reinterpret_cast<const void*>(&fused_gemm_kernel<DT, BM, BN, WM, WN, AMODE, BMODE, S>);
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
  hipLaunchKernelGGL((fused_gemm_kernel<DT, BM, BN, WM, WN, AMODE, BMODE, S>),
                     dim3((unsigned)(p.tiles_m * p.tiles_n * p.splits)), dim3(NT), LDS, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(-3, "kernel launch failed: %s", hipGetErrorString(e));
  return p.splits > 1 ? launch_reduce<DT>(p, stream) : 0;
}

// A tile that may ring through four LDS stages does so while the grid holds
// at most two workgroups per CU (MI355X: 256 CUs): then latency within a
// workgroup is what limits it.  Larger grids take two stages (32 KiB for a
// 64x64 tile), so up to five workgroups share a CU and hide each other's
// prologue and epilogue.  Measured 64x64 (us, four stages -> two): fp32
// 4096x2304x768 124.0 -> 114.9, 4096x768x3072 160.1 -> 148.4, bf16
// 1000x3072x1024 17.2 -> 14.0; bf16 512x4096x4096 (512 workgroups) 27.8 ->
// 33.1, 1024^3 (256) 7.9 -> 8.1.
constexpr int64_t kDeepRingMaxWgs = 2 * 256;

template <int DT, int BM, int BN, int WM, int WN, int AMODE, int BMODE>
int launch_one(const GemmArgs& p, hipStream_t stream) {
  constexpr int SMAX = lds_stages_max<BM, BN, AMODE, BMODE>();
  if constexpr (SMAX > 2) {
    if ((int64_t)p.tiles_m * p.tiles_n * p.splits <= kDeepRingMaxWgs)
      return launch_ring<DT, BM, BN, WM, WN, AMODE, BMODE, SMAX>(p, stream);
  }
  return launch_ring<DT, BM, BN, WM, WN, AMODE, BMODE, 2>(p, stream);
}

// One combination of a tile, or an error when the tile is not built for it
// (the planner refuses those requests first).
template <int DT, int BM, int BN, int WM, int WN, int COMBO, int AMODE, int BMODE>
int launch_combo(const GemmArgs& p, hipStream_t stream) {
  if constexpr (!combo_supported(DT == DT_F32 ? 0 : 1, BM, BN, WM * WN, COMBO))
    return set_error(-2, "tile %dx%d (%d waves) is not built for operand combination %d", BM, BN, WM * WN, COMBO);
  else
    return launch_one<DT, BM, BN, WM, WN, AMODE, BMODE>(p, stream);
}

template <int DT, int BM, int BN, int WM, int WN>
int launch_tile(const GemmArgs& p, int combo, hipStream_t stream) {
  if constexpr (BM * BN <= kSmallTileArea) {
    switch (combo) {
      case COMBO_K4_K4: return launch_combo<DT, BM, BN, WM, WN, COMBO_K4_K4, MODE_K4, MODE_K4>(p, stream);
      case COMBO_K4_MN: return launch_combo<DT, BM, BN, WM, WN, COMBO_K4_MN, MODE_K4, MODE_MN>(p, stream);
      case COMBO_G_MN: return launch_combo<DT, BM, BN, WM, WN, COMBO_G_MN, MODE_G, MODE_MN>(p, stream);
      default: break;
    }
  }
  switch (combo) {
    case COMBO_K_K: return launch_combo<DT, BM, BN, WM, WN, COMBO_K_K, MODE_K, MODE_K>(p, stream);
    case COMBO_K_MN: return launch_combo<DT, BM, BN, WM, WN, COMBO_K_MN, MODE_K, MODE_MN>(p, stream);
    case COMBO_MN_K: return launch_combo<DT, BM, BN, WM, WN, COMBO_MN_K, MODE_MN, MODE_K>(p, stream);
    case COMBO_MN_MN: return launch_combo<DT, BM, BN, WM, WN, COMBO_MN_MN, MODE_MN, MODE_MN>(p, stream);
    default: return launch_combo<DT, BM, BN, WM, WN, COMBO_G_G, MODE_G, MODE_G>(p, stream);
  }
}

// Few-row kernel: TM 16-row blocks per workgroup, `lw` the load width in
// bytes (16, 4 or 2) both operands' alignment allows.  All ceil(M/16) row
// blocks in one workgroup read each weight byte once; while the grid would
// cover at most half the CUs, the row blocks are split over workgroups
// instead (each re-reads its column group's weights, then from L2).
// Measured: 64x512x2048 21.6 -> 9.6 us, 64x2048x512 8.7 -> 5.8 us (fp32);
// splitting a grid of 192 column groups lost 9-24 %.
constexpr int64_t kSkinnySplitMaxWgs = 128;

// Chunks in flight per few-row wave: 2 while a wave's share of K is at most
// 6 chunks, else kSkinnyDepth.  Measured (bf16 1x3000x1531, 6 chunks per
// wave) 5.6 us at 2 against 6.2 at 4; fp32 (12 chunks) 7.8 at 4 against 8.6.
inline int skinny_depth(int64_t k, int esz) {
  const int64_t chunks = (k + 64 / esz - 1) / (64 / esz);
  return (chunks + kSkinnyWaves - 1) / kSkinnyWaves <= 6 ? 2 : kSkinnyDepth;
}

template <int DT, int TM, int LW>
int launch_skinny_one(const GemmArgs& p, hipStream_t stream) {
  const unsigned gx = (unsigned)((p.n + 15) / 16), gy = (unsigned)((p.m + 16 * TM - 1) / (16 * TM));
  if (skinny_depth(p.k, DTraits<DT>::ESZ) == 2)
    hipLaunchKernelGGL((skinny_gemm_kernel<DT, TM, LW, 2>), dim3(gx, gy), dim3(kSkinnyWaves * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<DT, TM, LW, kSkinnyDepth>), dim3(gx, gy), dim3(kSkinnyWaves * 64), 0, stream,
                       p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(-3, "kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

template <int DT, int LW>
int launch_skinny_lw(const GemmArgs& p, hipStream_t stream) {
  const int col_groups = (p.n + 15) / 16;
  int tm = (p.m + 15) / 16;
  while (tm > 1 && (int64_t)col_groups * ((((p.m + 15) / 16) + tm - 1) / tm) <= kSkinnySplitMaxWgs) tm = (tm + 1) / 2;
  switch (tm) {
    case 1: return launch_skinny_one<DT, 1, LW>(p, stream);
    case 2: return launch_skinny_one<DT, 2, LW>(p, stream);
    case 3: return launch_skinny_one<DT, 3, LW>(p, stream);
    default: return launch_skinny_one<DT, 4, LW>(p, stream);
  }
}

template <int DT>
int launch_skinny(const GemmArgs& p, int lw, hipStream_t stream) {
  if (lw == 16) return launch_skinny_lw<DT, 16>(p, stream);
  if constexpr (DT != DT_F32) {
    if (lw == 2) return launch_skinny_lw<DT, 2>(p, stream);
  }
  return launch_skinny_lw<DT, 4>(p, stream);
}

using TileLauncher = int (*)(const GemmArgs&, int, hipStream_t);

enum : int { KIND_TILED = 0, KIND_SKINNY = 1 };

// Tile table, defined in fused_gemm_abi.hip.
struct TileConfig {
  int dclass;  // 0 = fp32, 1 = 16-bit
  int bm, bn, wm, wn;
  int kind;    // KIND_TILED, or KIND_SKINNY (bm = most rows, bn = columns per workgroup)
  TileLauncher launch[3];  // indexed by DT_*; null where not built
  int occ, eff, solo_eff;  // shape-heuristic constants (see tile_table.hpp)
};

}  // namespace forgeml
