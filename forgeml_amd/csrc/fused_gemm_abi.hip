// fused_gemm_abi.hip — the extern "C" entry points declared in include/forgeml_hip.h.
//
// Argument validation mirrors what ForgeML's Python boundary checks before a
// launch (src/forgeml/kernels.py:62-112); the Python host side checks the same
// things first and raises GraphError, so a failure here means a caller that
// bypassed it.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "forgeml_hip.h"
#include "gemm_launch.hpp"
#include "tile_table.hpp"

namespace forgeml {

#define FORGEML_EXTERN_F32(bm, bn, wm, wn) \
  extern template int launch_tile<DT_F32, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t);
#define FORGEML_EXTERN_H16(bm, bn, wm, wn)                                                      \
  extern template int launch_tile<DT_BF16, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t); \
  extern template int launch_tile<DT_F16, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t);
FORGEML_F32_TILES(FORGEML_EXTERN_F32)
FORGEML_H16_TILES(FORGEML_EXTERN_H16)
#undef FORGEML_EXTERN_F32
#undef FORGEML_EXTERN_H16

static thread_local char g_last_error[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

static const TileConfig kTiles[] = {
#define FORGEML_ROW_F32(bm, bn, wm, wn) \
  {0, bm, bn, wm, wn, {&launch_tile<DT_F32, bm, bn, wm, wn>, nullptr, nullptr}},
#define FORGEML_ROW_H16(bm, bn, wm, wn) \
  {1, bm, bn, wm, wn, {nullptr, &launch_tile<DT_BF16, bm, bn, wm, wn>, &launch_tile<DT_F16, bm, bn, wm, wn>}},
    FORGEML_F32_TILES(FORGEML_ROW_F32) FORGEML_H16_TILES(FORGEML_ROW_H16)
#undef FORGEML_ROW_F32
#undef FORGEML_ROW_H16
};
static constexpr int kNumTiles = (int)(sizeof(kTiles) / sizeof(kTiles[0]));

static int esize_of(int dtype) { return dtype == FORGEML_DTYPE_F32 ? 4 : 2; }
static int dclass_of(int dtype) { return dtype == FORGEML_DTYPE_F32 ? 0 : 1; }

// Load mode of one operand viewed as rows x K with strides (s_mn, s_k).
// The vector modes address one workgroup's operand panel with 32-bit buffer
// offsets: rows of the widest tile (256) for K-contiguous operands, all of K
// for M/N-contiguous ones.
static constexpr int64_t kMaxPanelRows = 256;
static constexpr int64_t kMaxBufferBytes = (int64_t)1 << 31;

static int operand_mode(const void* base, int64_t rows, int64_t s_mn, int64_t s_k, int64_t k, int esz) {
  const int vec = 16 / esz;
  const bool aligned = ((uintptr_t)base % 16) == 0;
  if (aligned && s_k == 1 && s_mn >= 0 && (s_mn * esz) % 16 == 0 && k % vec == 0 &&
      (kMaxPanelRows * s_mn + k) * esz < kMaxBufferBytes)
    return MODE_K;
  if (aligned && s_mn == 1 && s_k >= 0 && (s_k * esz) % 16 == 0 && rows % vec == 0 &&
      (k * s_k + kMaxPanelRows) * esz < kMaxBufferBytes)
    return MODE_MN;
  return MODE_G;
}

static int combo_of(int ma, int mb) {
  if (ma == MODE_G || mb == MODE_G) return COMBO_G_G;
  if (ma == MODE_K) return mb == MODE_K ? COMBO_K_K : COMBO_K_MN;
  return mb == MODE_K ? COMBO_MN_K : COMBO_MN_MN;
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Shape heuristic behind FORGEML_CONFIG_AUTO: the largest tile that still
// gives every one of the 256 CUs at least one workgroup (the smallest tile
// otherwise).  Among equal areas, more waves per workgroup win (two waves
// per SIMD hide each other's stalls), but only where both operands are
// K-contiguous: the 8-wave tile's register budget does not fit the
// transposing loaders.
static int select_config(int64_t m, int64_t n, int64_t /*k*/, int dtype, int combo) {
  const int dclass = dclass_of(dtype);
  int best = -1, smallest = -1;
  int64_t best_area = -1, smallest_area = INT64_MAX;
  int best_waves = 0;
  for (int id = 0; id < kNumTiles; ++id) {
    const TileConfig& t = kTiles[id];
    if (t.dclass != dclass) continue;
    const int waves = t.wm * t.wn;
    if (waves > 4 && dclass == 1 && combo != COMBO_K_K) continue;
    const int64_t area = (int64_t)t.bm * t.bn;
    if (area < smallest_area) {
      smallest_area = area;
      smallest = id;
    }
    const int64_t tiles = cdiv(m, t.bm) * cdiv(n, t.bn);
    if (tiles >= 256 && (area > best_area || (area == best_area && waves > best_waves))) {
      best_area = area;
      best_waves = waves;
      best = id;
    }
  }
  return best >= 0 ? best : smallest;
}

}  // namespace forgeml

using namespace forgeml;

extern "C" {

int forgeml_hip_abi_version(void) { return FORGEML_HIP_ABI_VERSION; }

const char* forgeml_hip_last_error(void) { return g_last_error; }

int forgeml_hip_num_configs(void) { return kNumTiles; }

int forgeml_hip_config_info(int32_t id, int32_t* out) {
  if (out == nullptr) return set_error(FORGEML_EINVAL, "config_info: out is NULL");
  if (id < 0 || id >= kNumTiles) return set_error(FORGEML_ECONFIG, "config id %d out of range [0, %d)", id, kNumTiles);
  const TileConfig& t = kTiles[id];
  out[0] = t.dclass;
  out[1] = t.bm;
  out[2] = t.bn;
  out[3] = t.dclass == 0 ? kRowBytes / 4 : kRowBytes / 2;
  out[4] = t.wm * t.wn;
  out[5] = 2;
  out[6] = 1;
  out[7] = 2 * (t.bm + t.bn) * kRowBytes;
  return FORGEML_OK;
}

int forgeml_hip_select_config(int64_t m, int64_t n, int64_t k, int32_t dtype) {
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  if (m <= 0 || n <= 0 || k <= 0) return set_error(FORGEML_EINVAL, "select_config: M, N, K must be positive");
  return select_config(m, n, k, dtype, COMBO_K_K);
}

int64_t forgeml_hip_gemm_workspace_size(int64_t m, int64_t n, int64_t k, int32_t dtype, int32_t config_id) {
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  if (m <= 0 || n <= 0 || k <= 0) return set_error(FORGEML_EINVAL, "workspace_size: M, N, K must be positive");
  if (config_id != FORGEML_CONFIG_AUTO && (config_id < 0 || config_id >= kNumTiles))
    return set_error(FORGEML_ECONFIG, "config id %d out of range", config_id);
  return 0;
}

int forgeml_hip_gemm(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn,
                     const void* bias, int64_t sbi, void* c, int64_t m, int64_t n, int64_t k, int32_t dtype,
                     int32_t act, int32_t config_id, void* workspace, int64_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  g_last_error[0] = '\0';
  if (a == nullptr || b == nullptr || c == nullptr) return set_error(FORGEML_EINVAL, "a, b and c must be non-NULL");
  if (m <= 0 || n <= 0 || k <= 0) return set_error(FORGEML_EINVAL, "M, N, K must be positive (got %lld, %lld, %lld)",
                                                   (long long)m, (long long)n, (long long)k);
  if (m > INT_MAX || n > INT_MAX || k > INT_MAX || m * n > (int64_t)INT_MAX * 64)
    return set_error(FORGEML_EINVAL, "shape too large for this kernel family");
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  if (act < FORGEML_ACT_NONE || act > FORGEML_ACT_RELU) return set_error(FORGEML_EINVAL, "unknown activation %d", act);
  if (sam < 0 || sak < 0 || sbk < 0 || sbn < 0 || sbi < 0) return set_error(FORGEML_EINVAL, "negative strides are not supported");

  if (config_id != FORGEML_CONFIG_AUTO && (config_id < 0 || config_id >= kNumTiles))
    return set_error(FORGEML_ECONFIG, "config id %d out of range [0, %d)", config_id, kNumTiles);

  const int esz = esize_of(dtype);
  // A size-1 dimension has no meaningful stride; zero it so layout detection
  // looks only at the dimensions that are walked.
  if (m == 1) sam = 0;
  if (n == 1) sbn = 0;
  if (k == 1) {
    sak = 0;
    sbk = 0;
  }
  const int ma = operand_mode(a, m, sam, sak, k, esz);
  const int mb = operand_mode(b, n, sbn, sbk, k, esz);
  const int combo = combo_of(ma, mb);
  if (config_id == FORGEML_CONFIG_AUTO) config_id = select_config(m, n, k, dtype, combo);
  const TileConfig& t = kTiles[config_id];
  if (t.dclass != dclass_of(dtype) || t.launch[dtype] == nullptr)
    return set_error(FORGEML_ECONFIG, "config %d is not built for dtype %d", config_id, dtype);

  GemmArgs p;
  p.a = (const char*)a;
  p.b = (const char*)b;
  p.bias = (const char*)bias;
  p.c = (char*)c;
  p.sam = sam;
  p.sak = sak;
  p.sbk = sbk;
  p.sbn = sbn;
  p.sbi = sbi;
  p.m = (int)m;
  p.n = (int)n;
  p.k = (int)k;
  p.act = act;
  p.has_bias = bias != nullptr;
  p.tiles_m = (int)cdiv(m, t.bm);
  p.tiles_n = (int)cdiv(n, t.bn);
  p.group_m = p.tiles_m < 8 ? p.tiles_m : 8;
  if ((int64_t)p.tiles_m * p.tiles_n > INT_MAX) return set_error(FORGEML_EINVAL, "too many output tiles");
  return t.launch[dtype](p, combo, (hipStream_t)stream);
}

}  // extern "C"
