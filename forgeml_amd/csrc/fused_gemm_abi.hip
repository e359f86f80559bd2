// fused_gemm_abi.hip — the extern "C" entry points declared in include/forgeml_hip.h.
//
// Argument validation mirrors what ForgeML's Python boundary checks before a
// launch (src/forgeml/kernels.py:62-112); the Python host side checks the same
// things first and raises GraphError, so a failure here means a caller that
// bypassed it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>

#include "forgeml_hip.h"
#include "gemm_launch.hpp"
#include "tile_table.hpp"

namespace forgeml {

#define FORGEML_EXTERN_F32(bm, bn, wm, wn, ...) \
  extern template int launch_tile<DT_F32, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t);
#define FORGEML_EXTERN_H16(bm, bn, wm, wn, ...)                                                 \
  extern template int launch_tile<DT_BF16, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t); \
  extern template int launch_tile<DT_F16, bm, bn, wm, wn>(const GemmArgs&, int, hipStream_t);
FORGEML_F32_TILES(FORGEML_EXTERN_F32)
FORGEML_H16_TILES(FORGEML_EXTERN_H16)
extern template int launch_skinny<DT_F32>(const GemmArgs&, int, hipStream_t);
extern template int launch_skinny<DT_BF16>(const GemmArgs&, int, hipStream_t);
extern template int launch_skinny<DT_F16>(const GemmArgs&, int, hipStream_t);
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
#define FORGEML_ROW_F32(bm, bn, wm, wn, occ, eff, solo) \
  {0, bm, bn, wm, wn, KIND_TILED, {&launch_tile<DT_F32, bm, bn, wm, wn>, nullptr, nullptr}, occ, eff, solo},
#define FORGEML_ROW_H16(bm, bn, wm, wn, occ, eff, solo)                                                            \
  {1, bm, bn, wm, wn, KIND_TILED, {nullptr, &launch_tile<DT_BF16, bm, bn, wm, wn>, &launch_tile<DT_F16, bm, bn, wm, wn>}, \
   occ, eff, solo},
    FORGEML_F32_TILES(FORGEML_ROW_F32) FORGEML_H16_TILES(FORGEML_ROW_H16)
#undef FORGEML_ROW_F32
#undef FORGEML_ROW_H16
    // Few-row kernels (M <= 64, K-contiguous operands), last so the tiled ids stay put.
    {0, kSkinnyMaxRows, 16, 1, kSkinnyWaves, KIND_SKINNY, {&launch_skinny<DT_F32>, nullptr, nullptr}, 1, 100, 100},
    {1, kSkinnyMaxRows, 16, 1, kSkinnyWaves, KIND_SKINNY, {nullptr, &launch_skinny<DT_BF16>, &launch_skinny<DT_F16>}, 1, 100,
     100},
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
  const uintptr_t addr = (uintptr_t)base;
  // Room for the pipeline's reads one or two stages past K (out of range).
  const bool k_fits = s_k == 1 && s_mn >= 0 && s_mn < kMaxBufferBytes &&
                      (kMaxPanelRows * s_mn + k) * esz + 2 * kRowBytes < kMaxBufferBytes;
  const bool mn_fits = s_mn == 1 && s_k >= 0 && s_k < kMaxBufferBytes && (k * s_k + kMaxPanelRows) * esz < kMaxBufferBytes;
  if (addr % 16 == 0 && k_fits && (s_mn * esz) % 16 == 0 && k % vec == 0) return MODE_K;
  if (addr % 16 == 0 && mn_fits && (s_k * esz) % 16 == 0 && rows % vec == 0) return MODE_MN;
  if (addr % 4 == 0 && k_fits && (s_mn * esz) % 4 == 0 && (k * esz) % 4 == 0) return MODE_K4;
  return MODE_G;
}

// The built combination for an operand pair.  A 16-byte K-contiguous operand
// also meets the 4-byte mode's conditions and any operand can be read by
// element loads, so pairs without a kernel of their own step down to one that
// has.  `small_tile` says whether the tile (<= 128x128) has the extra combos.
static int combo_of(int ma, int mb, bool small_tile) {
  const bool a_k = ma == MODE_K, b_k = mb == MODE_K;
  const bool a_kk = a_k || ma == MODE_K4, b_kk = b_k || mb == MODE_K4;
  if (a_k && b_k) return COMBO_K_K;
  if (a_k && mb == MODE_MN) return COMBO_K_MN;
  if (ma == MODE_MN && b_k) return COMBO_MN_K;
  if (ma == MODE_MN && mb == MODE_MN) return COMBO_MN_MN;
  if (small_tile) {
    if (a_kk && b_kk) return COMBO_K4_K4;
    if (ma == MODE_K4 && mb == MODE_MN) return COMBO_K4_MN;
    if (mb == MODE_MN) return COMBO_G_MN;
  }
  return COMBO_G_G;
}

static bool needs_small_tile(int ma, int mb) {
  return combo_of(ma, mb, true) != combo_of(ma, mb, false);
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Work-items of one launch of tile t (a dispatch covers fewer than 2^32);
// the few-row kernel is bounded by one workgroup per 16 columns and 16 rows.
static constexpr int64_t kMaxItems = (int64_t)1 << 32;
static int64_t launch_items(const TileConfig& t, int64_t m, int64_t n, int64_t splits) {
  if (t.kind == KIND_SKINNY) return cdiv(n, 16) * cdiv(m, 16) * kSkinnyWaves * 64;
  return cdiv(m, t.bm) * cdiv(n, t.bn) * splits * (t.wm * t.wn * 64);
}

// Load width (bytes) of the few-row kernel for these operands, or 0 when it
// cannot run them: it needs M <= 64, both operands K-contiguous, and 32-bit
// byte offsets over A and over 16 rows of B.
static int skinny_width(int64_t m, int64_t k, int64_t sam, int64_t sak, int64_t sbn, int64_t sbk, int ma, int mb,
                        int esz) {
  if (m > kSkinnyMaxRows || sak != 1 || sbk != 1 || sam < 0 || sbn < 0 || sam >= kMaxBufferBytes ||
      sbn >= kMaxBufferBytes)
    return 0;
  // (+32: rows under 16-byte alignment round each operand's range out to 16-byte blocks)
  if (((m - 1) * sam + k) * esz + 32 >= kMaxBufferBytes || (15 * sbn + k) * esz + 32 >= kMaxBufferBytes) return 0;
  if (ma == MODE_K && mb == MODE_K) return 16;
  if ((ma == MODE_K || ma == MODE_K4) && (mb == MODE_K || mb == MODE_K4)) return 4;
  return esz == 2 ? 2 : 0;
}

// Whether the shape heuristic prefers the few-row kernel (it runs whenever
// skinny_width allows, if asked for by config id).  Its 8 waves per
// workgroup stream K in chunks of 64 bytes per row, and every workgroup (16
// columns) reads all of A.  Measured against the best tiled candidate with
// split K (HIP graph, weights cold): it wins on every shape with up to 48 rows
// and up to 24 chunks per wave, e.g. fp32 1x3000x4096 13.4 us against 29.3,
// fp32 17x3000x3000 19.7 against 24.6, fp32 33x3000x1531 16.9 against 21.9,
// as long as there are enough column groups to spread over the GPU; at 64 rows
// only up to 8 chunks per wave (fp32 64x3000x2048: 25.2 against 23.2).  Long
// K over few columns goes to the tiled kernels, whose split K uses every CU.
static bool skinny_preferred(int64_t m, int64_t n, int64_t k, int lw, int esz) {
  if (lw == 0) return false;
  const int64_t per_wave = cdiv(cdiv(k, 64 / esz), kSkinnyWaves);  // chunks each wave streams
  const int64_t groups = cdiv(n, 16);
  if (m <= 16) return per_wave <= 12 || (per_wave <= 32 && groups >= 64);
  if (m <= 48) return per_wave <= 24 && groups >= 48;
  return per_wave <= 8 && groups >= 48;
}

static int skinny_id(int dclass) {
  for (int id = 0; id < kNumTiles; ++id)
    if (kTiles[id].kind == KIND_SKINNY && kTiles[id].dclass == dclass) return id;
  return -1;
}

// K split for a grid of few output tiles: enough workgroups for two per CU,
// slices of at least kMinSliceStages stages, at most kMaxSplit slices.
static constexpr int64_t kSplitBelowTiles = 128;
static constexpr int64_t kSplitTargetWgs = 512;
static constexpr int64_t kMinSliceStages = 4;
static constexpr int64_t kMaxSplit = kMaxSplitK;

struct SplitPlan {
  int splits;  // 1 = no split
  int kslice;  // stages per slice
};

static SplitPlan split_plan(const TileConfig& t, int64_t m, int64_t n, int64_t k, int esz) {
  const int64_t tiles = cdiv(m, t.bm) * cdiv(n, t.bn);
  const int64_t nk = cdiv(k * esz, kRowBytes);
  SplitPlan plan{1, (int)nk};
  if (t.kind != KIND_TILED || tiles >= kSplitBelowTiles) return plan;
  int64_t s = cdiv(kSplitTargetWgs, tiles);
  s = std::min(s, nk / kMinSliceStages);
  s = std::min(s, kMaxSplit);
  if (s < 2) return plan;
  const int64_t slice = cdiv(nk, s);
  plan.kslice = (int)slice;
  plan.splits = (int)cdiv(nk, slice);  // every slice non-empty
  return plan;
}

static int64_t workspace_bytes_for(const SplitPlan& plan, int64_t m, int64_t n) {
  return plan.splits > 1 ? (int64_t)plan.splits * m * n * (int64_t)sizeof(float) : 0;
}

// Relative time of a tiled launch, for the shape heuristic.  Workgroups
// (tiles x K slices) are dealt to the 256 CUs; the busiest CU's share times
// one workgroup's work (its area times its K slice plus a fixed 8 stages of
// prologue and epilogue), divided by the tile's efficiency (the solo value
// when that CU holds fewer workgroups than the tile's occupancy), plus the
// split planes' traffic.  Fitted to measured times of every tile on MI355X;
// it picks the fastest tile or one within a few per cent of it.
static constexpr int64_t kCUs = 256;
static constexpr int64_t kOverheadStages = 8;

static double tile_cost(const TileConfig& t, int64_t m, int64_t n, int64_t k, int esz) {
  const SplitPlan sp = split_plan(t, m, n, k, esz);
  const int64_t bk = kRowBytes / esz;
  const int64_t units = cdiv(m, t.bm) * cdiv(n, t.bn) * sp.splits;
  const int64_t per_cu = cdiv(units, kCUs);
  const double eff = (per_cu >= t.occ ? t.eff : t.solo_eff) / 100.0;
  const int64_t kwork = std::min(k, (int64_t)sp.kslice * bk) + kOverheadStages * bk;
  double cost = (double)per_cu * t.bm * t.bn * kwork / eff;
  if (sp.splits > 1) cost += 2.0 * sp.splits * (double)m * n * 4 * 8 / kCUs;
  return cost;
}

// Shape heuristic behind FORGEML_CONFIG_AUTO for the tiled kernels: the
// lowest tile_cost, larger tiles winning within 1 %.  Only tiles built for
// the operand combination the layout runs on them are offered
// (combo_supported, the launch's own test): the 8-wave 16-bit tile takes
// K-contiguous operands only (its register budget does not fit the
// transposing loaders), and 16-bit element loads, including a pair of modes
// that steps down to them, run on 64x64 (their staged values and addresses
// outgrow the registers of larger tiles).  Layouts whose kernels exist only
// for small tiles choose among those.  Tiles whose grid would reach 2^32
// work-items are skipped; -1 when no allowed tile fits.
static int select_config(int64_t m, int64_t n, int64_t k, int dtype, int ma, int mb) {
  const int dclass = dclass_of(dtype);
  const int esz = esize_of(dtype);
  const int64_t max_area = needs_small_tile(ma, mb) ? kSmallTileArea : INT64_MAX;
  int best = -1;
  double best_cost = 0.0;
  for (int id = 0; id < kNumTiles; ++id) {
    const TileConfig& t = kTiles[id];
    if (t.dclass != dclass || t.kind != KIND_TILED) continue;
    const int64_t area = (int64_t)t.bm * t.bn;
    if (area > max_area) continue;
    if (!combo_supported(t.dclass, t.bm, t.bn, t.wm * t.wn, combo_of(ma, mb, area <= kSmallTileArea))) continue;
    if (launch_items(t, m, n, split_plan(t, m, n, k, esz).splits) >= kMaxItems) continue;
    const double cost = tile_cost(t, m, n, k, esz);
    bool take = best < 0 || cost < best_cost * 0.99;  // clearly cheaper
    if (!take && cost <= best_cost * 1.01) take = area > (int64_t)kTiles[best].bm * kTiles[best].bn;  // a tie: bigger
    if (take) {
      best = id;
      best_cost = cost;
    }
  }
  return best;
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
  out[4] = t.wm * t.wn;
  if (t.kind == KIND_SKINNY) {
    // block_k: K of one chunk (a 16-byte vector per lane, 4 lane groups);
    // stages: the most chunks in flight per wave (a launch may keep 2, as
    // skinny_depth decides); LDS: the cross-wave reduction.
    out[3] = t.dclass == 0 ? 16 : 32;
    out[5] = kSkinnyDepth;
    out[6] = 1;
    out[7] = kSkinnyWaves * (kSkinnyMaxRows / 16) * 64 * 16;
    return FORGEML_OK;
  }
  out[3] = t.dclass == 0 ? kRowBytes / 4 : kRowBytes / 2;
  // Stages and LDS at most, for K-contiguous operands (transposing loaders use
  // two stages, and a 64x64 tile runs two on grids of more than 512 workgroups).
  const int stages = (int64_t)t.bm * t.bn <= 64 * 64 ? 4 : 2;
  out[5] = stages;
  out[6] = (int32_t)kMaxSplit;
  out[7] = stages * (t.bm + t.bn) * kRowBytes + (t.dclass != 0 && t.bm * t.bn >= 256 * 256 && t.wm * t.wn == 8 ? kLutBytes : 0);
  return FORGEML_OK;
}

int forgeml_hip_select_config(int64_t m, int64_t n, int64_t k, int32_t dtype) {
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  if (m <= 0 || n <= 0 || k <= 0) return set_error(FORGEML_EINVAL, "select_config: M, N, K must be positive");
  if (m <= kSkinnyMaxRows && skinny_preferred(m, n, k, 16, esize_of(dtype)) &&
      launch_items(kTiles[skinny_id(dclass_of(dtype))], m, n, 1) < kMaxItems)
    return skinny_id(dclass_of(dtype));
  const int id = select_config(m, n, k, dtype, MODE_K, MODE_K);
  if (id < 0) return set_error(FORGEML_EINVAL, "select_config: no tile fits a launch of fewer than 2^32 work-items");
  return id;
}

int64_t forgeml_hip_gemm_workspace_size(int64_t m, int64_t n, int64_t k, int32_t dtype, int32_t config_id) {
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  if (m <= 0 || n <= 0 || k <= 0) return set_error(FORGEML_EINVAL, "workspace_size: M, N, K must be positive");
  if (config_id != FORGEML_CONFIG_AUTO && (config_id < 0 || config_id >= kNumTiles))
    return set_error(FORGEML_ECONFIG, "config id %d out of range", config_id);
  if (config_id != FORGEML_CONFIG_AUTO && kTiles[config_id].dclass != dclass_of(dtype))
    return set_error(FORGEML_ECONFIG, "config %d is not built for dtype %d", config_id, dtype);
  const int esz = esize_of(dtype);
  if (config_id != FORGEML_CONFIG_AUTO) return workspace_bytes_for(split_plan(kTiles[config_id], m, n, k, esz), m, n);
  // The automatic tile depends on the operands' layout: cover every choice.
  static const int kModePairs[][2] = {{MODE_K, MODE_K}, {MODE_K, MODE_MN}, {MODE_K4, MODE_K4}, {MODE_G, MODE_MN}};
  int64_t most = 0;
  for (const auto& mp : kModePairs) {
    const int id = select_config(m, n, k, dtype, mp[0], mp[1]);
    if (id < 0) continue;
    most = std::max(most, workspace_bytes_for(split_plan(kTiles[id], m, n, k, esz), m, n));
  }
  return most;
}

}  // extern "C"

namespace forgeml {

// Everything forgeml_hip_gemm decides before a launch: argument checks, the
// operands' load modes, the config, the K split and the workspace.
struct LaunchPlan {
  int config_id;
  int combo;  // tiled: COMBO_*; few-row kernel: load width in bytes
  SplitPlan split;
  int64_t ws_need;
  int64_t sam, sak, sbk, sbn;  // with size-1 dimensions' strides zeroed
};

static int plan_launch(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn, int64_t m,
                       int64_t n, int64_t k, int32_t dtype, int32_t config_id, LaunchPlan& out) {
  if (a == nullptr || b == nullptr) return set_error(FORGEML_EINVAL, "a and b must be non-NULL");
  if (m <= 0 || n <= 0 || k <= 0) return set_error(FORGEML_EINVAL, "M, N, K must be positive (got %lld, %lld, %lld)",
                                                   (long long)m, (long long)n, (long long)k);
  if (m > INT_MAX || n > INT_MAX || k > INT_MAX || m * n > (int64_t)INT_MAX * 64)
    return set_error(FORGEML_EINVAL, "shape too large for this kernel family");
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  if (sam < 0 || sak < 0 || sbk < 0 || sbn < 0) return set_error(FORGEML_EINVAL, "negative strides are not supported");
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
  const int lw = skinny_width(m, k, sam, sak, sbn, sbk, ma, mb, esz);
  if (config_id == FORGEML_CONFIG_AUTO)
    config_id = skinny_preferred(m, n, k, lw, esz) && launch_items(kTiles[skinny_id(dclass_of(dtype))], m, n, 1) < kMaxItems
                    ? skinny_id(dclass_of(dtype))
                    : select_config(m, n, k, dtype, ma, mb);
  if (config_id < 0)
    return set_error(FORGEML_EINVAL, "shape needs 2^32 or more work-items in one launch with every tile this layout allows");
  const TileConfig& t = kTiles[config_id];
  if (t.dclass != dclass_of(dtype) || t.launch[dtype] == nullptr)
    return set_error(FORGEML_ECONFIG, "config %d is not built for dtype %d", config_id, dtype);
  if (t.kind == KIND_SKINNY && lw == 0)
    return set_error(FORGEML_ECONFIG, "config %d (few-row kernel) needs M <= %d and K-contiguous A and B", config_id,
                     kSkinnyMaxRows);
  out.config_id = config_id;
  out.combo = t.kind == KIND_SKINNY ? lw : combo_of(ma, mb, (int64_t)t.bm * t.bn <= kSmallTileArea);
  if (t.kind == KIND_TILED && !combo_supported(t.dclass, t.bm, t.bn, t.wm * t.wn, out.combo))
    return set_error(FORGEML_ECONFIG,
                     "config %d (%dx%d, %d waves) is not built for this operand layout (%s); choose a smaller tile "
                     "or FORGEML_CONFIG_AUTO",
                     config_id, t.bm, t.bn, t.wm * t.wn,
                     t.wm * t.wn > 4 ? "it takes K-contiguous A and B with 16-byte rows" : "16-bit element loads");
  out.split = split_plan(t, m, n, k, esz);
  out.ws_need = workspace_bytes_for(out.split, m, n);
  out.sam = sam;
  out.sak = sak;
  out.sbk = sbk;
  out.sbn = sbn;
  if (launch_items(t, m, n, out.split.splits) >= kMaxItems)
    return set_error(FORGEML_EINVAL, "shape needs 2^32 or more work-items in one launch with config %d", config_id);
  return FORGEML_OK;
}

}  // namespace forgeml

extern "C" {

int forgeml_hip_gemm_plan(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn, int64_t m,
                          int64_t n, int64_t k, int32_t dtype, int32_t config_id, int64_t* out) {
  g_last_error[0] = '\0';
  if (out == nullptr) return set_error(FORGEML_EINVAL, "gemm_plan: out is NULL");
  LaunchPlan plan;
  const int rc = plan_launch(a, sam, sak, b, sbk, sbn, m, n, k, dtype, config_id, plan);
  if (rc != FORGEML_OK) return rc;
  out[0] = plan.config_id;
  out[1] = plan.split.splits;
  out[2] = plan.ws_need;
  out[3] = kTiles[plan.config_id].kind;
  return FORGEML_OK;
}

}  // extern "C"

namespace forgeml {

static int gemm_impl(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn, const void* bias,
                     int64_t sbi, void* c, const void* res, int64_t srm, int64_t srn, int64_t m, int64_t n, int64_t k,
                     int32_t dtype, int32_t act, int32_t config_id, void* workspace, int64_t workspace_bytes,
                     void* stream) {
  g_last_error[0] = '\0';
  if (a == nullptr || b == nullptr || c == nullptr) return set_error(FORGEML_EINVAL, "a, b and c must be non-NULL");
  if (act < FORGEML_ACT_NONE || act > FORGEML_ACT_RELU) return set_error(FORGEML_EINVAL, "unknown activation %d", act);
  if (sbi < 0 || srm < 0 || srn < 0) return set_error(FORGEML_EINVAL, "negative strides are not supported");
  LaunchPlan plan;
  const int rc = plan_launch(a, sam, sak, b, sbk, sbn, m, n, k, dtype, config_id, plan);
  if (rc != FORGEML_OK) return rc;
  if (res != nullptr && res != c) {
    // The residual may be C itself (each element is read, then written, by one
    // thread) but must not partly overlap it.
    const int esz = esize_of(dtype);
    const uintptr_t r0 = (uintptr_t)res, r1 = r0 + (uintptr_t)(((m - 1) * srm + (n - 1) * srn + 1) * esz);
    const uintptr_t c0 = (uintptr_t)c, c1 = c0 + (uintptr_t)(m * n * esz);
    if (r0 < c1 && c0 < r1) return set_error(FORGEML_EINVAL, "the residual partly overlaps C");
  }
  if (res == c && res != nullptr && !(srn == 1 && (srm == n || m == 1)))
    return set_error(FORGEML_EINVAL, "a residual that is C must have C's strides (N, 1)");
  const TileConfig& t = kTiles[plan.config_id];
  if (plan.ws_need > 0) {
    if (workspace == nullptr || workspace_bytes < plan.ws_need)
      return set_error(FORGEML_EWORKSPACE, "this shape splits K %d ways and needs %lld workspace bytes (got %lld)",
                       plan.split.splits, (long long)plan.ws_need,
                       (long long)(workspace == nullptr ? 0 : workspace_bytes));
    if (((uintptr_t)workspace & 15) != 0) return set_error(FORGEML_EWORKSPACE, "workspace must be 16-byte aligned");
  }

  GemmArgs p;
  p.a = (const char*)a;
  p.b = (const char*)b;
  p.bias = (const char*)bias;
  p.c = (char*)c;
  p.sam = plan.sam;
  p.sak = plan.sak;
  p.sbk = plan.sbk;
  p.sbn = plan.sbn;
  p.sbi = sbi;
  p.m = (int)m;
  p.n = (int)n;
  p.k = (int)k;
  p.act = act;
  p.has_bias = bias != nullptr;
  p.res = (const char*)res;
  p.srm = srm;
  p.srn = srn;
  p.tiles_m = (int)cdiv(m, t.bm);
  p.tiles_n = (int)cdiv(n, t.bn);
  // Tile rows per group of the workgroup order (tile_coords): an XCD (32 CUs)
  // runs about C = 32 * occ tiles at once, gsz rows by C / gsz columns of
  // tiles, which stream gsz * BM rows of A and C / gsz * BN columns of B
  // through its L2 together; gsz = sqrt(C * BN / BM) minimises that.  It is 6
  // for the 256x256 tiles (bf16 8192x14336x4096: 861 -> 824 us; a 256x128
  // fp32 tile took 4: fp32 4096^3 HBM fetch -20 %, same time); 8, the
  // earlier fixed choice, for the tiles that share a CU.
  const int gsz = (int)lround(sqrt(32.0 * t.occ * t.bn / t.bm));
  p.group_m = p.tiles_m < gsz ? p.tiles_m : gsz;
  p.splits = plan.split.splits;
  p.kslice = plan.split.kslice;
  p.ws = plan.ws_need > 0 ? (float*)workspace : nullptr;
  return t.launch[dtype](p, plan.combo, (hipStream_t)stream);
}

}  // namespace forgeml

extern "C" {

int forgeml_hip_gemm(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn,
                     const void* bias, int64_t sbi, void* c, int64_t m, int64_t n, int64_t k, int32_t dtype,
                     int32_t act, int32_t config_id, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_impl(a, sam, sak, b, sbk, sbn, bias, sbi, c, nullptr, 0, 0, m, n, k, dtype, act, config_id, workspace,
                   workspace_bytes, stream);
}

int forgeml_hip_gemm_add(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn,
                         const void* bias, int64_t sbi, const void* r, int64_t srm, int64_t srn, void* c, int64_t m,
                         int64_t n, int64_t k, int32_t dtype, int32_t act, int32_t config_id, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  if (r == nullptr) return set_error(FORGEML_EINVAL, "gemm_add: the residual must be non-NULL");
  return gemm_impl(a, sam, sak, b, sbk, sbn, bias, sbi, c, r, srm, srn, m, n, k, dtype, act, config_id, workspace,
                   workspace_bytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The allocation-free entry point.  Its split-K planes live in `scratch`, a
// file-scope device array every GPU holds a copy of from the library's first
// use on it until the process ends.  The host-side name `scratch` is only a
// stand-in for the symbol: the device address of this GPU's copy comes from
// hipGetSymbolAddress, looked up once per device with that device current
// and kept in g_scratch.  Nothing in the planes needs clearing between
// calls: each K slice overwrites its whole M x N plane before the reduce
// kernel reads it.
namespace forgeml {

constexpr int64_t kScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

static std::mutex g_scratch_lock;
static void* g_scratch[kMaxDevices];

static int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(FORGEML_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(FORGEML_EHIP, "device index %d out of range", dev);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(FORGEML_EHIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                       hipGetErrorString(e));
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return FORGEML_OK;
}

}  // namespace forgeml

extern "C" {

int64_t forgeml_hip_noalloc_scratch_bytes(void) { return kScratchBytes; }

int forgeml_hip_gemm_noalloc(const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk, int64_t sbn,
                             const void* bias, int64_t sbi, void* c, int64_t m, int64_t n, int64_t k, int32_t dtype,
                             int32_t act, int32_t config_id, void* stream) {
  g_last_error[0] = '\0';
  LaunchPlan plan;
  const int rc = plan_launch(a, sam, sak, b, sbk, sbn, m, n, k, dtype, config_id, plan);
  if (rc != FORGEML_OK) return rc;
  if (plan.ws_need > kScratchBytes)
    return set_error(FORGEML_EWORKSPACE,
                     "this shape splits K %d ways and needs %lld bytes of scratch; the allocation-free entry point "
                     "holds %lld (use forgeml_hip_gemm with a workspace)",
                     plan.split.splits, (long long)plan.ws_need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (plan.ws_need > 0) {
    const int src = scratch_for_current_device(&ws);
    if (src != FORGEML_OK) return src;
  }
  return gemm_impl(a, sam, sak, b, sbk, sbn, bias, sbi, c, nullptr, 0, 0, m, n, k, dtype, act, config_id, ws,
                   plan.ws_need, stream);
}

}  // extern "C"

