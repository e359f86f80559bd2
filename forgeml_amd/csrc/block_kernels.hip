// block_kernels.hip — the transformer block's non-GEMM hot ops on gfx950:
// LayerNorm over the last dimension and causal scaled-dot-product attention.
//
// ForgeML evaluates both with torch (src/forgeml/ops.py: `layer_norm` ->
// F.layer_norm, `sdpa` -> F.scaled_dot_product_attention), in the compiled
// transformer block between the GEMMs (src/forgeml/neural.py:18-53).
//
// LayerNorm: one wave per row; the row is held in registers as 16-byte
// vectors (up to 16 per lane; wider aligned rows spread over a workgroup of
// 256 or 1024 threads, and past that are read three times as vectors by a
// 1024-thread workgroup per row), mean
// and variance are two passes over those registers with reductions in a
// fixed order, y = (x - mean) / sqrt(var + eps) * w + b in
// fp32, rounded once to the output dtype.
//
// Attention (fp32, head dim D of 32, 64, 96 or 128): flash-style, two or four
// waves per 32 query rows, each streaming every second or fourth 32-key block
// with an online softmax, their states merged at the end.  A wave computes S^T = K Q^T on
// v_mfma_f32_32x32x2_f32, so that each lane
// owns one query column of S^T: the softmax row statistics are a reduction
// over the lane's 16 accumulator values plus one exchange with the other half
// wave, and the lane's probabilities are already the B operand of
// O^T += V^T P^T (the MFMA's K index runs over the keys the lane holds).  The
// output tile is transposed through LDS and stored as 16-byte rows.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>

#include "forgeml_hip.h"
#include "gemm_kernels.hpp"

namespace forgeml {

int set_error(int code, const char* fmt, ...);

// ---------------------------------------------------------------------------
// LayerNorm

struct LnArgs {
  const char* x;
  const char* w;  // nullable (then b is null too)
  const char* b;
  char* y;
  int64_t sx;  // row stride of x, elements
  int rows, cols;
  float eps;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The 16 / ESZ values of a 16-byte vector, as fp32.
template <int DT>
__device__ __forceinline__ void unpack16(const u32x4& w, float (&out)[16 / DTraits<DT>::ESZ]) {
  constexpr int ESZ = DTraits<DT>::ESZ;
#pragma unroll
  for (int e = 0; e < 16 / ESZ; ++e) {
    const uint32_t word = w[e * ESZ / 4];
    if constexpr (ESZ == 4) out[e] = __uint_as_float(word);
    else if constexpr (DT == DT_BF16) out[e] = bf16_to_f32((word >> (16 * (e & 1))) & 0xffffu);
    else out[e] = f16_to_f32((word >> (16 * (e & 1))) & 0xffffu);
  }
}

// y[c0 .. c0+VEC) = (v - mean) * rstd (* w + b), one 16-byte store.
template <int DT>
__device__ __forceinline__ void ln_store_vec(const LnArgs& p, char* yr, int64_t c0, const float* v, float mean,
                                             float rstd) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int VEC = 16 / ESZ;
  float o[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) o[e] = (v[e] - mean) * rstd;
  if (p.w != nullptr) {
    // Weight and bias as 16-byte vectors, like the row.
    float wv[VEC], bv[VEC];
    unpack16<DT>(*(const u32x4*)(p.w + c0 * ESZ), wv);
    unpack16<DT>(*(const u32x4*)(p.b + c0 * ESZ), bv);
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = o[e] * wv[e] + bv[e];
  }
  u32x4 w;
  if constexpr (ESZ == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(o[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack2<DT>(o[2 * e], o[2 * e + 1]);
  }
  // Non-temporal: the normalised row is streamed out, not kept in L2
  // (10-22 % faster on rows of 768 to 200000 elements).
  __builtin_nontemporal_store(w, (u32x4*)(yr + c0 * ESZ));
}

// Row held in registers: VPL 16-byte vectors per lane.
template <int DT, int VPL>
__global__ __launch_bounds__(256) void layer_norm_kernel(LnArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int VEC = 16 / ESZ;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // whole wave: no barrier below
  const char* xr = p.x + (int64_t)row * p.sx * ESZ;
  float v[VPL][VEC];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c0 = (lane + 64 * i) * VEC;
    if (c0 < p.cols) {
      unpack16<DT>(*(const u32x4*)(xr + (int64_t)c0 * ESZ), v[i]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += v[i][e];
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[i][e] = 0.0f;
    }
  }
  const float mean = wave_sum(sum) / (float)p.cols;
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c0 = (lane + 64 * i) * VEC;
    if (c0 < p.cols) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = v[i][e] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) / (float)p.cols + p.eps);
  char* yr = p.y + (int64_t)row * p.cols * ESZ;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c0 = (lane + 64 * i) * VEC;
    if (c0 < p.cols) ln_store_vec<DT>(p, yr, c0, v[i], mean, rstd);
  }
}

// Wider aligned rows, one workgroup of NT threads per row: the row held in
// registers as VPL 16-byte vectors per thread (at most 16 fp32 or 8 16-bit
// vectors, the most that stay in registers at 4 waves per SIMD), the wave
// sums combined through LDS in wave order.
template <int DT, int VPL, int NT>
__global__ __launch_bounds__(NT) void layer_norm_row_kernel(LnArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int VEC = 16 / ESZ;
  constexpr int NW = NT / 64;
  __shared__ float part_s[NW], part_q[NW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int row = blockIdx.x;  // one row per workgroup: every thread reaches the barriers
  const char* xr = p.x + (int64_t)row * p.sx * ESZ;
  float v[VPL][VEC];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c0 = ((int64_t)t + NT * i) * VEC;
    if (c0 < p.cols) {
      unpack16<DT>(*(const u32x4*)(xr + c0 * ESZ), v[i]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += v[i][e];
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[i][e] = 0.0f;
    }
  }
  sum = wave_sum(sum);
  if (lane == 0) part_s[wave] = sum;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) total += part_s[w];
  const float mean = total / (float)p.cols;
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c0 = ((int64_t)t + NT * i) * VEC;
    if (c0 < p.cols) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = v[i][e] - mean;
        sq += d * d;
      }
    }
  }
  sq = wave_sum(sq);
  if (lane == 0) part_q[wave] = sq;
  __syncthreads();
  float totq = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) totq += part_q[w];
  const float rstd = 1.0f / sqrtf(totq / (float)p.cols + p.eps);
  char* yr = p.y + (int64_t)row * p.cols * ESZ;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c0 = ((int64_t)t + NT * i) * VEC;
    if (c0 < p.cols) ln_store_vec<DT>(p, yr, c0, v[i], mean, rstd);
  }
}

// Chan, Golub and LeVeque's merge of two partial (count, mean, M2 = sum of
// squared deviations) statistics into (n, mean, m2).
__device__ __forceinline__ void chan_merge(float& n, float& mean, float& m2, float nb, float mb, float m2b) {
  const float nn = n + nb;
  if (nn == 0.0f) return;
  const float delta = mb - mean;
  const float r = nb / nn;
  mean = fmaf(delta, r, mean);
  m2 = m2 + m2b + delta * delta * n * r;
  n = nn;
}

// Rows wider still: one workgroup of 1024 threads per row, 16-byte vectors,
// the row read twice.  The first pass folds each vector's own mean and
// squared deviations into the thread's running (count, mean, M2) by Chan's
// merge, then merges lanes and waves the same way (waves in order): the
// centred variance without a separate pass for the mean (512x200000 fp32:
// 334 -> 274 us against three passes).  The second pass normalises.
constexpr int kLnWideThreads = 1024;
template <int DT>
__global__ __launch_bounds__(kLnWideThreads) void layer_norm_wide_kernel(LnArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int VEC = 16 / ESZ;
  constexpr int NT = kLnWideThreads, NW = NT / 64;
  __shared__ float part[3][NW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int row = blockIdx.x;  // one row per workgroup: every thread reaches the barrier
  const char* xr = p.x + (int64_t)row * p.sx * ESZ;
  float n = 0.0f, mean = 0.0f, m2 = 0.0f;
#pragma unroll 4
  for (int64_t c0 = (int64_t)t * VEC; c0 < p.cols; c0 += NT * VEC) {  // rows hold whole vectors
    float v[VEC];
    unpack16<DT>(*(const u32x4*)(xr + c0 * ESZ), v);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += v[e];
    const float mb = s * (1.0f / VEC);
    float q = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float d = v[e] - mb;
      q = fmaf(d, d, q);
    }
    chan_merge(n, mean, m2, (float)VEC, mb, q);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float nb = __shfl_xor(n, off, 64), mb = __shfl_xor(mean, off, 64), qb = __shfl_xor(m2, off, 64);
    chan_merge(n, mean, m2, nb, mb, qb);
  }
  if (lane == 0) {
    part[0][wave] = n;
    part[1][wave] = mean;
    part[2][wave] = m2;
  }
  __syncthreads();
  float tn = part[0][0], tm = part[1][0], tq = part[2][0];
#pragma unroll
  for (int w = 1; w < NW; ++w) chan_merge(tn, tm, tq, part[0][w], part[1][w], part[2][w]);
  const float rstd = 1.0f / sqrtf(tq / (float)p.cols + p.eps);
  char* yr = p.y + (int64_t)row * p.cols * ESZ;
#pragma unroll 4
  for (int64_t c0 = (int64_t)t * VEC; c0 < p.cols; c0 += NT * VEC) {
    float v[VEC];
    unpack16<DT>(*(const u32x4*)(xr + c0 * ESZ), v);
    ln_store_vec<DT>(p, yr, c0, v, tm, rstd);
  }
}

// Unaligned rows: element loads, the row read three times.
template <int DT>
__global__ __launch_bounds__(256) void layer_norm_any_kernel(LnArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const char* xr = p.x + (int64_t)row * p.sx * ESZ;
  float sum = 0.0f;
  for (int64_t c = lane; c < p.cols; c += 64) sum += load_as_f32<DT>(xr + c * ESZ);
  const float mean = wave_sum(sum) / (float)p.cols;
  float sq = 0.0f;
  for (int64_t c = lane; c < p.cols; c += 64) {
    const float d = load_as_f32<DT>(xr + c * ESZ) - mean;
    sq += d * d;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) / (float)p.cols + p.eps);
  char* yr = p.y + (int64_t)row * p.cols * ESZ;
  for (int64_t c = lane; c < p.cols; c += 64) {
    float t = (load_as_f32<DT>(xr + c * ESZ) - mean) * rstd;
    if (p.w != nullptr) t = t * load_as_f32<DT>(p.w + c * ESZ) + load_as_f32<DT>(p.b + c * ESZ);
    store_from_f32<DT>(yr + c * ESZ, t);
  }
}

template <int DT, int NT>
static bool launch_layer_norm_row(const LnArgs& p, hipStream_t stream) {
  constexpr int VEC = 16 / DTraits<DT>::ESZ;
  const int64_t per_thread = ((int64_t)p.cols + NT * VEC - 1) / (NT * VEC);
  const dim3 grid((unsigned)p.rows), block(NT);
  if (per_thread <= 8) {
    hipLaunchKernelGGL((layer_norm_row_kernel<DT, 8, NT>), grid, block, 0, stream, p);
    return true;
  }
  if constexpr (DTraits<DT>::ESZ == 4) {
    if (per_thread <= 16) {
      hipLaunchKernelGGL((layer_norm_row_kernel<DT, 16, NT>), grid, block, 0, stream, p);
      return true;
    }
  }
  return false;
}

// Rows per launch: a dispatch covers fewer than 2^32 work-items, and a
// workgroup-per-row kernel has 1024 threads per row at most.
static constexpr int64_t kLnRowsPerLaunch = (int64_t)1 << 21;

template <int DT>
static void launch_layer_norm_chunk(const LnArgs& p, bool vec, hipStream_t stream) {
  constexpr int VEC = 16 / DTraits<DT>::ESZ;
  const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
  const int per_lane = (p.cols + 64 * VEC - 1) / (64 * VEC);
  if (!vec) hipLaunchKernelGGL((layer_norm_any_kernel<DT>), grid, block, 0, stream, p);
  else if (per_lane > 16) {
    if (!launch_layer_norm_row<DT, 256>(p, stream) && !launch_layer_norm_row<DT, 1024>(p, stream))
      hipLaunchKernelGGL((layer_norm_wide_kernel<DT>), dim3((unsigned)p.rows), dim3(kLnWideThreads), 0, stream, p);
  }
  else if (per_lane <= 1) hipLaunchKernelGGL((layer_norm_kernel<DT, 1>), grid, block, 0, stream, p);
  else if (per_lane <= 2) hipLaunchKernelGGL((layer_norm_kernel<DT, 2>), grid, block, 0, stream, p);
  else if (per_lane <= 4) hipLaunchKernelGGL((layer_norm_kernel<DT, 4>), grid, block, 0, stream, p);
  else if (per_lane <= 8) hipLaunchKernelGGL((layer_norm_kernel<DT, 8>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((layer_norm_kernel<DT, 16>), grid, block, 0, stream, p);
}

template <int DT>
static int launch_layer_norm(const LnArgs& p, bool vec, hipStream_t stream) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  for (int64_t r0 = 0; r0 < p.rows; r0 += kLnRowsPerLaunch) {
    LnArgs c = p;
    c.x = p.x + r0 * p.sx * ESZ;
    c.y = p.y + r0 * p.cols * ESZ;
    c.rows = (int)(p.rows - r0 < kLnRowsPerLaunch ? p.rows - r0 : kLnRowsPerLaunch);
    launch_layer_norm_chunk<DT>(c, vec, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(FORGEML_EHIP, "layer_norm launch failed: %s", hipGetErrorString(e));
  }
  return FORGEML_OK;
}

// ---------------------------------------------------------------------------
// Causal (or full) attention, fp32.

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t sq[4], sk[4], sv[4], so[4];  // element strides (batch, head, sequence, dim)
  int batch, heads, lq, lk;
  int nqb;       // query blocks of 32 per (batch, head)
  int nitems;    // work items per (batch, head): its query blocks
  int causal;
  float scale_log2;  // scale * log2(e): softmax in base 2
};

// kAttnSplit (2 or 4) waves share a work item: wave w takes the item's key
// blocks kb with kb % kAttnSplit == w and keeps its own online-softmax state
// (m, l, O); the others hand their states to wave 0 through LDS, which
// merges, normalises and transposes the output, and all of them store it.
// The split multiplies the waves in flight and shortens each wave's serial
// chain of key blocks; two waves give each wave a longer pipelined chain and
// half the merging.  Measured (us, four waves -> two): head dim 128: 8x12x512
// causal 115 -> 86, 4x32x1024 causal 444 -> 353, full 688 -> 608; head dim
// 96 causal 67 -> 61; head dim 64: 8x12x512 causal 49.8 -> 45.6, 4x16x1024
// causal 91.9 -> 90.9, but full 8x12x512 66 -> 77 and 2x8x333 (dim 32)
// causal 7.7 -> 10.6.  attention_split() holds the rule.
inline int attention_split(int64_t items, int64_t dim, bool causal) {
  return dim >= 96 || (causal && items >= 1024) ? 2 : 4;
}

// One workgroup: one work item of head (b, h), query block qb (rows [32*qb,
// 32*qb + 32)).  With the causal mask, workgroup g takes query block
// nqb-1-g/(B*H): the grid lists the items longest first (qb + 1 key blocks),
// so as workgroups finish, the dispatcher hands the free CUs ever shorter
// items and the GPU drains evenly (longest-processing-time-first).  Measured
// against pairing blocks t and nqb-1-t into equal items (whose count, 3/2 of
// the workgroup slots on an 8x12x512 problem, left half the CUs idle in a
// second round): 54.2 -> 51.8 us at 8x12x512x64, 12.2 -> 9.1 us at 2x8x333x32.
// Two waves per SIMD up to head dim 96: at 96 that spills some registers and
// is still faster than one wave per SIMD (76 vs 98 us on an 8x12x512 causal
// problem).  Head dim 128 holds twice dim 64's fragments: one wave per SIMD,
// so nothing else hides a key block's K load: that wave loads the next key
// block's K while it works on this one (883 -> 794 us on full attention at
// 4x32x1024x128; at dim 64 the extra registers cost what they hide).
// kShort: lk < 32, one key block, whose V rows go in the loads' vector
// offsets (see load_v).
template <int D, int kAttnSplit, bool kShort>
__global__ __launch_bounds__(kAttnSplit * 64) __attribute__((amdgpu_waves_per_eu(D <= 96 ? 2 : 1, 8)))
void attention_kernel(AttnArgs p) {
  static_assert(D % 32 == 0 && D <= 128, "head dim must be 32, 64, 96 or 128");
  constexpr int NC = D / 8;   // 8-element chunks of the head dim
  constexpr int NB = D / 32;  // 32-row blocks of O^T
  __shared__ float tr[32][D + 1];        // merged output transpose; odd row length: conflict-free column writes
  __shared__ float part[kAttnSplit - 1][NB * 16][64];  // waves 1.. unnormalised O^T, accumulator layout
  __shared__ float part_ml[kAttnSplit - 1][2][64];     // their running max and sum per lane

  const int lane = threadIdx.x & 63, half = lane >> 5, lc = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;  // the grid is exactly one workgroup per work item
  const int nbh = p.batch * p.heads;
  const int t = g / nbh, bh = g % nbh;
  const int b = bh / p.heads, h = bh % p.heads;
  const float* qp = p.q + b * p.sq[0] + h * p.sq[1];
  const float* kp = p.k + b * p.sk[0] + h * p.sk[1];
  const float* vp = p.v + b * p.sv[0] + h * p.sv[1];
  const __amdgpu_buffer_rsrc_t qr = make_rsrc((const char*)qp, (uint32_t)(((int64_t)(p.lq - 1) * p.sq[2] + D) * 4));
  const __amdgpu_buffer_rsrc_t kr = make_rsrc((const char*)kp, (uint32_t)(((int64_t)(p.lk - 1) * p.sk[2] + D) * 4));
  const __amdgpu_buffer_rsrc_t vr = make_rsrc((const char*)vp, (uint32_t)(((int64_t)(p.lk - 1) * p.sv[2] + D) * 4));

  const int qb = p.causal ? p.nqb - 1 - t : t;
  const int q0 = qb * 32;
  // Q^T operand: this lane's query row lc, dims 8c + 4*half + e.
  const int qrow = q0 + lc;
  u32x4 qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t off = qrow < p.lq ? (uint32_t)(((int64_t)qrow * p.sq[2] + 8 * c + 4 * half) * 4) : kOutOfRange;
    qf[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, (int)off, 0, 0));
  }

  const int last_key = p.causal ? min(p.lk, q0 + 32) : p.lk;  // keys [0, last_key) can be visible
  const int nkb = (last_key + 31) / 32;

  // Loads of a key block: a lane's offset within the block is the same for
  // every block, and the block's own offset is wave-uniform, so it rides in
  // the loads' scalar offset and the loop spends no vector instructions on
  // addresses.  The buffer range check covers the vector offset only, not
  // the scalar one, so no block may reach past key lk through its scalar
  // offset: the last block, when lk is not a multiple of 32, starts at key
  // lk - 32 instead (its first keys, already counted by the block before,
  // are masked in the softmax).  With lk < 32 the one block starts at key 0,
  // its scalar offset is 0, and keys past lk fall past the resources' ends
  // (rows are at least D elements apart): they read as zeros.
  const uint32_t k_lane = (uint32_t)(((int64_t)lc * p.sk[2] + 4 * half) * 4);
  const uint32_t v_lane = (uint32_t)(((int64_t)4 * half * p.sv[2] + lc) * 4);
  auto key0 = [&](int kb) { return kb * 32 + 32 > p.lk && p.lk >= 32 ? p.lk - 32 : kb * 32; };
  auto load_k = [&](int kb, u32x4 (&kf)[NC]) {
    const int blk = (int)((int64_t)key0(kb) * p.sk[2] * 4);
#pragma unroll
    for (int c = 0; c < NC; ++c)
      kf[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, (int)(k_lane + 32 * c), blk, 0));
  };

  f32x16 o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[nb][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  // V^T operand of a key block: dim lc + 32*nb, key 8*(s/4) + 4*half + s%4.
  // A lane's V rows vary with s, and so does the scalar offset: with lk < 32
  // the row offset goes in the vector offset instead, where the range check
  // zeros the rows past lk.
  auto load_v = [&](int kb, float (&vf)[NB][16]) {
    const int k0 = key0(kb);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int blk = (int)((int64_t)(k0 + 8 * (s >> 2) + (s & 3)) * p.sv[2] * 4);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        vf[nb][s] = __uint_as_float(kShort ? __builtin_amdgcn_raw_buffer_load_b32(vr, (int)(v_lane + 128 * nb + blk), 0, 0)
                                           : __builtin_amdgcn_raw_buffer_load_b32(vr, (int)(v_lane + 128 * nb), blk, 0));
    }
  };

  // S^T[key][query] of the block in kf: one chain of dependent MFMAs, summed
  // over the head dim in order (two chains, even and odd dim chunks, cost 16
  // more VGPRs and an add per score, and measured no faster).
  auto scores = [&](const u32x4 (&kf)[NC], f32x16& s) {
    s = f32x16{};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(kf[c][e]), __uint_as_float(qf[c][e]), s, 0, 0, 0);
  };
  // Online softmax for query qrow (this lane's column) over block kb's keys of
  // this half: P into s; m, l and O^T rescaled.  Only the item's last key
  // block can hold keys that are masked (causal diagonal, keys past the end,
  // or, in a block moved back to start at key lk - 32, keys below kb * 32).
  auto softmax = [&](int kb, f32x16& s, bool masked) {
    float mx = -INFINITY;
    const int k0 = key0(kb);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float x = s[i] * p.scale_log2;
      if (masked) {
        const int key = k0 + 8 * (i >> 2) + 4 * half + (i & 3);
        x = (key >= kb * 32 && key < p.lk && (!p.causal || key <= qrow)) ? x : -INFINITY;
      }
      s[i] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float base = m_new == -INFINITY ? 0.0f : m_new;  // rows with nothing visible yet
    // v_exp_f32 directly: results under 2^-126 (flushed) are below a
    // rounding error of a sum that holds a 1.
    const float alpha = __builtin_amdgcn_exp2f(m - base);
    float rs = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = __builtin_amdgcn_exp2f(s[i] - base);
      rs += s[i];
    }
    rs += __shfl_xor(rs, 32, 64);
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[nb][i] *= alpha;
  };
  // O^T[dim][query] += V^T[dim][key] P^T[key][query]: step i takes the key of
  // this lane's accumulator value i.
  auto accumulate = [&](const float (&vf)[NB][16], const f32x16& s) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) o[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[nb][i], s[i], o[nb], 0, 0, 0);
  };

  // This wave's key blocks kb_j = wave + kAttnSplit*j, j < n, software
  // pipelined: iteration j issues the S MFMAs of block j+1, then the softmax
  // of block j (VALU work the SIMD runs while the matrix pipe is busy), block
  // j's PV MFMAs, and the loads of K of block j+2 and V of block j+1 behind
  // them.  Keys past the end read as zeros (the resources end at key lk, and
  // rows are at least D apart) and are masked in the last block's softmax.
  const int n = wave < nkb ? (nkb - 1 - wave) / kAttnSplit + 1 : 0;
  const int kb_last = wave + kAttnSplit * (n - 1);
  u32x4 kf[NC];
  float vf[NB][16];
  f32x16 s;
  if (n > 0) {
    load_k(wave, kf);
    load_v(wave, vf);
    scores(kf, s);
    load_k(min(wave + kAttnSplit, kb_last), kf);
  }
  for (int j = 0; j + 1 < n; ++j) {
    const int kb = wave + kAttnSplit * j;
    f32x16 sn;
    scores(kf, sn);
    load_k(min(kb + 2 * kAttnSplit, kb_last), kf);
    softmax(kb, s, false);
    accumulate(vf, s);
    load_v(kb + kAttnSplit, vf);
    s = sn;
  }
  if (n > 0) {
    softmax(kb_last, s, kb_last == nkb - 1);
    accumulate(vf, s);
  }

  // Merge the waves' states (base-2 running max m, sum l, unnormalised O^T):
  // each is rescaled by 2^(m_w - max), summed in wave order, normalised and
  // transposed through LDS.  A wave that saw no visible key has m = -inf and
  // contributes nothing.
  if (wave > 0) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) part[wave - 1][nb * 16 + i][lane] = o[nb][i];
    part_ml[wave - 1][0][lane] = m;
    part_ml[wave - 1][1][lane] = l;
  }
  __syncthreads();
  if (wave == 0) {
    float mm = m;
#pragma unroll
    for (int w = 0; w < kAttnSplit - 1; ++w) mm = fmaxf(mm, part_ml[w][0][lane]);
    const float base = mm == -INFINITY ? 0.0f : mm;
    const float a0 = m == -INFINITY ? 0.0f : exp2f(m - base);
    float aw[kAttnSplit - 1];
    float lt = l * a0;
#pragma unroll
    for (int w = 0; w < kAttnSplit - 1; ++w) {
      const float mw = part_ml[w][0][lane];
      aw[w] = mw == -INFINITY ? 0.0f : exp2f(mw - base);
      lt += part_ml[w][1][lane] * aw[w];
    }
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = o[nb][i] * a0;
#pragma unroll
        for (int w = 0; w < kAttnSplit - 1; ++w) v += part[w][nb * 16 + i][lane] * aw[w];
        tr[lc][nb * 32 + 8 * (i >> 2) + 4 * half + (i & 3)] = v * inv;
      }
  }
  __syncthreads();
  float* op = p.o + b * p.so[0] + h * p.so[1];
  constexpr int VPR = D / 4;  // 16-byte vectors per output row
  for (int idx = threadIdx.x; idx < 32 * VPR; idx += kAttnSplit * 64) {
    const int r = idx / VPR, c4 = (idx % VPR) * 4;
    const int qi = q0 + r;
    if (qi < p.lq) {
      float* dst = op + (int64_t)qi * p.so[2] + c4;
      const f32x4 val = {tr[r][c4], tr[r][c4 + 1], tr[r][c4 + 2], tr[r][c4 + 3]};
      if (p.so[3] == 1 && (((uintptr_t)dst) & 15) == 0) {
        __builtin_nontemporal_store(val, (f32x4*)dst);  // streamed out, as the GEMM epilogue's stores
      } else {
        dst[0] = val.x;
        dst[p.so[3]] = val.y;
        dst[2 * p.so[3]] = val.z;
        dst[3 * p.so[3]] = val.w;
      }
    }
  }
}

template <int D>
static int launch_attention(const AttnArgs& p, hipStream_t stream) {
  const int64_t items = (int64_t)p.batch * p.heads * p.nitems;
  if (p.lk < 32)
    hipLaunchKernelGGL((attention_kernel<D, 2, true>), dim3((unsigned)items), dim3(2 * 64), 0, stream, p);
  else if (attention_split(items, D, p.causal) == 2)
    hipLaunchKernelGGL((attention_kernel<D, 2, false>), dim3((unsigned)items), dim3(2 * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((attention_kernel<D, 4, false>), dim3((unsigned)items), dim3(4 * 64), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FORGEML_EHIP, "attention launch failed: %s", hipGetErrorString(e));
  return FORGEML_OK;
}

}  // namespace forgeml

using namespace forgeml;

extern "C" {

int forgeml_hip_layer_norm(const void* x, int64_t sx, const void* w, const void* b, void* y, int64_t rows,
                           int64_t cols, float eps, int32_t dtype, void* stream) {
  if (x == nullptr || y == nullptr) return set_error(FORGEML_EINVAL, "layer_norm: x and y must be non-NULL");
  if ((w == nullptr) != (b == nullptr)) return set_error(FORGEML_EINVAL, "layer_norm: give both weight and bias or neither");
  if (rows <= 0 || cols <= 0 || rows > INT_MAX || cols > INT_MAX || sx < cols)
    return set_error(FORGEML_EINVAL, "layer_norm: bad shape or row stride");
  if (!(eps > 0.0f) || !std::isfinite(eps)) return set_error(FORGEML_EINVAL, "layer_norm: eps must be finite and positive");
  if (dtype < FORGEML_DTYPE_F32 || dtype > FORGEML_DTYPE_F16) return set_error(FORGEML_EINVAL, "unknown dtype %d", dtype);
  const int esz = dtype == FORGEML_DTYPE_F32 ? 4 : 2;
  LnArgs p;
  p.x = (const char*)x;
  p.w = (const char*)w;
  p.b = (const char*)b;
  p.y = (char*)y;
  p.sx = sx;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.eps = eps;
  const bool vec = (cols * esz) % 16 == 0 && (sx * esz) % 16 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 &&
                   ((uintptr_t)w & 15) == 0 && ((uintptr_t)b & 15) == 0;
  switch (dtype) {
    case FORGEML_DTYPE_F32: return launch_layer_norm<DT_F32>(p, vec, (hipStream_t)stream);
    case FORGEML_DTYPE_BF16: return launch_layer_norm<DT_BF16>(p, vec, (hipStream_t)stream);
    default: return launch_layer_norm<DT_F16>(p, vec, (hipStream_t)stream);
  }
}

int forgeml_hip_attention(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const void* v,
                          const int64_t* sv, void* o, const int64_t* so, int64_t batch, int64_t heads, int64_t lq,
                          int64_t lk, int64_t dim, int32_t causal, float scale, int32_t dtype, void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || sq == nullptr || sk == nullptr || sv == nullptr ||
      so == nullptr)
    return set_error(FORGEML_EINVAL, "attention: pointers must be non-NULL");
  if (dtype != FORGEML_DTYPE_F32) return set_error(FORGEML_EINVAL, "attention: only fp32 is built");
  if (dim != 32 && dim != 64 && dim != 96 && dim != 128)
    return set_error(FORGEML_EINVAL, "attention: head dim must be 32, 64, 96 or 128 (got %lld)", (long long)dim);
  if (batch <= 0 || heads <= 0 || lq <= 0 || lk <= 0) return set_error(FORGEML_EINVAL, "attention: empty shape");
  if (sq[3] != 1 || sk[3] != 1 || sv[3] != 1)
    return set_error(FORGEML_EINVAL, "attention: q, k and v need a unit stride along the head dim");
  for (int i = 0; i < 4; ++i)
    if (sq[i] < 0 || sk[i] < 0 || sv[i] < 0 || so[i] < 0) return set_error(FORGEML_EINVAL, "attention: negative stride");
  if (((uintptr_t)q & 15) || ((uintptr_t)k & 15) || (sq[2] % 4) || (sk[2] % 4) || (sq[0] % 4) || (sq[1] % 4) ||
      (sk[0] % 4) || (sk[1] % 4))
    return set_error(FORGEML_EINVAL, "attention: q and k rows must be 16-byte aligned");
  // K and V rows at least a head dim apart: the last key block's resources
  // end at key lk's row, and keys past lk then start past that end.
  if (sk[2] < dim || sv[2] < dim)
    return set_error(FORGEML_EINVAL, "attention: k and v rows must be at least the head dim apart");
  // 32-bit byte offsets within one (batch, head) slice, up to the end of the
  // last 32-key block.
  if (((lq - 1) * sq[2] + dim) * 4 >= ((int64_t)1 << 31) || ((lk + 31) * sk[2] + dim) * 4 >= ((int64_t)1 << 31) ||
      ((lk + 31) * sv[2] + dim) * 4 >= ((int64_t)1 << 31))
    return set_error(FORGEML_EINVAL, "attention: a (batch, head) slice exceeds 2 GiB");
  const int64_t nqb = (lq + 31) / 32;
  // One workgroup per work item: the dispatch must cover fewer than 2^32 work-items.
  if (batch * heads * nqb * (4 * 64) >= ((int64_t)1 << 32))
    return set_error(FORGEML_EINVAL, "attention: more than 2^24 query blocks in one call");
  if (!(scale > 0.0f) || !std::isfinite(scale)) return set_error(FORGEML_EINVAL, "attention: scale must be finite and positive");
  AttnArgs p;
  p.q = (const float*)q;
  p.k = (const float*)k;
  p.v = (const float*)v;
  p.o = (float*)o;
  for (int i = 0; i < 4; ++i) {
    p.sq[i] = sq[i];
    p.sk[i] = sk[i];
    p.sv[i] = sv[i];
    p.so[i] = so[i];
  }
  p.batch = (int)batch;
  p.heads = (int)heads;
  p.lq = (int)lq;
  p.lk = (int)lk;
  p.nqb = (int)nqb;
  p.nitems = (int)nqb;
  p.causal = causal != 0;
  p.scale_log2 = scale * 1.44269504088896340736f;
  switch (dim) {
    case 32: return launch_attention<32>(p, (hipStream_t)stream);
    case 64: return launch_attention<64>(p, (hipStream_t)stream);
    case 96: return launch_attention<96>(p, (hipStream_t)stream);
    default: return launch_attention<128>(p, (hipStream_t)stream);
  }
}

}  // extern "C"
