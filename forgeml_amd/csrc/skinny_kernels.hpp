// skinny_kernels.hpp — gfx950 fused GEMM + bias + activation for few rows
// (M <= 64): decode-style linear layers, where C is a handful of rows and the
// weight is streamed from HBM once.
//
// Same contract as the tiled kernels (src/forgeml/_triton.py:6-62):
//   C[M,N] = act(rnd(rnd(sum_k A[m,k] B[k,n]) + bias[n]))
// for A and B both K-contiguous (A row-major, B = W^T of an nn.Linear weight).
//
// Design:
//  * A workgroup owns 16 output columns and 16*TM rows (TM <= 4): rows are
//    padded to 16 for v_mfma_f32_16x16x4_f32 (fp32) or
//    v_mfma_f32_16x16x32_{bf16,f16} (16-bit), instead of to a 64-row tile,
//    and split over workgroups when the column groups alone leave CUs idle.
//  * Its 8 waves split K.  Each wave streams its K range in chunks of one
//    16-byte vector per lane per operand (16 fp32 or 32 bf16 of K), straight
//    from global memory into registers, with 4 chunks in flight: no LDS
//    staging, and every weight byte is read once.
//  * Lane l holds column (or row) l%16 and K group l/16 of a chunk.  For fp32
//    the 4 values of a lane's vector feed 4 MFMAs (K elements 4g+e, e = 0..3),
//    the same permutation of K for A and B, so the sum is unchanged.
//  * The 8 partial sums are added in LDS in wave order (deterministic), then
//    rounded, biased, activated and stored.
//  * Rows past M, columns past N and K past the end are out of range of the
//    buffer resources: loads return zeros without touching memory.
//  * Load width follows the operands' alignment: 16-byte vectors, or 4-byte
//    or 2-byte pieces assembled into the same registers when rows are not
//    16-byte aligned (an odd K).
#pragma once

#include "gemm_kernels.hpp"

namespace forgeml {

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyThreads = kSkinnyWaves * 64;
constexpr int kSkinnyDepth = 4;     // chunks in flight per wave
constexpr int kSkinnyMaxRows = 64;  // 16 * TM, TM <= 4

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// One lane's 16 bytes of an operand row: K elements [k, k + 16/ESZ) of the
// row at byte offset `row_off` (kOutOfRange for a padding row).  LW is the
// load width in bytes (16, 4 or 2); each piece is in range only if its
// first element is below K (for LW 4 with 16-bit data, K is even).
template <int DT, int LW>
__device__ __forceinline__ u32x4 skinny_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t row_off, int k, int kdim) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int EPL = LW / ESZ > 0 ? LW / ESZ : 1;  // elements per piece
  const uint32_t base = row_off + (uint32_t)(k * ESZ);
  if constexpr (LW == 16) {
    const uint32_t off = (row_off != kOutOfRange && k < kdim) ? base : kOutOfRange;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, 0, 0));
  } else if constexpr (LW == 4) {
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = row_off != kOutOfRange && k + e * EPL < kdim;
      v[e] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)(ok ? base + 4 * e : kOutOfRange), 0, 0);
    }
    return v;
  } else {
    static_assert(LW == 2 && ESZ == 2, "2-byte pieces are for 16-bit data");
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok0 = row_off != kOutOfRange && k + 2 * e < kdim;
      const bool ok1 = row_off != kOutOfRange && k + 2 * e + 1 < kdim;
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rsrc, (int)(ok0 ? base + 4 * e : kOutOfRange), 0, 0);
      const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rsrc, (int)(ok1 ? base + 4 * e + 2 : kOutOfRange), 0, 0);
      v[e] = (lo & 0xffffu) | (hi << 16);
    }
    return v;
  }
}

template <int DT>
__device__ __forceinline__ f32x4 skinny_mma(const u32x4& a, const u32x4& b, f32x4 acc) {
  if constexpr (DT == DT_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(b[e]), acc, 0, 0, 0);
    return acc;
  } else if constexpr (DT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), acc,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), acc,
                                                  0, 0, 0);
  }
}

template <int DT, int ACT>
__device__ __forceinline__ void skinny_store(const GemmArgs& p, float v, int row, int col) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  float x = round_to<DT>(v);
  if (p.has_bias) x = round_to<DT>(x + load_as_f32<DT>(p.bias + (int64_t)col * p.sbi * ESZ));
  x = activate<DT, ACT>(x);
  if (p.res != nullptr) x = round_to<DT>(x + residual_at<DT>(p, row, col));
  store_from_f32<DT>(p.c + ((int64_t)row * p.n + col) * ESZ, x);
}

// Grid: ceil(N / 16) x ceil(M / (16 * TM)) workgroups of kSkinnyThreads;
// workgroup (x, y) owns columns [16x, 16x + 16) of rows [16*TM*y,
// 16*TM*(y + 1)).  The host guarantees M <= 64, both operands K-contiguous
// (sak = sbk = 1) with the alignment LW needs, and 32-bit byte offsets for
// both operands.
template <int DT, int TM, int LW>
__global__ __launch_bounds__(kSkinnyThreads) void skinny_gemm_kernel(GemmArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int VEC = 16 / ESZ;  // K elements per lane per chunk
  constexpr int CK = 4 * VEC;    // K elements per chunk (4 lane groups)
  constexpr int D = kSkinnyDepth;
  __shared__ f32x4 red[kSkinnyWaves][TM][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * TM;
  const int j = lane & 15, kq = lane >> 4;

  // This wave's chunks [c0, c1) of the K dimension.
  const int nk = (p.k + CK - 1) / CK;
  const int per = (nk + kSkinnyWaves - 1) / kSkinnyWaves;
  const int c0 = wave * per;
  const int c1 = min(nk, c0 + per);

  const uint32_t a_span = (uint32_t)(((int64_t)(p.m - 1) * p.sam + p.k) * ESZ);
  const int ncols = min(16, p.n - n0);
  const uint32_t b_span = (uint32_t)(((int64_t)(ncols - 1) * p.sbn + p.k) * ESZ);
  const __amdgpu_buffer_rsrc_t ra_rsrc = make_rsrc(p.a, a_span);
  const __amdgpu_buffer_rsrc_t rb_rsrc = make_rsrc(p.b + (int64_t)n0 * p.sbn * ESZ, b_span);
  uint32_t a_row[TM];
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) {
    const int row = m0 + mt * 16 + j;
    a_row[mt] = row < p.m ? (uint32_t)((int64_t)row * p.sam * ESZ) : kOutOfRange;
  }
  const uint32_t b_row = j < ncols ? (uint32_t)((int64_t)j * p.sbn * ESZ) : kOutOfRange;

  f32x4 acc[TM];
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Ring of D chunks in registers: slot i holds chunk c + i.  Chunks past this
  // wave's range load as out of range (no memory traffic).
  u32x4 ra[D][TM], rb[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int k = (c0 + i) * CK + kq * VEC;
    const int kl = c0 + i < c1 ? p.k : 0;
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) ra[i][mt] = skinny_load<DT, LW>(ra_rsrc, a_row[mt], k, kl);
    rb[i] = skinny_load<DT, LW>(rb_rsrc, b_row, k, kl);
  }
  for (int c = c0; c < c1; c += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      if (c + i < c1) {
#pragma unroll
        for (int mt = 0; mt < TM; ++mt) acc[mt] = skinny_mma<DT>(ra[i][mt], rb[i], acc[mt]);
      }
      const int cn = c + i + D;
      const int k = cn * CK + kq * VEC;
      const int kl = cn < c1 ? p.k : 0;
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) ra[i][mt] = skinny_load<DT, LW>(ra_rsrc, a_row[mt], k, kl);
      rb[i] = skinny_load<DT, LW>(rb_rsrc, b_row, k, kl);
    }
  }

  // Partial sums of the 8 waves, added in wave order.  Lane l of a 16x16
  // accumulator holds column l%16, rows 4*(l/16) + r.
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();
  for (int o = threadIdx.x; o < TM * 256; o += kSkinnyThreads) {
    const int mt = o >> 8, i = (o >> 4) & 15, jj = o & 15;
    const int src = (i >> 2) * 16 + jj, r = i & 3;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) v += red[w][mt][src][r];
    const int row = m0 + mt * 16 + i, col = n0 + jj;
    if (row < p.m && col < p.n) {
      switch (p.act) {
        case ACT_GELU_ERF: skinny_store<DT, ACT_GELU_ERF>(p, v, row, col); break;
        case ACT_GELU_TANH: skinny_store<DT, ACT_GELU_TANH>(p, v, row, col); break;
        case ACT_RELU: skinny_store<DT, ACT_RELU>(p, v, row, col); break;
        default: skinny_store<DT, ACT_NONE>(p, v, row, col); break;
      }
    }
  }
}

}  // namespace forgeml
