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
//  * Its 8 waves split K into 8 ranges (rotated over the waves from one
//    workgroup to the next).  Each wave streams its K range in chunks of one
//    16-byte vector per lane per operand (16 fp32 or 32 bf16 of K), straight
//    from global memory into registers, with D = 2 or 4 chunks in flight: no
//    LDS staging, and every weight byte is read once.
//  * Lane l holds column (or row) l%16 and K group l/16 of a chunk.  For fp32
//    the 4 values of a lane's vector feed 4 MFMAs (K elements 4g+e, e = 0..3),
//    the same permutation of K for A and B, so the sum is unchanged.
//  * The 8 partial sums are added in LDS in K-range order (deterministic),
//    then rounded, biased, activated and stored.
//  * Rows past M, columns past N and K past the end are out of range of the
//    buffer resources: loads return zeros without touching memory.
//  * Rows that are not 16-byte aligned (an odd K) still load 16-byte
//    vectors, from dword-aligned addresses (2-byte rows add the next dword
//    and shift the pair by 2 bytes); only the lanes at the very end of the
//    operand realign an aligned vector in registers.
#pragma once

#include "gemm_kernels.hpp"

namespace forgeml {

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyDepth = 4;     // most chunks in flight per wave
constexpr int kSkinnyMaxRows = 64;  // 16 * TM, TM <= 4

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// Buffer resource over an operand: with LW < 16 it starts at the operand's
// base rounded down to 16 bytes (`mis` = base mod 16 bytes earlier) and ends
// at its last byte rounded up to 16 (`nrec` bytes), so the extra bytes share
// a 16-byte block (so a page) with the operand's own.
template <int LW>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t skinny_rsrc(const char* base, uint32_t span, uint32_t& mis,
                                                              uint32_t& nrec) {
  mis = LW == 16 ? 0u : (uint32_t)((uintptr_t)base & 15);
  nrec = LW == 16 ? span : ((span + mis + 15u) & ~15u);
  return make_rsrc(base - mis, nrec);
}

// Byte position of a lane's 16 bytes from the resource base.
template <int DT>
__device__ __forceinline__ uint32_t skinny_pos(uint32_t row_off, int k, uint32_t mis) {
  return row_off + (uint32_t)(k * DTraits<DT>::ESZ) + mis;
}

// A lane's load of one chunk: 16 bytes, and with LW == 2 the dword after them.
struct SkinnyVec {
  u32x4 v;
  uint32_t x;
};

// One lane's 16 bytes of an operand row for the chunk at K element `k`: the
// row at byte offset `row_off` (kOutOfRange for a padding row) from the
// operand's base; zeros when `k` is at or past `kdim`.  Rows under 16-byte
// alignment are read with dword-aligned 16-byte loads (legal at any dword
// address; 2-byte-aligned vector loads are split by the hardware and measured
// slower): for 2-byte rows the load starts at the lane's first byte rounded
// down to a dword, and the dword after it is loaded too when that rounding
// moved the start (skinny_join shifts the pair into place).  A lane whose
// bytes would run past the resource's end loads the aligned block holding
// its first byte instead, for skinny_tail.
template <int DT, int LW>
__device__ __forceinline__ SkinnyVec skinny_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t row_off, int k, int kdim,
                                                 uint32_t mis, uint32_t nrec) {
  const bool ok = row_off != kOutOfRange && k < kdim;
  uint32_t o = kOutOfRange, ox = kOutOfRange;
  if constexpr (LW == 16) {
    if (ok) o = skinny_pos<DT>(row_off, k, 0);
  } else {
    static_assert(LW == 4 || (LW == 2 && DTraits<DT>::ESZ == 2), "2-byte rows are for 16-bit data");
    const uint32_t pos = skinny_pos<DT>(row_off, k, mis), p4 = pos & ~3u;
    if (ok) {
      o = p4 + 16u <= nrec ? p4 : (pos & ~15u);
      if (LW == 2 && (pos & 2u) != 0 && p4 + 16u < nrec) ox = p4 + 16u;
    }
  }
  SkinnyVec r;
  r.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)o, 0, 0));
  r.x = LW == 2 ? __builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)ox, 0, 0) : 0u;
  return r;
}

// The lane's 16 bytes from a dword-aligned load of 2-byte rows: `b2` (0 or 2)
// bytes into v:x.
__device__ __forceinline__ u32x4 skinny_join(const SkinnyVec& r, uint32_t b2) {
  u32x4 v;
  v[0] = __builtin_amdgcn_alignbyte(r.v[1], r.v[0], b2);
  v[1] = __builtin_amdgcn_alignbyte(r.v[2], r.v[1], b2);
  v[2] = __builtin_amdgcn_alignbyte(r.v[3], r.v[2], b2);
  v[3] = __builtin_amdgcn_alignbyte(r.x, r.v[3], b2);
  return v;
}

// The chunk holding the end of K, with LW < 16.  A lane whose bytes ran past
// the resource's end loaded an aligned block: it shifts it down by its
// misalignment (dword select, then v_alignbyte_b32 for a 2-byte offset; the
// bytes past the end read as zero); the others shift as skinny_join does.
// Then elements at or past `kdim` (the next row's bytes) are zeroed.
template <int DT, int LW>
__device__ __forceinline__ u32x4 skinny_tail(const SkinnyVec& r, uint32_t row_off, int k, int kdim, uint32_t mis,
                                             uint32_t nrec) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  const uint32_t pos = skinny_pos<DT>(row_off, k, mis);
  const bool whole = (pos & ~3u) + 16u <= nrec;
  const uint32_t sh = row_off == kOutOfRange ? 0u : whole ? (pos & 3u) : (pos & 15u);
  const uint32_t x = whole ? r.x : 0u;
  // d_i = dword i + sh/4 of v:x, chosen among named values (an array here
  // would be indexed by a lane value and spill to scratch).
  const bool s1 = (sh & 4u) != 0, s2 = (sh & 8u) != 0;
  auto pick = [&](uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    return s2 ? (s1 ? w3 : w2) : (s1 ? w1 : w0);
  };
  const u32x4& w = r.v;
  const uint32_t d0 = pick(w[0], w[1], w[2], w[3]);
  const uint32_t d1 = pick(w[1], w[2], w[3], x);
  const uint32_t d2 = pick(w[2], w[3], x, 0u);
  const uint32_t d3 = pick(w[3], x, 0u, 0u);
  u32x4 v;
  if constexpr (LW == 2) {
    const uint32_t d4 = pick(x, 0u, 0u, 0u);
    const uint32_t b = sh & 3u;  // 0 or 2 bytes
    v[0] = __builtin_amdgcn_alignbyte(d1, d0, b);
    v[1] = __builtin_amdgcn_alignbyte(d2, d1, b);
    v[2] = __builtin_amdgcn_alignbyte(d3, d2, b);
    v[3] = __builtin_amdgcn_alignbyte(d4, d3, b);
  } else {
    v[0] = d0;
    v[1] = d1;
    v[2] = d2;
    v[3] = d3;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (ESZ == 4) {
      v[i] = k + i < kdim ? v[i] : 0u;
    } else {
      const uint32_t keep = (k + 2 * i < kdim ? 0x0000ffffu : 0u) | (k + 2 * i + 1 < kdim ? 0xffff0000u : 0u);
      v[i] &= keep;
    }
  }
  return v;
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
  if (p.res != nullptr) x = round_to<DT>(round_to<DT>(x) + residual_at<DT>(p, row, col));
  store_from_f32<DT>(p.c + ((int64_t)row * p.n + col) * ESZ, x);
}

// Grid: ceil(N / 16) x ceil(M / (16 * TM)) workgroups of kSkinnyWaves
// waves; workgroup (x, y) owns columns [16x, 16x + 16) of rows [16*TM*y,
// 16*TM*(y + 1)).  The waves split K; each keeps D chunks in flight, and
// needs one memory latency per round of D chunks.  The host guarantees
// M <= 64, both operands K-contiguous (sak = sbk = 1) with the alignment LW
// needs, and 32-bit byte offsets for both operands.
template <int DT, int TM, int LW, int D>
__global__ __launch_bounds__(kSkinnyWaves * 64) void skinny_gemm_kernel(GemmArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int VEC = 16 / ESZ;  // K elements per lane per chunk
  constexpr int CK = 4 * VEC;    // K elements per chunk (4 lane groups)
  constexpr int WV = kSkinnyWaves;
  static_assert(TM >= 1 && TM <= 4 && (D == 2 || D == kSkinnyDepth), "few-row variant not built");
  __shared__ f32x4 red[WV][TM][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * TM;
  const int j = lane & 15, kq = lane >> 4;

  // This wave's K range: chunks [c0, c1), range `slot` of WV.  The ranges
  // rotate over the waves from one workgroup of an XCD to the next (an XCD
  // runs every eighth workgroup index), so the workgroups side by side on an
  // XCD start on different parts of A, which all of them read in full (1-3 %
  // faster).  The partial sums are added in range order, whichever wave holds
  // a range, so results do not depend on the rotation.
  const int nk = (p.k + CK - 1) / CK;
  const int per = (nk + WV - 1) / WV;
  const int slot = (wave + (int)(blockIdx.x >> 3) + (int)blockIdx.y) % WV;
  const int c0 = slot * per;
  const int c1 = min(nk, c0 + per);

  const uint32_t a_span = (uint32_t)(((int64_t)(p.m - 1) * p.sam + p.k) * ESZ);
  const int ncols = min(16, p.n - n0);
  const uint32_t b_span = (uint32_t)(((int64_t)(ncols - 1) * p.sbn + p.k) * ESZ);
  uint32_t a_mis, b_mis, a_nrec, b_nrec;
  const __amdgpu_buffer_rsrc_t ra_rsrc = skinny_rsrc<LW>(p.a, a_span, a_mis, a_nrec);
  const __amdgpu_buffer_rsrc_t rb_rsrc = skinny_rsrc<LW>(p.b + (int64_t)n0 * p.sbn * ESZ, b_span, b_mis, b_nrec);
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

  // 2-byte rows: bytes a lane's dword-aligned loads start before its data
  // (the same for every chunk, whose size is a multiple of 16 bytes).
  uint32_t a_b2[TM], b_b2 = (b_row + b_mis) & 2u;
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) a_b2[mt] = (a_row[mt] + a_mis) & 2u;

  // Ring of D chunks in registers: slot i holds chunk c + i.  Chunks past this
  // wave's range load as out of range (no memory traffic).
  SkinnyVec ra[D][TM], rb[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int k = (c0 + i) * CK + kq * VEC;
    const int kl = c0 + i < c1 ? p.k : 0;
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) ra[i][mt] = skinny_load<DT, LW>(ra_rsrc, a_row[mt], k, kl, a_mis, a_nrec);
    rb[i] = skinny_load<DT, LW>(rb_rsrc, b_row, k, kl, b_mis, b_nrec);
  }
  for (int c = c0; c < c1; c += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      if (c + i < c1) {
        u32x4 b, a[TM];
        if (LW != 16 && c + i == nk - 1) {  // wave-uniform: the chunk holding the end of K
          const int k = (c + i) * CK + kq * VEC;
          b = skinny_tail<DT, LW>(rb[i], b_row, k, p.k, b_mis, b_nrec);
#pragma unroll
          for (int mt = 0; mt < TM; ++mt) a[mt] = skinny_tail<DT, LW>(ra[i][mt], a_row[mt], k, p.k, a_mis, a_nrec);
        } else if constexpr (LW == 2) {
          b = skinny_join(rb[i], b_b2);
#pragma unroll
          for (int mt = 0; mt < TM; ++mt) a[mt] = skinny_join(ra[i][mt], a_b2[mt]);
        } else {
          b = rb[i].v;
#pragma unroll
          for (int mt = 0; mt < TM; ++mt) a[mt] = ra[i][mt].v;
        }
#pragma unroll
        for (int mt = 0; mt < TM; ++mt) acc[mt] = skinny_mma<DT>(a[mt], b, acc[mt]);
      }
      const int cn = c + i + D;
      const int k = cn * CK + kq * VEC;
      const int kl = cn < c1 ? p.k : 0;
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) ra[i][mt] = skinny_load<DT, LW>(ra_rsrc, a_row[mt], k, kl, a_mis, a_nrec);
      rb[i] = skinny_load<DT, LW>(rb_rsrc, b_row, k, kl, b_mis, b_nrec);
    }
  }

  // Partial sums of the WV K ranges, added in range order.  Lane l of a
  // 16x16 accumulator holds column l%16, rows 4*(l/16) + r.
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) red[slot][mt][lane] = acc[mt];
  __syncthreads();
  for (int o = threadIdx.x; o < TM * 256; o += WV * 64) {
    const int mt = o >> 8, i = (o >> 4) & 15, jj = o & 15;
    const int src = (i >> 2) * 16 + jj, r = i & 3;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WV; ++w) v += red[w][mt][src][r];
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
