// gemm_kernels.hpp — gfx950 (CDNA4) fused GEMM + bias + activation kernels.
//
// One kernel template covers every case of ForgeML's `_matmul_kernel`
// (src/forgeml/_triton.py:6-62):
//   C[M,N] = act(rnd(rnd(sum_k A[m,k] B[k,n]) + bias[n]))
// with fp32 accumulation, A and B of arbitrary element strides and C
// contiguous with row stride N (src/forgeml/_triton.py:58-62).
//
// Design (MI355X-first, not a translation of the Triton program):
//  * A workgroup owns a BM x BN output tile and walks K in stages of 128 bytes
//    (32 fp32 or 64 bf16/fp16 elements).  Each stage of A and of B is staged in
//    LDS as "rows" (an M row of A or an N column of B) of 128 bytes, so the
//    MFMA operand reads are the same byte pattern for every dtype.
//  * The 16-byte chunks of an LDS row are XOR-swizzled by (r ^ r>>3) & 7, which
//    keeps the MFMA operand reads (8 consecutive rows per 16-byte read group),
//    the K-contiguous stores (8 chunks of one row) and the transposing
//    MN-contiguous stores (8 rows of one chunk) free of bank conflicts.
//  * Global -> LDS staging goes through registers with two LDS buffers: the
//    next stage's global loads are issued before the current stage's MFMAs and
//    written to the other buffer afterwards, one barrier per stage.
//  * Operands whose K is contiguous load 16-byte vectors; operands whose M/N
//    is contiguous (nn.Linear's W^T stored [K,N], or a transposed view) load
//    16-byte vectors along M/N and transpose VEC x VEC blocks in registers;
//    anything else uses element loads.
//  * Waves compute 32x32 MFMA blocks: v_mfma_f32_32x32x2_f32 (IEEE fp32 path)
//    or v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation.
//  * The epilogue rounds to the output dtype, adds the bias in fp32, rounds
//    again, applies GELU (erf or tanh) or clamp_min(x,0) in registers and
//    stores once.
//  * Workgroup ids are remapped so each XCD (8 per MI355X, each with its own
//    L2) works on a contiguous, M-grouped block of output tiles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace forgeml {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum : int { MODE_K = 0, MODE_MN = 1, MODE_G = 2 };
enum : int { ACT_NONE = 0, ACT_GELU_ERF = 1, ACT_GELU_TANH = 2, ACT_RELU = 3 };

constexpr int kRowBytes = 128;  // bytes of K per LDS row and per stage

struct GemmArgs {
  const char* a;
  const char* b;
  const char* bias;
  char* c;
  int64_t sam, sak;  // A element strides (m, k)
  int64_t sbk, sbn;  // B element strides (k, n)
  int64_t sbi;       // bias element stride
  int m, n, k;
  int act;
  int has_bias;
  int tiles_m, tiles_n;
  int group_m;
};

template <int DT>
struct DTraits {
  static constexpr int ESZ = DT == DT_F32 ? 4 : 2;
  static constexpr int VEC = 16 / ESZ;         // elements per 16-byte vector
  static constexpr int BKE = kRowBytes / ESZ;  // K elements per stage
};

// Byte offset of logical 16-byte chunk `c` of LDS row `r`.
__device__ __forceinline__ int lds_off(int r, int c) {
  return r * kRowBytes + (((c ^ r ^ (r >> 3)) & 7) << 4);
}

// ---------------------------------------------------------------------------
// Element conversions.  bf16 rounding is round-to-nearest-even with NaN kept
// quiet, the rounding torch's `.to(torch.bfloat16)` performs.
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits);
  return (float)h;
}
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const char* p) {
  if constexpr (DT == DT_F32) return *(const float*)p;
  else if constexpr (DT == DT_BF16) return bf16_to_f32(*(const uint16_t*)p);
  else return f16_to_f32(*(const uint16_t*)p);
}

// Round a float to the output dtype and back (identity for fp32).
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == DT_F32) return v;
  else if constexpr (DT == DT_BF16) return bf16_to_f32(f32_to_bf16(v));
  else return (float)(_Float16)v;
}

template <int DT>
__device__ __forceinline__ void store_from_f32(char* p, float v) {
  if constexpr (DT == DT_F32) *(float*)p = v;
  else if constexpr (DT == DT_BF16) *(uint16_t*)p = (uint16_t)f32_to_bf16(v);
  else *(uint16_t*)p = (uint16_t)f32_to_f16(v);
}

// GELU from its definition: x/2 (1 + erf(x/sqrt 2)), and the tanh form
// x/2 (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).  erff/tanhf are ROCm's OCML.
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}
__device__ __forceinline__ float gelu_tanh(float x) {
  const float inner = 0.79788456080286535588f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}
__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == ACT_GELU_ERF) return gelu_erf(v);
  if (act == ACT_GELU_TANH) return gelu_tanh(v);
  if (act == ACT_RELU) return v < 0.0f ? 0.0f : v;  // clamp_min keeps NaN
  return v;
}

// ---------------------------------------------------------------------------
// Operand stage loaders.  An operand is viewed as ROWS x K with element
// (r, k) at base + (r*s_mn + k*s_k) elements: A is (M rows, sam, sak), B is
// (N rows, sbn, sbk).  load(kt) fetches stage kt from global memory into
// registers, store(lds) writes it into one LDS buffer.

// K contiguous: 16-byte vectors along K, 8 per LDS row.
template <int DT, int ROWS, int NT>
struct LoaderK {
  static constexpr int UNITS = ROWS * 8;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  const char* base;
  int64_t ld_bytes;
  int row0, rows, kbytes;
  u32x4 v[PER];

  __device__ void init(const char* b, int64_t s_mn, int64_t /*s_k*/, int r0, int nrows, int k) {
    base = b;
    ld_bytes = s_mn * DTraits<DT>::ESZ;
    row0 = r0;
    rows = nrows;
    kbytes = k * DTraits<DT>::ESZ;
  }
  __device__ __forceinline__ void load(int kt) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = threadIdx.x + i * NT;
      const int r = q >> 3, c = q & 7;
      const int kb = kt * kRowBytes + c * 16;
      const bool ok = (UNITS % NT == 0 || q < UNITS) && (row0 + r < rows) && (kb < kbytes);
      u32x4 z = {0u, 0u, 0u, 0u};
      v[i] = ok ? *(const u32x4*)(base + (int64_t)(row0 + r) * ld_bytes + kb) : z;
    }
  }
  __device__ __forceinline__ void store(char* lds) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = threadIdx.x + i * NT;
      if (UNITS % NT == 0 || q < UNITS) {
        const int r = q >> 3, c = q & 7;
        *(u32x4*)(lds + lds_off(r, c)) = v[i];
      }
    }
  }
};

// M/N contiguous: each unit is VEC rows x VEC K values, fetched as VEC
// 16-byte vectors along M/N (one per K value) and transposed in registers
// into one 16-byte LDS chunk per row.
template <int DT, int ROWS, int NT>
struct LoaderMN {
  static constexpr int ESZ = DTraits<DT>::ESZ;
  static constexpr int VEC = DTraits<DT>::VEC;
  static constexpr int UM = ROWS / VEC;
  static constexpr int UNITS = UM * 8;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  const char* base;
  int64_t ld_bytes;  // bytes between consecutive K
  int row0, rows, k;
  u32x4 v[PER][VEC];

  __device__ void init(const char* b, int64_t /*s_mn*/, int64_t s_k, int r0, int nrows, int kk) {
    base = b;
    ld_bytes = s_k * ESZ;
    row0 = r0;
    rows = nrows;
    k = kk;
  }
  __device__ __forceinline__ void load(int kt) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = threadIdx.x + i * NT;
      const int u = q % UM, g = q / UM;
      const int mn = row0 + u * VEC;
      const bool okq = (UNITS % NT == 0 || q < UNITS) && mn < rows;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int kk = kt * DTraits<DT>::BKE + g * VEC + j;
        const bool ok = okq && kk < k;
        u32x4 z = {0u, 0u, 0u, 0u};
        v[i][j] = ok ? *(const u32x4*)(base + (int64_t)kk * ld_bytes + (int64_t)mn * ESZ) : z;
      }
    }
  }
  __device__ __forceinline__ void store(char* lds) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = threadIdx.x + i * NT;
      if (UNITS % NT == 0 || q < UNITS) {
        const int u = q % UM, g = q / UM;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          u32x4 w;
          if constexpr (ESZ == 4) {
            w[0] = v[i][0][e];
            w[1] = v[i][1][e];
            w[2] = v[i][2][e];
            w[3] = v[i][3][e];
          } else {
            const int word = e >> 1;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const uint32_t lo = v[i][2 * d][word];
              const uint32_t hi = v[i][2 * d + 1][word];
              w[d] = (e & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
            }
          }
          const int r = u * VEC + e;
          *(u32x4*)(lds + lds_off(r, g)) = w;
        }
      }
    }
  }
};

// Any strides: element loads, issued when the stage is written to LDS.
// Consecutive threads walk the operand's smaller stride for coalescing.
template <int DT, int ROWS, int NT>
struct LoaderG {
  static constexpr int ESZ = DTraits<DT>::ESZ;
  static constexpr int BKE = DTraits<DT>::BKE;
  static constexpr int ELEMS = ROWS * BKE;
  static constexpr int PER = (ELEMS + NT - 1) / NT;
  static constexpr int BATCH = 16;
  const char* base;
  int64_t s_mn, s_k;
  int row0, rows, k, kt_pending;
  bool mn_fast;

  __device__ void init(const char* b, int64_t smn, int64_t sk, int r0, int nrows, int kk) {
    base = b;
    s_mn = smn;
    s_k = sk;
    row0 = r0;
    rows = nrows;
    k = kk;
    kt_pending = 0;
    const int64_t amn = smn < 0 ? -smn : smn, ak = sk < 0 ? -sk : sk;
    mn_fast = nrows > 1 && (k == 1 || amn < ak);
  }
  __device__ __forceinline__ void load(int kt) { kt_pending = kt; }
  __device__ __forceinline__ void store(char* lds) {
    const int kt = kt_pending;
#pragma unroll
    for (int i0 = 0; i0 < PER; i0 += BATCH) {
      uint32_t val[BATCH];
      int off[BATCH];
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const int e = threadIdx.x + (i0 + j) * NT;
        int r, kk;
        if (mn_fast) {
          r = e % ROWS;
          kk = e / ROWS;
        } else {
          r = e / BKE;
          kk = e % BKE;
        }
        const int gk = kt * BKE + kk;
        const bool ok = (ELEMS % NT == 0 || e < ELEMS) && (i0 + j < PER) && row0 + r < rows && gk < k;
        const char* p = base + ((int64_t)(row0 + r) * s_mn + (int64_t)gk * s_k) * ESZ;
        if constexpr (ESZ == 4) val[j] = ok ? *(const uint32_t*)p : 0u;
        else val[j] = ok ? (uint32_t)(*(const uint16_t*)p) : 0u;
        const int bytek = kk * ESZ;
        off[j] = (ELEMS % NT == 0 || e < ELEMS) && (i0 + j < PER) ? lds_off(r, bytek >> 4) + (bytek & 15) : -1;
      }
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        if (off[j] >= 0) {
          if constexpr (ESZ == 4) *(uint32_t*)(lds + off[j]) = val[j];
          else *(uint16_t*)(lds + off[j]) = (uint16_t)val[j];
        }
      }
    }
  }
};

template <int MODE, int DT, int ROWS, int NT>
struct LoaderSel;
template <int DT, int ROWS, int NT>
struct LoaderSel<MODE_K, DT, ROWS, NT> { using type = LoaderK<DT, ROWS, NT>; };
template <int DT, int ROWS, int NT>
struct LoaderSel<MODE_MN, DT, ROWS, NT> { using type = LoaderMN<DT, ROWS, NT>; };
template <int DT, int ROWS, int NT>
struct LoaderSel<MODE_G, DT, ROWS, NT> { using type = LoaderG<DT, ROWS, NT>; };

// ---------------------------------------------------------------------------
// MFMA over one LDS stage.  Lane l of a wave covers M (or N) index l%32 of a
// 32x32 block and K half h = l/32: it reads logical chunks 4h..4h+3 of its row.
// Both operands use the same K assignment, so each 32x32 accumulator receives
// the full 128-byte K slice.
template <int DT, int TM, int TN>
__device__ __forceinline__ void mfma_stage(const char* lda, const char* ldb, f32x16 (&acc)[TM][TN],
                                           int wr0, int wc0, int lane) {
  const int lr = lane & 31, h = lane >> 5;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int c = h * 4 + s;
    u32x4 af[TM], bfr[TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) af[tm] = *(const u32x4*)(lda + lds_off(wr0 + tm * 32 + lr, c));
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) bfr[tn] = *(const u32x4*)(ldb + lds_off(wc0 + tn * 32 + lr, c));
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        if constexpr (DT == DT_F32) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(af[tm][j]),
                                                               __uint_as_float(bfr[tn][j]),
                                                               acc[tm][tn], 0, 0, 0);
        } else if constexpr (DT == DT_BF16) {
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[tm]),
                                                                __builtin_bit_cast(bf16x8, bfr[tn]),
                                                                acc[tm][tn], 0, 0, 0);
        } else {
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, af[tm]),
                                                               __builtin_bit_cast(f16x8, bfr[tn]),
                                                               acc[tm][tn], 0, 0, 0);
        }
      }
    }
  }
}

// Output tile of this workgroup: XCD-contiguous, then grouped along M.
__device__ __forceinline__ void tile_coords(const GemmArgs& p, int& pm, int& pn) {
  const int nwg = p.tiles_m * p.tiles_n;
  const int b = blockIdx.x;
  const int xcd = b & 7, local = b >> 3;
  const int full = nwg >> 3, rem = nwg & 7;
  const int lin = xcd * full + (xcd < rem ? xcd : rem) + local;
  const int per_group = p.group_m * p.tiles_n;
  const int g = lin / per_group;
  const int first_m = g * p.group_m;
  const int left = p.tiles_m - first_m;
  const int gsz = left < p.group_m ? left : p.group_m;
  const int in = lin - g * per_group;
  pm = first_m + in % gsz;
  pn = in / gsz;
}

// Orders this wave's LDS writes before its later LDS reads (and vice versa)
// when lanes exchange data through LDS without a workgroup barrier.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Fused epilogue for one wave's TM x TN blocks of 32x32 accumulators.
//
// Accumulator element i of a block sits at row 8*(i/4) + 4*(lane/32) + i%4
// and column lane%32.  Each band of TN blocks (32 rows) is written to the
// wave's own slice of the (now idle) LDS, then read back so that every lane
// owns 16 output bytes of one row: the epilogue math runs in a short loop and
// the stores are 16-byte vectors along rows.  LDS accesses of one wave
// complete in program order, so the slice needs no barrier.
//
// Order of operations follows the reference kernel (src/forgeml/_triton.py:
// 43-57): round to the output dtype, add the bias in fp32, round again,
// activate, store.
template <int DT, int ACT, int TM, int TN>
__device__ __forceinline__ void epilogue(const GemmArgs& p, const f32x16 (&acc)[TM][TN], float* buf,
                                         int row_base, int col_base, int lane) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int EPV = 16 / ESZ;          // output elements per lane per step
  constexpr int CPR = 32 / EPV;          // lane-chunks per 32-column block row
  constexpr int STEPS = TN * 32 * CPR / 64;
  const int lr = lane & 31, h = lane >> 5;
  const bool vec_ok = (p.n % EPV) == 0 && (((uintptr_t)p.c) & 15) == 0;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int i = 0; i < 16; ++i) buf[(tn * 32 + 8 * (i >> 2) + 4 * h + (i & 3)) * 32 + lr] = acc[tm][tn][i];
    wave_sync();
#pragma unroll 2
    for (int st = 0; st < STEPS; ++st) {
      const int q = st * 64 + lane;
      const int tn = q / (32 * CPR);
      const int r = (q / CPR) & 31;
      const int c0 = (q % CPR) * EPV;
      const int row = row_base + tm * 32 + r;
      const int col = col_base + tn * 32 + c0;
      float v[EPV];
#pragma unroll
      for (int j = 0; j < EPV; j += 4) {
        const float4 f = *(const float4*)&buf[(tn * 32 + r) * 32 + c0 + j];
        v[j] = f.x;
        v[j + 1] = f.y;
        v[j + 2] = f.z;
        v[j + 3] = f.w;
      }
#pragma unroll
      for (int j = 0; j < EPV; ++j) {
        float x = round_to<DT>(v[j]);
        if (p.has_bias && col + j < p.n) x = round_to<DT>(x + load_as_f32<DT>(p.bias + (int64_t)(col + j) * p.sbi * ESZ));
        v[j] = apply_act(x, ACT);
      }
      if (row < p.m) {
        char* dst = p.c + ((int64_t)row * p.n + col) * ESZ;
        if (vec_ok && col + EPV <= p.n) {
          u32x4 w;
          if constexpr (ESZ == 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = __float_as_uint(v[j]);
          } else if constexpr (DT == DT_BF16) {
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = f32_to_bf16(v[2 * j]) | (f32_to_bf16(v[2 * j + 1]) << 16);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = f32_to_f16(v[2 * j]) | (f32_to_f16(v[2 * j + 1]) << 16);
          }
          *(u32x4*)dst = w;
        } else {
#pragma unroll
          for (int j = 0; j < EPV; ++j)
            if (col + j < p.n) store_from_f32<DT>(dst + j * ESZ, v[j]);
        }
      }
    }
    wave_sync();
  }
}

// ---------------------------------------------------------------------------
template <int DT, int BM, int BN, int WM, int WN, int AMODE, int BMODE>
__global__ __launch_bounds__(WM* WN * 64) void fused_gemm_kernel(GemmArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int TM = BM / (WM * 32);
  constexpr int TN = BN / (WN * 32);
  constexpr int STAGE = (BM + BN) * kRowBytes;
  static_assert(TM * WM * 32 == BM && TN * WN * 32 == BN, "tile must split into 32x32 blocks");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  int pm, pn;
  tile_coords(p, pm, pn);
  const int row0 = pm * BM, col0 = pn * BN;

  typename LoaderSel<AMODE, DT, BM, NT>::type la;
  typename LoaderSel<BMODE, DT, BN, NT>::type lb;
  la.init(p.a, p.sam, p.sak, row0, p.m, p.k);
  lb.init(p.b, p.sbn, p.sbk, col0, p.n, p.k);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr0 = (wave / WN) * (TM * 32);
  const int wc0 = (wave % WN) * (TN * 32);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[tm][tn][i] = 0.0f;

  const int nk = (p.k * ESZ + kRowBytes - 1) / kRowBytes;
  la.load(0);
  lb.load(0);
  la.store(smem);
  lb.store(smem + BM * kRowBytes);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    char* cur = smem + (kt & 1) * STAGE;
    char* nxt = smem + ((kt + 1) & 1) * STAGE;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(kt + 1);
      lb.load(kt + 1);
    }
    mfma_stage<DT, TM, TN>(cur, cur + BM * kRowBytes, acc, wr0, wc0, lane);
    if (more) {
      la.store(nxt);
      lb.store(nxt + BM * kRowBytes);
    }
    __syncthreads();
  }

  // The last loop iteration ended with a barrier, so all of LDS is free.
  static_assert(WM * WN * TN * 32 * 32 * 4 <= 2 * STAGE, "epilogue slices must fit in LDS");
  float* buf = (float*)(smem + wave * (TN * 32 * 32 * 4));
  const int row_base = row0 + wr0, col_base = col0 + wc0;
  switch (p.act) {
    case ACT_GELU_ERF: epilogue<DT, ACT_GELU_ERF, TM, TN>(p, acc, buf, row_base, col_base, lane); break;
    case ACT_GELU_TANH: epilogue<DT, ACT_GELU_TANH, TM, TN>(p, acc, buf, row_base, col_base, lane); break;
    case ACT_RELU: epilogue<DT, ACT_RELU, TM, TN>(p, acc, buf, row_base, col_base, lane); break;
    default: epilogue<DT, ACT_NONE, TM, TN>(p, acc, buf, row_base, col_base, lane); break;
  }
}

}  // namespace forgeml
