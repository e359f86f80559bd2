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
//    or v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation; four-wave
//    16-bit tiles up to 128x128 with both operands K-contiguous use 16x16
//    blocks of v_mfma_f32_16x16x32_{bf16,f16}, whose LDS rows use a swizzle
//    that repeats every 16 rows.
//  * The epilogue rounds to the output dtype, adds the bias in fp32, rounds
//    again, applies GELU (erf or tanh; for bf16 on the 8-wave 256x256 tile
//    from a table of its values in LDS) or clamp_min(x,0) in registers and
//    stores once.
//  * Workgroup ids are remapped so each XCD (8 per MI355X, each with its own
//    L2) works on a contiguous, M-grouped block of output tiles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace forgeml {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum : int { MODE_K = 0, MODE_MN = 1, MODE_G = 2, MODE_K4 = 3 };
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
  // Optional residual R[M,N] (element (m,n) at res + m*srm + n*srn elements),
  // added to the rounded activation: C = rnd(rnd(act(...)) + R), as an add
  // kernel reading the GEMM's output would compute.  res may equal c.
  const char* res;
  int64_t srm, srn;
  int tiles_m, tiles_n;
  int group_m;
  // Split K: `splits` workgroups share each output tile, slice z covering
  // stages [z*kslice, (z+1)*kslice).  With splits > 1 each slice stores its
  // raw fp32 sums to ws[z][M][N] and splitk_reduce_kernel applies the
  // epilogue.  splits == 1: kslice is the whole K, ws is unused.
  int splits, kslice;
  float* ws;
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

// Swizzle of the 16x16x32 MFMA path: (r & 7) ^ ((r >> 3) & 1) repeats every
// 16 rows, so all fragments of a step (16-row blocks) sit at one per-lane base
// plus immediate offsets; 8 consecutive rows of one chunk still cover 8
// distinct 16-byte bank groups, and 16 rows 16 groups of a 256-byte line.
__device__ __forceinline__ int lds_swz16(int r) {
  return (r & 7) ^ ((r >> 3) & 1);
}
__device__ __forceinline__ int lds_off16(int r, int c) {
  return r * kRowBytes + ((c ^ lds_swz16(r)) << 4);
}

// ---------------------------------------------------------------------------
// Element conversions.
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits);
  return (float)h;
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const char* p) {
  if constexpr (DT == DT_F32) return *(const float*)p;
  else if constexpr (DT == DT_BF16) return bf16_to_f32(*(const uint16_t*)p);
  else return f16_to_f32(*(const uint16_t*)p);
}

// Residual value (row, col) as fp32.
template <int DT>
__device__ __forceinline__ float residual_at(const GemmArgs& p, int row, int col) {
  return load_as_f32<DT>(p.res + ((int64_t)row * p.srm + (int64_t)col * p.srn) * DTraits<DT>::ESZ);
}

// Round a float to the output dtype and back (identity for fp32).  gfx950
// converts fp32 -> bf16 in hardware (v_cvt_pk_bf16_f32, round to nearest even).
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == DT_F32) return v;
  else if constexpr (DT == DT_BF16) return (float)(__bf16)v;
  else return (float)(_Float16)v;
}

template <int DT>
__device__ __forceinline__ void store_from_f32(char* p, float v) {
  if constexpr (DT == DT_F32) *(float*)p = v;
  else if constexpr (DT == DT_BF16) *(__bf16*)p = (__bf16)v;
  else *(_Float16*)p = (_Float16)v;
}

// Two floats packed into one dword of the 16-bit output dtype.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  if constexpr (DT == DT_BF16) {
    typedef __bf16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
  }
}

// GELU, x/2 (1 + erf(x/sqrt 2)) and its tanh form
// x/2 (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), in forms accurate to a few
// fp32 ulps relative to the result everywhere: far inside the 16-bit output
// rounding (2^-9 relative for bf16, 2^-11 for fp16), and inside fp32 parity
// by three orders of magnitude, at about half the instructions of the
// library erff/tanhf (the transformer block's FFN up GEMM, 4096x3072x768
// fp32, 157 -> 147 us).
//  * erf GELU = x * Phi(x), with Phi(-|x|) = erfc(|x|/sqrt 2)/2 from the
//    Chebyshev fit of Press et al., Numerical Recipes in C (2nd ed.), 6.2
//    ("erfcc"): erfc(z) = t exp(-z^2 + P(t)), t = 1/(1 + z/2), P a degree-9
//    polynomial, relative error below 1.2e-7 for every z >= 0.  A relative
//    bound matters in the negative tail, where x Phi(x) is small: an
//    absolute-error fit (Abramowitz & Stegun 7.1.26) is off there by up to
//    4 % of the result, and 1 + erf cancels.
//  * tanh GELU = x * sigmoid(2u) = x / (1 + exp(-2u)), an identity of the
//    tanh form that avoids 1 + tanh(u) cancelling for negative x.
__device__ __forceinline__ float gelu_erf(float x) {
  const float z = fabsf(x) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = fmaf(0.17087277f, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  p = fmaf(p, t, -1.26551223f);
  const float q = 0.5f * t * __expf(fmaf(-z, z, p));  // Phi(-|x|)
  return x * (x >= 0.0f ? 1.0f - q : q);
}
__device__ __forceinline__ float gelu_tanh(float x) {
  const float u = 0.79788456080286535588f * fmaf(0.044715f * x, x * x, x);
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * u));
}

template <int DT, int ACT>
__device__ __forceinline__ float activate(float v) {
  if constexpr (ACT == ACT_GELU_ERF) return gelu_erf(v);
  else if constexpr (ACT == ACT_GELU_TANH) return gelu_tanh(v);
  else if constexpr (ACT == ACT_RELU) return v < 0.0f ? 0.0f : v;  // clamp_min keeps NaN
  else return v;
}

// GELU of bf16 values by table.  The activation's input is itself a bf16
// value (the bias sum is rounded first), so a tile with many outputs per
// workgroup (the 8-wave 256x256 tile: 65536; the 4-wave one has no
// registers to spare beside its accumulators) evaluates the activation once per
// bf16 input of magnitude in [2^-16, 16), either sign (20 binades of 128
// mantissas), into LDS, rounded to bf16 as the store would round it, and
// its epilogue looks the outputs up: the same bits as evaluating each one,
// for about a quarter of the vector ALU work.  Inputs outside the table
// (magnitudes below 2^-16 or from 16 up, zeros, infinities, NaN) take the
// arithmetic path.  Entry i: sign i / kLutSpan, bf16 exponent and mantissa
// bits (kLutLoExp << 7) + i % kLutSpan.
constexpr int kLutLoExp = 127 - 16;
constexpr int kLutSpan = 20 * 128;
constexpr int kLutBytes = 2 * kLutSpan * 2;

template <int DT, int BM, int BN, int WAVES>
constexpr bool gelu_lut_tile() {
  return DT == DT_BF16 && BM * BN >= 256 * 256 && WAVES == 8;
}

__device__ __forceinline__ uint16_t bf16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}

template <int ACT>
__device__ __forceinline__ void build_gelu_lut(uint16_t* lut, int tid, int nt) {
  for (int i = tid; i < 2 * kLutSpan; i += nt) {
    const int neg = i >= kLutSpan;
    const uint32_t bits = ((uint32_t)neg << 15) | (((uint32_t)kLutLoExp << 7) + (uint32_t)(i - neg * kLutSpan));
    lut[i] = bf16_bits(activate<DT_BF16, ACT>(bf16_to_f32(bits)));
  }
}

// Table index of bf16 value x (held in a float), and whether it is inside.
__device__ __forceinline__ bool gelu_lut_index(float x, uint32_t& idx) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t t = ((u >> 16) & 0x7fffu) - ((uint32_t)kLutLoExp << 7);
  idx = t + (u >> 31) * (uint32_t)kLutSpan;
  return t < (uint32_t)kLutSpan;
}

// ---------------------------------------------------------------------------
// Operand stage loaders.  An operand is viewed as ROWS x K with element
// (r, k) at base + (r*s_mn + k*s_k) elements: A is (M rows, sam, sak), B is
// (N rows, sbn, sbk).  Each loader fetches one 128-byte-K stage:
//   issue(kt, stage)  starts the global reads of stage kt;
//   commit(stage)     finishes writing it into an LDS buffer.
// Direct loaders (kDirect) DMA global memory straight into LDS in issue()
// and need only a vmcnt wait before the barrier; the others stage through
// registers and write LDS in commit().
//
// Global reads go through buffer resources: a lane whose element is outside
// the operand (M/N edge or K tail) gets an offset past the resource's range
// and the hardware returns zeros, with no branch and no select on the data.

constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const char* base, uint32_t bytes) {
  // Word 3 0x00020000: raw (untyped) buffer access on gfx9-family GPUs.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// K contiguous: DMA 16-byte vectors along K straight into LDS.  One
// buffer_load_dwordx4 ... lds of a wave writes a contiguous 1 KB block (lane
// L at byte 16*L) = 8 LDS rows; each lane fetches the chunk whose swizzled
// LDS position is its own slot.
template <int DT, int ROWS, int NT, bool SW16 = false>
struct LoaderK {
  static constexpr bool kDirect = true;
  static constexpr int BLOCKS = ROWS / 8;
  static constexpr int NWAVES = NT / 64;
  static constexpr int PER = (BLOCKS + NWAVES - 1) / NWAVES;
  static constexpr int kGlobalLoads = PER, kLdsWrites = 0;  // per thread per stage
  static constexpr bool kExactPer = BLOCKS % NWAVES == 0;    // every wave issues PER DMAs
  // With the 16-row swizzle a lane's chunk is the same in every block it
  // loads when the wave count is even (block parity = wave parity).
  static constexpr bool kOneChunk = SW16 && NWAVES % 2 == 0;
  __amdgpu_buffer_rsrc_t rsrc;
  int kbytes;
  // This lane's byte offset in stage 0 per block, or out of range.  With one
  // chunk, only block 0's offset and row are kept: block i is i * NWAVES * 8
  // rows further (fewer registers next to the 16x16x32 path's fragments).
  uint32_t voff[kOneChunk ? 1 : PER];
  int kchunk[kOneChunk ? 1 : PER];  // byte offset of this lane's chunk within a stage
  int vrow, valid, step_bytes;      // one chunk: block 0's row; rows in range; bytes per block step

  __device__ __forceinline__ void init(const char* b, int64_t s_mn, int64_t /*s_k*/, int r0, int nrows, int k) {
    const int ld_bytes = (int)(s_mn * DTraits<DT>::ESZ);
    kbytes = k * DTraits<DT>::ESZ;
    const int valid_rows = min(ROWS, nrows - r0);
    const int64_t span = (int64_t)(valid_rows - 1) * ld_bytes + kbytes;
    rsrc = make_rsrc(b + (int64_t)r0 * s_mn * DTraits<DT>::ESZ, (uint32_t)span);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = wave + i * NWAVES;
      const int r = blk * 8 + (lane >> 3);
      // logical chunk stored at physical slot lane&7
      const int c = SW16 ? ((lane & 7) ^ lds_swz16(r)) : ((lane ^ r ^ (r >> 3)) & 7);
      if constexpr (kOneChunk) {
        if (i == 0) {
          kchunk[0] = c * 16;
          voff[0] = (uint32_t)(r * ld_bytes + c * 16);
          vrow = r;
        }
      } else {
        kchunk[i] = c * 16;
        voff[i] = (r < valid_rows && blk < BLOCKS) ? (uint32_t)(r * ld_bytes + c * 16) : kOutOfRange;
      }
    }
    valid = valid_rows;
    step_bytes = NWAVES * 8 * ld_bytes;
  }
  // DMAs [P0, P1) of this wave's PER for stage kt.  Stage kt's K offset goes
  // in the scalar offset; lanes past the K tail get an out-of-range vector
  // offset.
  template <int P0, int P1>
  __device__ __forceinline__ void issue_part(int kt, char* stage) {
    // The wave index is uniform: keep the LDS destination (M0) in SGPRs.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kbase = kt * kRowBytes;
    const int klimit = kbytes - kbase;
#pragma unroll
    for (int i = P0; i < P1; ++i) {
      const int blk = wave + i * NWAVES;  // uniform per wave
      if (BLOCKS % NWAVES == 0 || blk < BLOCKS) {
        uint32_t off;
        if constexpr (kOneChunk) {
          const bool ok = vrow + i * NWAVES * 8 < valid && blk < BLOCKS && kchunk[0] < klimit;
          off = ok ? voff[0] + (uint32_t)(i * step_bytes) : kOutOfRange;
        } else {
          off = kchunk[i] < klimit ? voff[i] : kOutOfRange;
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(stage + blk * 1024), 16, off, kbase, 0, 0);
      }
    }
  }
  __device__ __forceinline__ void issue(int kt, char* stage) { issue_part<0, PER>(kt, stage); }
  __device__ __forceinline__ void commit(char*) {}
};

// K contiguous with rows only 4-byte aligned (e.g. an odd fp32 K): DMA one
// dword per lane.  A wave's buffer_load_dword ... lds writes 256 contiguous
// LDS bytes = 2 rows; lane L lands at byte 4*L, i.e. row L/32, physical chunk
// (L%32)/4, dword L%4, and fetches the dword of the logical chunk stored
// there.  For row pair `blk` (rows 2blk, 2blk+1) the swizzle term
// (r ^ r>>3) & 7 is (2blk ^ blk>>2 ^ L/32) & 7, so a lane's chunk is its own
// constant XOR a wave-uniform value, and the row pair's base offset goes in
// the scalar offset with the stage's K offset.
template <int DT, int ROWS, int NT>
struct LoaderK4 {
  static constexpr bool kDirect = true;
  static constexpr int BLOCKS = ROWS / 2;
  static constexpr int NWAVES = NT / 64;
  static constexpr int PER = (BLOCKS + NWAVES - 1) / NWAVES;
  static constexpr int kGlobalLoads = PER, kLdsWrites = 0;
  static constexpr bool kExactPer = BLOCKS % NWAVES == 0;
  __amdgpu_buffer_rsrc_t rsrc;
  int kbytes, ld_bytes, valid_rows;
  int lane_off;  // (L/32)*ld_bytes + (L%4)*4
  int lane_c;    // ((L%32)/4 ^ L/32) & 7
  int lane_dw;   // (L%4)*4
  int lane_r;    // L/32

  __device__ __forceinline__ void init(const char* b, int64_t s_mn, int64_t /*s_k*/, int r0, int nrows, int k) {
    ld_bytes = (int)(s_mn * DTraits<DT>::ESZ);
    kbytes = k * DTraits<DT>::ESZ;
    valid_rows = min(ROWS, nrows - r0);
    const int64_t span = (int64_t)(valid_rows - 1) * ld_bytes + kbytes;
    rsrc = make_rsrc(b + (int64_t)r0 * s_mn * DTraits<DT>::ESZ, (uint32_t)span);
    const int lane = threadIdx.x & 63;
    lane_r = lane >> 5;
    lane_dw = (lane & 3) * 4;
    lane_off = lane_r * ld_bytes + lane_dw;
    lane_c = (((lane & 31) >> 2) ^ lane_r) & 7;
  }
  __device__ __forceinline__ void issue(int kt, char* stage) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kbase = kt * kRowBytes;
    const int klimit = kbytes - kbase;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = wave + i * NWAVES;  // uniform per wave
      if (BLOCKS % NWAVES == 0 || blk < BLOCKS) {
        const int cb = ((lane_c ^ (2 * blk) ^ (blk >> 2)) & 7) * 16;
        const bool ok = 2 * blk + lane_r < valid_rows && cb + lane_dw < klimit;
        const uint32_t off = ok ? (uint32_t)(lane_off + cb) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(stage + blk * 256), 4, off,
                                                 kbase + 2 * blk * ld_bytes, 0, 0);
      }
    }
  }
  __device__ __forceinline__ void commit(char*) {}
};

// M/N contiguous: each unit is VEC rows x VEC K values, fetched as VEC
// 16-byte vectors along M/N (one per K value) into registers and transposed
// there into one 16-byte LDS chunk per row.
template <int DT, int ROWS, int NT>
struct LoaderMN {
  static constexpr bool kDirect = false;
  static constexpr int ESZ = DTraits<DT>::ESZ;
  static constexpr int VEC = DTraits<DT>::VEC;
  static constexpr int UM = ROWS / VEC;
  static constexpr int UNITS = UM * 8;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int kGlobalLoads = PER * VEC, kLdsWrites = PER * VEC;
  static constexpr bool kExactPer = false;
  __amdgpu_buffer_rsrc_t rsrc;
  int ld_bytes, k, valid;  // ld_bytes: bytes between consecutive K
  u32x4 v[PER][VEC];

  __device__ __forceinline__ void init(const char* b, int64_t /*s_mn*/, int64_t s_k, int r0, int nrows, int kk) {
    ld_bytes = (int)(s_k * ESZ);
    k = kk;
    valid = min(ROWS, nrows - r0);
    const int64_t span = (int64_t)(kk - 1) * ld_bytes + (int64_t)valid * ESZ;
    rsrc = make_rsrc(b + (int64_t)r0 * ESZ, (uint32_t)span);
  }
  __device__ __forceinline__ void issue(int kt, char*) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = threadIdx.x + i * NT;
      const int u = q % UM, g = q / UM;
      const bool okq = (UNITS % NT == 0 || q < UNITS) && u * VEC < valid;  // valid % VEC == 0 here
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int kk = kt * DTraits<DT>::BKE + g * VEC + j;
        const uint32_t off = (okq && kk < k) ? (uint32_t)(kk * ld_bytes + u * VEC * ESZ) : kOutOfRange;
        v[i][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, 0, 0));
      }
    }
  }
  __device__ __forceinline__ void commit(char* lds) {
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

// Any strides: element loads.  Consecutive threads walk the operand's
// smaller stride for coalescing; either way a thread's elements of a stage lie
// on one line of the stage, (r0 + i*dr, kk0 + i*dk), because the thread count
// is a multiple of both ROWS and the stage's K extent.  Up to 32 elements per
// thread are held in registers from issue() to commit(), so the loads overlap
// the MFMAs like the vector loaders'; larger tiles load in commit().
template <int DT, int ROWS, int NT>
struct LoaderG {
  static constexpr bool kDirect = false;
  static constexpr int ESZ = DTraits<DT>::ESZ;
  static constexpr int BKE = DTraits<DT>::BKE;
  static constexpr int ELEMS = ROWS * BKE;
  static constexpr int PER = ELEMS / NT;
  static constexpr bool kStaged = PER <= 16;
  static constexpr int BATCH = 16;
  static constexpr int kGlobalLoads = kStaged ? PER : 0, kLdsWrites = kStaged ? PER : 0;
  static constexpr bool kExactPer = false;
  static_assert(ELEMS % NT == 0 && NT % ROWS == 0 && NT % BKE == 0, "thread count must tile the stage");
  const char* safe;      // element (row0, 0): always inside the operand
  const char* p0;        // this thread's first element of stage 0
  int64_t step_bytes;    // between a thread's consecutive elements of a stage
  int64_t stage_bytes;   // between stages (BKE * s_k elements)
  int r0, kk0, dr, dk, rows_left, k;
  int kt_pending;
  // Staged values; 16-bit elements are packed two to a register.
  static constexpr int NVAL = kStaged ? (ESZ == 4 ? PER : (PER + 1) / 2) : 1;
  uint32_t val[NVAL];

  __device__ __forceinline__ void init(const char* b, int64_t smn, int64_t sk, int row0, int nrows, int kk) {
    const int64_t amn = smn < 0 ? -smn : smn, ak = sk < 0 ? -sk : sk;
    const bool mn_fast = nrows > 1 && (kk == 1 || amn < ak);
    const int t = threadIdx.x;
    if (mn_fast) {
      r0 = t % ROWS;
      kk0 = t / ROWS;
      dr = 0;
      dk = NT / ROWS;
    } else {
      r0 = t / BKE;
      kk0 = t % BKE;
      dr = NT / BKE;
      dk = 0;
    }
    safe = b + (int64_t)row0 * smn * ESZ;
    p0 = b + ((int64_t)(row0 + r0) * smn + (int64_t)kk0 * sk) * ESZ;
    step_bytes = ((int64_t)dr * smn + (int64_t)dk * sk) * ESZ;
    stage_bytes = (int64_t)BKE * sk * ESZ;
    rows_left = nrows - row0;
    k = kk;
    kt_pending = 0;
  }
  // Branch-free: a lane outside the operand reads the always-valid element
  // and discards it.
  __device__ __forceinline__ uint32_t fetch(int i, int kt) const {
    const bool ok = r0 + i * dr < rows_left && kt * BKE + kk0 + i * dk < k;
    const char* p = ok ? p0 + kt * stage_bytes + i * step_bytes : safe;
    uint32_t v;
    if constexpr (ESZ == 4) v = *(const uint32_t*)p;
    else v = *(const uint16_t*)p;
    return ok ? v : 0u;
  }
  __device__ __forceinline__ void put(char* lds, int i, uint32_t v) const {
    const int bytek = (kk0 + i * dk) * ESZ;
    char* dst = lds + lds_off(r0 + i * dr, bytek >> 4) + (bytek & 15);
    if constexpr (ESZ == 4) *(uint32_t*)dst = v;
    else *(uint16_t*)dst = (uint16_t)v;
  }
  __device__ __forceinline__ void issue(int kt, char*) {
    if constexpr (kStaged) {
      if constexpr (ESZ == 4) {
#pragma unroll
        for (int i = 0; i < PER; ++i) val[i] = fetch(i, kt);
      } else {
#pragma unroll
        for (int i = 0; i < PER; i += 2)
          val[i / 2] = fetch(i, kt) | (i + 1 < PER ? fetch(i + 1, kt) << 16 : 0u);
      }
    } else {
      kt_pending = kt;
    }
  }
  __device__ __forceinline__ void commit(char* lds) {
    if constexpr (kStaged) {
#pragma unroll
      for (int i = 0; i < PER; ++i) put(lds, i, ESZ == 4 ? val[i] : (val[i / 2] >> (16 * (i & 1))) & 0xffffu);
    } else {
#pragma unroll
      for (int i0 = 0; i0 < PER; i0 += BATCH) {
        uint32_t v[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) v[j] = fetch(i0 + j, kt_pending);
#pragma unroll
        for (int j = 0; j < BATCH; ++j) put(lds, i0 + j, v[j]);
      }
    }
  }
};

// Most LDS stage buffers a kernel may ring through: small tiles whose
// operands both arrive by DMA stream K with little MFMA work per stage, so
// they can keep four stages in flight (64 KiB, two workgroups per CU); the
// others use two.  The launcher picks the ring per grid (launch_one).
template <int BM, int BN, int AMODE, int BMODE>
constexpr int lds_stages_max() {
  return ((AMODE == MODE_K || AMODE == MODE_K4) && (BMODE == MODE_K || BMODE == MODE_K4) && BM * BN <= 64 * 64) ? 4
                                                                                                              : 2;
}

// SW16: the operand is read by the 16x16x32 path (lds_off16 layout; K-contiguous only).
template <int MODE, int DT, int ROWS, int NT, bool SW16 = false>
struct LoaderSel;
template <int DT, int ROWS, int NT, bool SW16>
struct LoaderSel<MODE_K, DT, ROWS, NT, SW16> { using type = LoaderK<DT, ROWS, NT, SW16>; };
template <int DT, int ROWS, int NT>
struct LoaderSel<MODE_MN, DT, ROWS, NT, false> { using type = LoaderMN<DT, ROWS, NT>; };
template <int DT, int ROWS, int NT>
struct LoaderSel<MODE_G, DT, ROWS, NT, false> { using type = LoaderG<DT, ROWS, NT>; };
template <int DT, int ROWS, int NT>
struct LoaderSel<MODE_K4, DT, ROWS, NT, false> { using type = LoaderK4<DT, ROWS, NT>; };

// ---------------------------------------------------------------------------
// MFMA over one LDS stage.  Lane l of a wave covers M (or N) index l%32 of a
// 32x32 block and K half h = l/32: it reads logical chunks 4h..4h+3 of its row.
// Both operands use the same K assignment, so each 32x32 accumulator receives
// the full 128-byte K slice.  The operand fragments are double-buffered in
// registers: the LDS reads of step s+1 are in flight while the MFMAs of step
// s issue, so the matrix cores do not wait on LDS latency between steps.
template <int TM, int TN>
struct Frags {
  u32x4 a[TM];
  u32x4 b[TN];
};

// Reads are issued in the order the MFMAs (tm outer, tn inner) first use
// them, so each MFMA waits only for its own operands.
template <int TM, int TN>
__device__ __forceinline__ void load_frags(Frags<TM, TN>& f, const char* lda, const char* ldb, int wr0, int wc0,
                                           int lr, int c) {
  f.a[0] = *(const u32x4*)(lda + lds_off(wr0 + lr, c));
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) f.b[tn] = *(const u32x4*)(ldb + lds_off(wc0 + tn * 32 + lr, c));
#pragma unroll
  for (int tm = 1; tm < TM; ++tm) f.a[tm] = *(const u32x4*)(lda + lds_off(wr0 + tm * 32 + lr, c));
}

template <int DT, int TM, int TN>
__device__ __forceinline__ void mma_frags(const Frags<TM, TN>& f, f32x16 (&acc)[TM][TN]) {
  if constexpr (DT == DT_F32) {
    // The 4 K elements of the chunk outermost: consecutive MFMAs go to
    // different accumulator blocks, and each block still adds its K elements
    // in the same order (bit-identical results; about 1 % faster on 4096^3).
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(f.a[tm][j]), __uint_as_float(f.b[tn][j]),
                                                             acc[tm][tn], 0, 0, 0);
    return;
  }
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if constexpr (DT == DT_BF16) {
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, f.a[tm]),
                                                              __builtin_bit_cast(bf16x8, f.b[tn]), acc[tm][tn], 0, 0, 0);
      } else {
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, f.a[tm]),
                                                             __builtin_bit_cast(f16x8, f.b[tn]), acc[tm][tn], 0, 0, 0);
      }
    }
  }
}

// Four-wave 16-bit tiles up to 128x128 fed by DMA use
// v_mfma_f32_16x16x32_{bf16,f16} instead: a stage is two MFMA steps of 32 K
// elements, lane l covering M (or N) index l%16 of a 16x16 block and K chunk
// l/16 of the step (logical chunk 4*step + l/16 of its row).  A step is
// twice as many MFMA cycles as with the 32x32 shape (32 K instead of 16) for
// the same LDS bytes per K, so the next step's fragment reads have twice as
// long to return; its fragments take twice the registers.  TM and TN count
// 16-row and 16-column blocks here.
// `ao`/`bo`: this lane's byte offset of the step's chunk in its first A / B
// row (lds_off16 of row wr0 + l%16 / wc0 + l%16); block t is 16 rows further.
template <int TM, int TN>
__device__ __forceinline__ void load_frags16(Frags<TM, TN>& f, const char* lda, const char* ldb, int ao, int bo) {
  f.a[0] = *(const u32x4*)(lda + ao);
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) f.b[tn] = *(const u32x4*)(ldb + bo + tn * 16 * kRowBytes);
#pragma unroll
  for (int tm = 1; tm < TM; ++tm) f.a[tm] = *(const u32x4*)(lda + ao + tm * 16 * kRowBytes);
}

template <int DT, int TM, int TN>
__device__ __forceinline__ void mma_frags(const Frags<TM, TN>& f, f32x4 (&acc)[TM][TN]) {
  static_assert(DT != DT_F32, "the 16x16x32 path is for 16-bit inputs");
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if constexpr (DT == DT_BF16) {
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, f.a[tm]),
                                                              __builtin_bit_cast(bf16x8, f.b[tn]), acc[tm][tn], 0, 0, 0);
      } else {
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, f.a[tm]),
                                                             __builtin_bit_cast(f16x8, f.b[tn]), acc[tm][tn], 0, 0, 0);
      }
    }
  }
}

// Instruction-order hints for the scheduler (masks: 0x008 MFMA, 0x100 LDS
// read, 0x200 LDS write, 0x010 any global memory access; the DMA loads count
// as both a global read and an LDS write, so they match only the generic
// mask).  Each helper lays out one MFMA step: the next step's LDS reads all
// follow the first MFMA, so they have the rest of the step to land, and the
// LDS writes and global loads are spread evenly between the MFMAs so the
// matrix pipe stays fed while memory work issues.
template <int NM, int NR, int NW, int NG>
__device__ __forceinline__ void sched_step() {
  // Each step is its own scheduling region (sched_barrier below), so the LDS
  // reads placed in it can only be the next step's fragments.
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (NR > 0) {
      if (i == 0) __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
    }
    if constexpr (NW > 0) {
#pragma unroll
      for (int j = (i * NW) / NM; j < ((i + 1) * NW) / NM; ++j) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
    if constexpr (NG > 0) {
#pragma unroll
      for (int j = (i * NG) / NM; j < ((i + 1) * NG) / NM; ++j) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Output tile and K slice of this workgroup: XCD-contiguous, the K slices of
// a tile adjacent, tiles grouped along M.
__device__ __forceinline__ void tile_coords(const GemmArgs& p, int& pm, int& pn, int& z) {
  const int nwg = p.tiles_m * p.tiles_n * p.splits;
  const int b = blockIdx.x;
  const int xcd = b & 7, local = b >> 3;
  const int full = nwg >> 3, rem = nwg & 7;
  const int lin_all = xcd * full + (xcd < rem ? xcd : rem) + local;
  const int lin = lin_all / p.splits;
  z = lin_all - lin * p.splits;
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
// wave's own slice of the (now idle) LDS and read back so that every lane
// owns EPV consecutive outputs (16 bytes) of one row: the epilogue math is
// per row segment and the stores are 16-byte vectors.  A lane's columns
// within a block are the same for every row, so its bias values are loaded
// once.  LDS accesses of one wave complete in program order; wave_sync keeps
// the compiler from reordering them.
//
// Order of operations follows the reference kernel (src/forgeml/_triton.py:
// 43-57): round to the output dtype, add the bias in fp32, round again,
// activate, store.
// Writes 32-row band `tm` of a wave's accumulators to its LDS slice as
// [32-column block][row][column] floats.  32x32 blocks: element i of lane l
// is row 8*(i/4) + 4*(l/32) + i%4, column l%32.  16x16 blocks (two per band
// row and column): element i of lane l is row 4*(l/16) + i, column l%16.
template <int TM, int TN>
__device__ __forceinline__ void write_band(const f32x16 (&acc)[TM][TN], int tm, float* buf, int lane) {
  const int lr = lane & 31, h = lane >> 5;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int i = 0; i < 16; ++i) buf[(tn * 32 + 8 * (i >> 2) + 4 * h + (i & 3)) * 32 + lr] = acc[tm][tn][i];
}
template <int TM2, int TN2>
__device__ __forceinline__ void write_band(const f32x4 (&acc)[TM2][TN2], int tm, float* buf, int lane) {
  const int c16 = lane & 15, r4 = (lane >> 4) * 4;
#pragma unroll
  for (int hm = 0; hm < 2; ++hm)
#pragma unroll
    for (int tn = 0; tn < TN2; ++tn)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        buf[((tn >> 1) * 32 + hm * 16 + r4 + i) * 32 + (tn & 1) * 16 + c16] = acc[2 * tm + hm][tn][i];
}

// STREAM: non-temporal output stores (the final C); split-K partial planes,
// which the reduce kernel reads right after, are stored plainly.
// LUT: the activation by table (gelu_lut_tile), from `lut` in LDS.
template <int DT, int ACT, int TM, int TN, bool INTERIOR, bool STREAM, bool LUT, class Acc>
__device__ __forceinline__ void epilogue(const GemmArgs& p, const Acc& acc, float* buf, int row_base, int col_base,
                                         int lane, const uint16_t* lut) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int EPV = 16 / ESZ;      // outputs per lane per row segment
  constexpr int CPR = 32 / EPV;      // lanes per 32-column block row
  constexpr int SEGS = 32 * CPR / 64;  // row segments per lane per block
  const int cq = (lane % CPR) * EPV;  // this lane's first column within a block
  const bool vec_ok = INTERIOR || ((p.n % EPV) == 0 && (((uintptr_t)p.c) & 15) == 0);
  float bias[TN][EPV];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int j = 0; j < EPV; ++j) {
      const int col = col_base + tn * 32 + cq + j;
      bias[tn][j] = (p.has_bias && (INTERIOR || col < p.n)) ? load_as_f32<DT>(p.bias + (int64_t)col * p.sbi * ESZ) : 0.0f;
    }
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    write_band(acc, tm, buf, lane);
    wave_sync();
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
      for (int sg = 0; sg < SEGS; ++sg) {
        const int r = (sg * 64 + lane) / CPR;
        const int row = row_base + tm * 32 + r;
        const int col = col_base + tn * 32 + cq;
        float v[EPV];
#pragma unroll
        for (int j = 0; j < EPV; j += 4) {
          const float4 f = *(const float4*)&buf[(tn * 32 + r) * 32 + cq + j];
          v[j] = f.x;
          v[j + 1] = f.y;
          v[j + 2] = f.z;
          v[j + 3] = f.w;
        }
        if constexpr (LUT) {
          // One table read per output when all of the lane's segment is
          // inside the table, else the arithmetic form for the segment.
          float x[EPV];
          uint32_t idx[EPV];
          bool inside = true;
#pragma unroll
          for (int j = 0; j < EPV; ++j) {
            x[j] = round_to<DT>(v[j]);
            if (p.has_bias) x[j] = round_to<DT>(x[j] + bias[tn][j]);
            inside &= gelu_lut_index(x[j], idx[j]);
          }
          if (inside) {
#pragma unroll
            for (int j = 0; j < EPV; ++j) v[j] = bf16_to_f32(lut[idx[j]]);
          } else {
#pragma unroll
            for (int j = 0; j < EPV; ++j) v[j] = round_to<DT>(activate<DT, ACT>(x[j]));
          }
        } else {
          // Activations that commute with rounding (none, relu) skip the
          // rounding of the bias sum: the store rounds, and so does the
          // residual add's first step.
          constexpr bool KEEP = ACT == ACT_NONE || ACT == ACT_RELU;
#pragma unroll
          for (int j = 0; j < EPV; ++j) {
            float x = round_to<DT>(v[j]);
            if (p.has_bias) x = KEEP ? x + bias[tn][j] : round_to<DT>(x + bias[tn][j]);
            v[j] = activate<DT, ACT>(x);
          }
        }
        if (p.res != nullptr && (INTERIOR || row < p.m)) {
          // Residual add to the rounded activation, rounded like torch's add.
          const char* rp = p.res + ((int64_t)row * p.srm + (int64_t)col * p.srn) * ESZ;
          if (p.srn == 1 && (((uintptr_t)rp) & 15) == 0 && (INTERIOR || col + EPV <= p.n)) {
            const u32x4 w = *(const u32x4*)rp;
#pragma unroll
            for (int j = 0; j < EPV; ++j) {
              const uint32_t word = w[j * ESZ / 4];
              const float r = ESZ == 4 ? __uint_as_float(word)
                                       : (DT == DT_BF16 ? bf16_to_f32((word >> (16 * (j & 1))) & 0xffffu)
                                                        : f16_to_f32((word >> (16 * (j & 1))) & 0xffffu));
              v[j] = round_to<DT>(round_to<DT>(v[j]) + r);
            }
          } else {
#pragma unroll
            for (int j = 0; j < EPV; ++j)
              if (INTERIOR || col + j < p.n) v[j] = round_to<DT>(round_to<DT>(v[j]) + residual_at<DT>(p, row, col + j));
          }
        }
        if (INTERIOR || row < p.m) {
          char* dst = p.c + ((int64_t)row * p.n + col) * ESZ;
          if (vec_ok && (INTERIOR || col + EPV <= p.n)) {
            u32x4 w;
            if constexpr (ESZ == 4) {
#pragma unroll
              for (int j = 0; j < 4; ++j) w[j] = __float_as_uint(v[j]);
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j) w[j] = pack2<DT>(v[2 * j], v[2 * j + 1]);
            }
            // Non-temporal store: the tile is written out, not kept in
            // L2 for a re-read (bf16 4096^3 3 % faster, bf16 4096x2304x768
            // 10 %, fp32 up to 2 %, never slower beyond noise); split-K
            // planes stay plain (64x512x2048 split 16 ways: 7 % faster).
            if constexpr (STREAM) __builtin_nontemporal_store(w, (u32x4*)dst);
            else *(u32x4*)dst = w;
          } else {
#pragma unroll
            for (int j = 0; j < EPV; ++j)
              if (col + j < p.n) store_from_f32<DT>(dst + j * ESZ, v[j]);
          }
        }
      }
    }
    wave_sync();
  }
}

template <int DT, int ACT, int TM, int TN, bool STREAM = true, bool LUT = false, class Acc>
__device__ __forceinline__ void epilogue_dispatch(const GemmArgs& p, const Acc& acc, float* buf, int row_base,
                                                  int col_base, int lane, bool interior,
                                                  const uint16_t* lut = nullptr) {
  if (interior) epilogue<DT, ACT, TM, TN, true, STREAM, LUT>(p, acc, buf, row_base, col_base, lane, lut);
  else epilogue<DT, ACT, TM, TN, false, STREAM, LUT>(p, acc, buf, row_base, col_base, lane, lut);
}

// ---------------------------------------------------------------------------
// Occupancy the register allocation targets: tiles whose accumulators fill
// the AGPR file run one wave per SIMD and may use the whole register file.
// 16-bit tiles whose loaders stage through registers (M/N-contiguous or
// element loads) hold 8 vectors or 32 packed elements per operand in flight,
// so they are given the register budget of two waves per SIMD.
template <int DT, int BM, int BN, int WM, int WN, int AMODE, int BMODE>
struct Occupancy {
  static constexpr int ACC_REGS = (BM / (WM * 32)) * (BN / (WN * 32)) * 16;
  static constexpr bool REG_STAGED = DT != DT_F32 && (AMODE == MODE_MN || AMODE == MODE_G || BMODE == MODE_MN ||
                                                      BMODE == MODE_G);
  static constexpr int WAVES = ACC_REGS >= 128 ? 1 : ((ACC_REGS >= 64 || REG_STAGED) ? 2 : 4);
};

template <int DT, int BM, int BN, int WM, int WN, int AMODE, int BMODE, int S>
__global__ __launch_bounds__(WM* WN * 64)
__attribute__((amdgpu_waves_per_eu(Occupancy<DT, BM, BN, WM, WN, AMODE, BMODE>::WAVES, 8)))
void fused_gemm_kernel(GemmArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int ESZ = DTraits<DT>::ESZ;
  constexpr int TM = BM / (WM * 32);
  constexpr int TN = BN / (WN * 32);
  constexpr int STAGE = (BM + BN) * kRowBytes;
  static_assert(TM * WM * 32 == BM && TN * WN * 32 == BN, "tile must split into 32x32 blocks");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  int pm, pn, z;
  tile_coords(p, pm, pn, z);
  const int row0 = pm * BM, col0 = pn * BN;
  // This workgroup's K stages [kt0, kt0 + nks); the loaders treat the slice
  // end as the end of K, so nothing past it is read.
  const int kt0 = z * p.kslice;
  const int nks = min((p.k * ESZ + kRowBytes - 1) / kRowBytes - kt0, p.kslice);
  const int kend = min(p.k, (kt0 + nks) * DTraits<DT>::BKE);

  // Four-wave 16-bit tiles up to 128x128 whose operands are both
  // K-contiguous use 16x16x32 MFMAs, two steps per stage; the others 32x32
  // MFMAs, four steps per stage (register loaders write LDS in step 2).  A
  // 16x16x32 step holds twice the fragment registers of a 32x32 step: the
  // 256x256 tiles have no room for them next to their accumulators.
  constexpr bool M16 = DT != DT_F32 && AMODE == MODE_K && BMODE == MODE_K && WM * WN == 4 && BM * BN <= 128 * 128;
  using LA = typename LoaderSel<AMODE, DT, BM, NT, M16>::type;
  using LB = typename LoaderSel<BMODE, DT, BN, NT, M16>::type;
  LA la;
  LB lb;
  la.init(p.a, p.sam, p.sak, row0, p.m, kend);
  lb.init(p.b, p.sbn, p.sbk, col0, p.n, kend);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr0 = (wave / WN) * (TM * 32);
  const int wc0 = (wave % WN) * (TN * 32);

  const int lr = lane & 31, h = lane >> 5;
  constexpr bool ANY_DIRECT = LA::kDirect || LB::kDirect;
  constexpr int NSTEP = M16 ? 2 : 4;
  constexpr int FTM = M16 ? 2 * TM : TM, FTN = M16 ? 2 * TN : TN;  // operand fragments per step
  using Acc = std::conditional_t<M16, f32x4[2 * TM][2 * TN], f32x16[TM][TN]>;
  Acc acc = {};
  constexpr int NM = FTM * FTN * (DT == DT_F32 ? 4 : 1);  // MFMAs per step
  constexpr int NR = FTM + FTN;                            // LDS reads per step
  constexpr int NG_DIRECT = (LA::kDirect ? LA::kGlobalLoads : 0) + (LB::kDirect ? LB::kGlobalLoads : 0);
  constexpr int NG_REG = (LA::kDirect ? 0 : LA::kGlobalLoads) + (LB::kDirect ? 0 : LB::kGlobalLoads);
  constexpr int NW = LA::kLdsWrites + LB::kLdsWrites;
  static_assert(S == 2 || (S <= lds_stages_max<BM, BN, AMODE, BMODE>() && LA::kDirect && LB::kDirect &&
                            LA::kExactPer && LB::kExactPer),
                "rings deeper than two stages count DMA instructions per wave exactly");
  using Fr = Frags<FTM, FTN>;
  // 16x16x32 path: per-lane offsets of the two steps' chunks (rows 16 apart
  // share them).
  const int ao0 = lds_off16(wr0 + (lane & 15), lane >> 4), bo0 = lds_off16(wc0 + (lane & 15), lane >> 4);
  const int ao1 = lds_off16(wr0 + (lane & 15), 4 + (lane >> 4)), bo1 = lds_off16(wc0 + (lane & 15), 4 + (lane >> 4));
  // Fragments of MFMA step `step` of the stage at `base`.
  auto read_step = [&](Fr& f, const char* base, int step) {
    if constexpr (M16) load_frags16(f, base, base + BM * kRowBytes, step ? ao1 : ao0, step ? bo1 : bo0);
    else load_frags(f, base, base + BM * kRowBytes, wr0, wc0, lr, h * 4 + step);
  };

  // Two-stage rings of K-contiguous operands with four MFMA steps per stage
  // split each stage's DMA in two halves issued one step apart: the texture
  // unit takes a stage's fetches (64 KB for a 256x256 16-bit tile) at about
  // 64 B per clock, and a burst of them fills its command queue, which
  // stalls the issuing wave and with it that wave's MFMAs behind the blocked
  // load.
  constexpr bool SPLIT_DMA =
      NSTEP == 4 && S == 2 && AMODE == MODE_K && BMODE == MODE_K && LA::kExactPer && LB::kExactPer;
  constexpr int HA = LA::kGlobalLoads / 2, HB = LB::kGlobalLoads / 2;  // first halves
  constexpr bool PRIO = DT != DT_F32 && !M16 && WM * WN == 8;

  // Software pipeline over K stages, NSTEP MFMA steps per stage, S LDS
  // buffers used as a ring:
  //   steps 0..NSTEP-2: the LDS reads of step s+1 are in flight while step
  //             s's MFMAs issue;
  //   step 0:   (split DMA) the second half of stage kt+1's DMA;
  //   step 2:   (four steps) register loaders write stage kt+1 into the next
  //             buffer;
  //   last step: wait until stage kt+1 has landed, one barrier, then the
  //             next stage's step-0 reads, the DMA of stage kt+S (its first
  //             half with split DMA) into the buffer just released and the
  //             register loaders' global reads of stage kt+2 all overlap this
  //             stage's last MFMAs.
  // A buffer is refilled only after the barrier that follows its last read,
  // and read only after the barrier that follows its fill.  The DMA of a stage
  // has S-1 stages of MFMAs to land (three steps for a split second half);
  // vector memory reads complete in issue order, so "at most (S-2) stages of
  // DMA outstanding" means stage kt+1 has landed.  The body is branch-free:
  // past the last stage every global read is out of range (zeros) and the
  // extra LDS writes land in a buffer nothing reads.
  la.issue(kt0, smem);
  lb.issue(kt0, smem + BM * kRowBytes);
  la.commit(smem);
  lb.commit(smem + BM * kRowBytes);
  // The GELU table, past the ring, while the first stage lands (the barrier
  // before the main loop orders it before the epilogue's reads).
  constexpr bool LUT_TILE = gelu_lut_tile<DT, BM, BN, WM * WN>();
  uint16_t* const lut = (uint16_t*)(smem + S * STAGE);
  if constexpr (LUT_TILE) {
    if (p.splits == 1 && p.act == ACT_GELU_ERF) build_gelu_lut<ACT_GELU_ERF>(lut, threadIdx.x, NT);
    else if (p.splits == 1 && p.act == ACT_GELU_TANH) build_gelu_lut<ACT_GELU_TANH>(lut, threadIdx.x, NT);
  }
  if constexpr (SPLIT_DMA) {
    la.template issue_part<0, HA>(kt0 + 1, smem + STAGE);
    lb.template issue_part<0, HB>(kt0 + 1, smem + STAGE + BM * kRowBytes);
    __builtin_amdgcn_s_waitcnt(0x0F70 | (HA + HB));  // stage kt0 landed
  } else {
#pragma unroll
    for (int d = 1; d < S; ++d) {
      if constexpr (LA::kDirect) la.issue(kt0 + d, smem + d * STAGE);
      if constexpr (LB::kDirect) lb.issue(kt0 + d, smem + d * STAGE + BM * kRowBytes);
    }
    if constexpr (!LA::kDirect) la.issue(kt0 + 1, nullptr);
    if constexpr (!LB::kDirect) lb.issue(kt0 + 1, nullptr);
    if constexpr (ANY_DIRECT) __builtin_amdgcn_s_waitcnt(0x0F70 | ((S - 2) * NG_DIRECT));  // stages kt0, kt0+1 landed
  }
  __syncthreads();
  Fr f0, f1;
  read_step(f0, smem, 0);
  int bi = 0;  // ring index of stage kt
  for (int it = 0; it < nks; ++it) {
    const int kt = kt0 + it;
    const int bn = bi + 1 == S ? 0 : bi + 1;
    char* cur = smem + bi * STAGE;
    char* nxt = smem + bn * STAGE;
    read_step(f1, cur, 1);
    // The 16-bit 8-wave tile runs its steps at raised wave priority until the
    // stage barrier: the arbiter then favours MFMA issue over the other
    // wave's memory instructions (decoder GEMMs 1-4 % faster).
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(3);
    if constexpr (SPLIT_DMA) {
      // nxt (stage kt+1) was released at the previous iteration's barrier.
      la.template issue_part<HA, LA::kGlobalLoads>(kt + 1, nxt);
      lb.template issue_part<HB, LB::kGlobalLoads>(kt + 1, nxt + BM * kRowBytes);
    }
    mma_frags<DT>(f0, acc);
    sched_step<NM, NR, 0, SPLIT_DMA ? NG_DIRECT - HA - HB : 0>();
    if constexpr (NSTEP == 4) {
      read_step(f0, cur, 2);
      mma_frags<DT>(f1, acc);
      sched_step<NM, NR, 0, 0>();
      read_step(f1, cur, 3);
      if constexpr (!LA::kDirect) la.commit(nxt);
      if constexpr (!LB::kDirect) lb.commit(nxt + BM * kRowBytes);
      mma_frags<DT>(f0, acc);
      sched_step<NM, NR, NW, 0>();
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    if constexpr (ANY_DIRECT) __builtin_amdgcn_s_waitcnt(0x0F70 | ((S - 2) * NG_DIRECT));  // stage kt+1 landed
    __syncthreads();
    read_step(f0, nxt, 0);
    if constexpr (SPLIT_DMA) {
      la.template issue_part<0, HA>(kt + S, cur);
      lb.template issue_part<0, HB>(kt + S, cur + BM * kRowBytes);
    } else {
      if constexpr (LA::kDirect) la.issue(kt + S, cur);
      if constexpr (LB::kDirect) lb.issue(kt + S, cur + BM * kRowBytes);
      if constexpr (!LA::kDirect) la.issue(kt + 2, nullptr);
      if constexpr (!LB::kDirect) lb.issue(kt + 2, nullptr);
    }
    mma_frags<DT>(f1, acc);
    sched_step<NM, NR, 0, SPLIT_DMA ? HA + HB : NG_DIRECT + NG_REG>();
    bi = bn;
  }
  __syncthreads();

  // All LDS stage reads are complete (barrier above), so LDS is free.
  static_assert(WM * WN * TN * 32 * 32 * 4 <= 2 * STAGE, "epilogue slices must fit in LDS");
  float* buf = (float*)(smem + wave * (TN * 32 * 32 * 4));
  const int row_base = row0 + wr0, col_base = col0 + wc0;
  if (p.splits > 1) {
    // K slice: raw fp32 sums to this slice's plane of the workspace.
    GemmArgs q = p;
    q.c = (char*)(p.ws + (int64_t)z * p.m * p.n);
    q.has_bias = 0;
    q.res = nullptr;
    const bool interior_ws = row0 + BM <= p.m && col0 + BN <= p.n && (p.n % 4) == 0 && (((uintptr_t)q.c) & 15) == 0;
    epilogue_dispatch<DT_F32, ACT_NONE, TM, TN, false>(q, acc, buf, row_base, col_base, lane, interior_ws);
    return;
  }
  // Interior tiles (the workgroup's whole tile inside C) skip per-element bounds checks.
  const bool interior = row0 + BM <= p.m && col0 + BN <= p.n && (p.n % DTraits<DT>::VEC) == 0 &&
                        (((uintptr_t)p.c) & 15) == 0;
  switch (p.act) {
    case ACT_GELU_ERF:
      epilogue_dispatch<DT, ACT_GELU_ERF, TM, TN, true, LUT_TILE>(p, acc, buf, row_base, col_base, lane, interior, lut);
      break;
    case ACT_GELU_TANH:
      epilogue_dispatch<DT, ACT_GELU_TANH, TM, TN, true, LUT_TILE>(p, acc, buf, row_base, col_base, lane, interior, lut);
      break;
    case ACT_RELU: epilogue_dispatch<DT, ACT_RELU, TM, TN>(p, acc, buf, row_base, col_base, lane, interior); break;
    default: epilogue_dispatch<DT, ACT_NONE, TM, TN>(p, acc, buf, row_base, col_base, lane, interior); break;
  }
}

// ---------------------------------------------------------------------------
// Split-K epilogue: C = act(rnd(rnd(sum_z ws[z]) + bias)), the slices summed
// in order z = 0, 1, ... so results do not depend on scheduling.  Each thread
// owns 4 consecutive elements of C (row-major, flattened).
constexpr int kMaxSplitK = 16;  // most K slices a GEMM is split into

struct ReduceArgs {
  const float* ws;
  const char* bias;
  char* c;
  const char* res;  // optional residual, added to the rounded activation
  int64_t srm, srn;
  int64_t sbi;
  int64_t mn;  // M * N
  int n, splits, has_bias;
  int vec;     // mn % 4 == 0 and ws, c aligned for 4-element vectors
};

template <int DT, int ACT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs p) {
  constexpr int ESZ = DTraits<DT>::ESZ;
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e0 >= p.mn) return;
  const int cnt = p.mn - e0 < 4 ? (int)(p.mn - e0) : 4;
  // Every slice's values are loaded before the first add, so the loads are
  // in flight together rather than one latency per slice.
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (p.vec) {
    float4 w[kMaxSplitK];
#pragma unroll
    for (int z = 0; z < kMaxSplitK; ++z)
      if (z < p.splits) w[z] = *(const float4*)(p.ws + (int64_t)z * p.mn + e0);
#pragma unroll
    for (int z = 0; z < kMaxSplitK; ++z) {
      if (z < p.splits) {
        v[0] += w[z].x;
        v[1] += w[z].y;
        v[2] += w[z].z;
        v[3] += w[z].w;
      }
    }
  } else {
    for (int z = 0; z < p.splits; ++z)
      for (int j = 0; j < cnt; ++j) v[j] += p.ws[(int64_t)z * p.mn + e0 + j];
  }
  int col = (int)(e0 % p.n);
  int64_t row = e0 / p.n;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float x = round_to<DT>(v[j]);
    if (p.has_bias && j < cnt) x = round_to<DT>(x + load_as_f32<DT>(p.bias + (int64_t)col * p.sbi * ESZ));
    x = activate<DT, ACT>(x);
    if (p.res != nullptr && j < cnt)
      x = round_to<DT>(round_to<DT>(x) + load_as_f32<DT>(p.res + (row * p.srm + (int64_t)col * p.srn) * ESZ));
    v[j] = x;
    if (col + 1 == p.n) {
      col = 0;
      ++row;
    } else {
      ++col;
    }
  }
  char* dst = p.c + e0 * ESZ;
  if (p.vec) {
    if constexpr (ESZ == 4) {
      *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint2 w;
      w.x = pack2<DT>(v[0], v[1]);
      w.y = pack2<DT>(v[2], v[3]);
      *(uint2*)dst = w;
    }
  } else {
    for (int j = 0; j < cnt; ++j) store_from_f32<DT>(dst + j * ESZ, v[j]);
  }
}

}  // namespace forgeml
