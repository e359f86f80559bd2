/*
 * forgeml_hip.h — C ABI of the MI355X (gfx950) fused linear kernels.
 *
 * The library computes, on one HIP stream,
 *
 *     C[M,N] = act( rnd( rnd( sum_k A[m,k] * B[k,n] ) + bias[n] ) )
 *
 * with fp32 accumulation on MFMA, where rnd() rounds to the output dtype
 * (identity for fp32), the bias add is optional and act is none, exact-erf
 * GELU, tanh GELU or clamp_min(x, 0).  A and B may have any element strides;
 * C is contiguous with row stride N.  This is the contract of ForgeML's
 * Triton `_matmul_kernel` (src/forgeml/_triton.py:6-62), whose launcher
 * `launch(a, b, bias, out, approximate, config, activation)`
 * (src/forgeml/_triton.py:65-93) is what `forgeml_hip_gemm` replaces.
 *
 * Ownership: every pointer belongs to the caller.  The library never
 * allocates or frees device memory.  Kernels that split the K reduction use
 * the caller's workspace (see forgeml_hip_gemm_workspace_size).
 *
 * Threading: all entry points are reentrant.  Errors are reported through the
 * return code and a thread-local message (forgeml_hip_last_error).
 */
#ifndef FORGEML_HIP_H
#define FORGEML_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (the reference accepts fp16, bf16 and fp32: kernels.py:29-32). */
#define FORGEML_DTYPE_F32 0
#define FORGEML_DTYPE_BF16 1
#define FORGEML_DTYPE_F16 2

/* Epilogue activations.  1 and 2 are the reference's ACT codes
 * (src/forgeml/_triton.py:47-57, :70); 3 is the executor's relu slot writer,
 * clamp_min(x, 0) (src/forgeml/compiler.py:103-104), fused here. */
#define FORGEML_ACT_NONE 0
#define FORGEML_ACT_GELU_ERF 1
#define FORGEML_ACT_GELU_TANH 2
#define FORGEML_ACT_RELU 3

/* Return codes. */
#define FORGEML_OK 0
#define FORGEML_EINVAL (-1)   /* bad argument: shape, stride, dtype, act, pointer */
#define FORGEML_ECONFIG (-2)  /* config id unknown or not built for this dtype */
#define FORGEML_EHIP (-3)     /* the HIP runtime reported an error */
#define FORGEML_EWORKSPACE (-4) /* workspace missing or too small */

/* Config id meaning "choose by shape" (the reference's DEFAULT_CONFIG,
 * src/forgeml/kernels.py:13-21, is a fixed tile; here the default is a
 * shape heuristic over the MI355X tile table). */
#define FORGEML_CONFIG_AUTO (-1)

/* Fields returned by forgeml_hip_config_info, in order. */
#define FORGEML_CONFIG_INFO_FIELDS 8
/* [0] dtype class: 0 = fp32, 1 = 16-bit (bf16 and fp16)
 * [1] block_m   [2] block_n   [3] block_k (elements per LDS stage)
 * [4] waves per workgroup     [5] LDS stages (at most: a launch may ring
 *     through fewer, as the grid size and operand layout decide)
 * [6] split_k (1 = none; >1 = K split over workgroups, needs a workspace)
 * [7] LDS bytes per workgroup (at the most stages; for the 8-wave 16-bit
 *     256x256 tile including the 10 KiB table of bf16 GELU values) */

/*
 * Fused GEMM + bias + activation.  Replaces `launch` in
 * src/forgeml/_triton.py:65-93 (called from kernels.matmul,
 * src/forgeml/kernels.py:206-209).
 *
 *   a        [M,K] element (m,k) at a + (m*sam + k*sak) elements
 *   b        [K,N] element (k,n) at b + (k*sbk + n*sbn) elements
 *   bias     [N] element n at bias + n*sbi; NULL for no bias
 *   c        [M,N] contiguous, element (m,n) at c + m*N + n
 *   dtype    FORGEML_DTYPE_*; a, b, bias and c share it
 *   act      FORGEML_ACT_*
 *   config_id  index into the tile table, or FORGEML_CONFIG_AUTO
 *   workspace, workspace_bytes  device scratch for split-K configs
 *            (may be NULL/0 when forgeml_hip_gemm_workspace_size is 0)
 *   stream   hipStream_t to launch on (NULL = the null stream)
 *
 * Returns FORGEML_OK or a negative FORGEML_E* code (FORGEML_EINVAL also when
 * the config's grid would need 2^32 or more work-items; FORGEML_CONFIG_AUTO
 * plans a config that fits when the operands' layout allows one).  The
 * launch is asynchronous; errors raised
 * while the kernel runs surface on the stream.
 */
int forgeml_hip_gemm(const void* a, int64_t sam, int64_t sak,
                     const void* b, int64_t sbk, int64_t sbn,
                     const void* bias, int64_t sbi,
                     void* c, int64_t m, int64_t n, int64_t k,
                     int32_t dtype, int32_t act, int32_t config_id,
                     void* workspace, int64_t workspace_bytes,
                     void* stream);

/*
 * Fused GEMM + bias + activation + residual add:
 *
 *     C = rnd( rnd( act( rnd( rnd(A·B) + bias ) ) ) + R )
 *
 * i.e. forgeml_hip_gemm followed, in the same epilogue, by the `add` node
 * the reference's executor runs next on the GEMM's result (the residual
 * connections of the transformer block: ops.py's `add`, compiled by the
 * torch slot writer at src/forgeml/compiler.py:93-98).  R[M,N] has element
 * (m,n) at r + (m*srm + n*srn) elements and may be C itself (strides N, 1),
 * but must not partly overlap it.  Other arguments, errors and workspace
 * rules are forgeml_hip_gemm's.  No reference counterpart as one call: the
 * reference runs the GEMM and the add as two kernels.
 */
int forgeml_hip_gemm_add(const void* a, int64_t sam, int64_t sak,
                         const void* b, int64_t sbk, int64_t sbn,
                         const void* bias, int64_t sbi,
                         const void* r, int64_t srm, int64_t srn,
                         void* c, int64_t m, int64_t n, int64_t k,
                         int32_t dtype, int32_t act, int32_t config_id,
                         void* workspace, int64_t workspace_bytes,
                         void* stream);

/*
 * forgeml_hip_gemm without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  No counterpart in the reference (its
 * launcher has no split-K workspace).  A shape whose K is split keeps its
 * fp32 partial planes in a scratch array the library holds on each GPU it
 * runs on, from the first call there until the process ends, of
 * forgeml_hip_noalloc_scratch_bytes() bytes (32 MiB); a shape that needs
 * more is refused with FORGEML_EWORKSPACE and nothing is launched.  The
 * call allocates nothing.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or threads) race and
 * must be serialised by the caller.  Other arguments, errors and results
 * are forgeml_hip_gemm's (the same kernels run).
 */
int forgeml_hip_gemm_noalloc(const void* a, int64_t sam, int64_t sak,
                             const void* b, int64_t sbk, int64_t sbn,
                             const void* bias, int64_t sbi,
                             void* c, int64_t m, int64_t n, int64_t k,
                             int32_t dtype, int32_t act, int32_t config_id,
                             void* stream);

/* Bytes of the per-GPU scratch array of forgeml_hip_gemm_noalloc. */
int64_t forgeml_hip_noalloc_scratch_bytes(void);

/* What forgeml_hip_gemm would run for these operands, without launching:
 *   out[0]  the config id (resolved when config_id is FORGEML_CONFIG_AUTO)
 *   out[1]  the number of K slices (1 = K is not split)
 *   out[2]  workspace bytes the call needs (0 when K is not split)
 *   out[3]  kernel kind: 0 = tiled, 1 = few-row (M <= 64)
 * Pointers are used only for their alignment.  Returns FORGEML_OK or the
 * error forgeml_hip_gemm would return for them.  No reference counterpart:
 * the reference's launcher has no split-K workspace to size. */
int forgeml_hip_gemm_plan(const void* a, int64_t sam, int64_t sak,
                          const void* b, int64_t sbk, int64_t sbn,
                          int64_t m, int64_t n, int64_t k,
                          int32_t dtype, int32_t config_id, int64_t* out);

/* Bytes of workspace forgeml_hip_gemm needs for this shape and config, for
 * any operand layout (an upper bound when config_id is FORGEML_CONFIG_AUTO;
 * forgeml_hip_gemm_plan gives the exact figure for given operands).  0 when
 * no layout splits K; negative on bad arguments.  No reference counterpart:
 * the reference has no split-K kernel. */
int64_t forgeml_hip_gemm_workspace_size(int64_t m, int64_t n, int64_t k,
                                        int32_t dtype, int32_t config_id);

/* The config id FORGEML_CONFIG_AUTO resolves to for this shape when both
 * operands are K-contiguous with 16-byte aligned rows (forgeml_hip_gemm also
 * weighs the actual layout).  Counterpart of DEFAULT_CONFIG
 * (src/forgeml/kernels.py:21). */
int forgeml_hip_select_config(int64_t m, int64_t n, int64_t k, int32_t dtype);

/* Number of entries in the tile table.  Counterpart of
 * len(CANDIDATES) (src/forgeml/kernels.py:22-27). */
int forgeml_hip_num_configs(void);

/* Writes FORGEML_CONFIG_INFO_FIELDS int32 values describing config `id`.
 * Counterpart of the KernelConfig fields (src/forgeml/kernels.py:12-18). */
int forgeml_hip_config_info(int32_t id, int32_t* out);

/*
 * LayerNorm over the last dimension:
 *     y[r, :] = (x[r, :] - mean) / sqrt(var + eps) * w + b     (biased variance)
 * computed in fp32 and rounded once to the dtype.  x has `rows` rows of
 * `cols` contiguous elements, row stride sx >= cols; y is contiguous.  w and b
 * ([cols], contiguous) are both given or both NULL.  Replaces the torch call
 * F.layer_norm of the `layer_norm` op (src/forgeml/ops.py, _layer_norm).
 */
int forgeml_hip_layer_norm(const void* x, int64_t sx, const void* w, const void* b,
                           void* y, int64_t rows, int64_t cols, float eps,
                           int32_t dtype, void* stream);

/*
 * Scaled dot-product attention, fp32:
 *     O = softmax(Q K^T * scale + causal mask) V
 * per (batch, head), Q [lq, dim], K and V [lk, dim], the causal mask letting
 * query i see keys j <= i (top-left aligned, as torch's is_causal).  Each of
 * q, k, v, o is described by 4 element strides (batch, head, sequence, dim);
 * q, k and v need unit stride along dim and 16-byte aligned rows of q and k.
 * dim is 32, 64, 96 or 128.  Replaces F.scaled_dot_product_attention of the
 * `sdpa` op without an attention mask (src/forgeml/ops.py, _sdpa).
 */
int forgeml_hip_attention(const void* q, const int64_t* sq, const void* k, const int64_t* sk,
                          const void* v, const int64_t* sv, void* o, const int64_t* so,
                          int64_t batch, int64_t heads, int64_t lq, int64_t lk, int64_t dim,
                          int32_t causal, float scale, int32_t dtype, void* stream);

/* Thread-local text of the last error on this thread ("" if none).
 * The reference raises Python exceptions instead (kernels.py:62-112). */
const char* forgeml_hip_last_error(void);

/* ABI version of this header; bumped on any signature change. */
int forgeml_hip_abi_version(void);

#define FORGEML_HIP_ABI_VERSION 5

#ifdef __cplusplus
}
#endif

#endif /* FORGEML_HIP_H */
