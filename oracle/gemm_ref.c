/*
 * gemm_ref.c — fp64 brute-force restatement of the fused linear contract.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle that pins the torch-CPU restatement
 * in oracle/fused_linear.py.  Nothing in the product links or calls it.
 *
 *   c[m,n] = act( sum_k a[m,k] * b[k,n] + bias[n] )
 *
 * in double precision with a plain triple loop: the GEMM of ForgeML's
 * `ops.evaluate` for `linear` / `fused_linear_gelu` (src/forgeml/ops.py:28-31,
 * 48-53) and the GELU of src/forgeml/_triton.py:47-57, evaluated with the C
 * library's erf and tanh.  Strides are in elements, as in the kernel ABI.
 */
#include <math.h>
#include <stdint.h>

enum { ACT_NONE = 0, ACT_GELU_ERF = 1, ACT_GELU_TANH = 2, ACT_RELU = 3 };

static double act_apply(double x, int act) {
  switch (act) {
    case ACT_GELU_ERF:
      return 0.5 * x * (1.0 + erf(x / sqrt(2.0)));
    case ACT_GELU_TANH: {
      const double k = sqrt(2.0 / 3.14159265358979323846);
      return 0.5 * x * (1.0 + tanh(k * (x + 0.044715 * x * x * x)));
    }
    case ACT_RELU:
      return x < 0.0 ? 0.0 : x;
    default:
      return x;
  }
}

int oracle_fused_linear_f64(const double* a, int64_t sam, int64_t sak, const double* b, int64_t sbk,
                            int64_t sbn, const double* bias, int64_t sbi, double* c, int64_t m, int64_t n,
                            int64_t k, int act) {
  if (m <= 0 || n <= 0 || k <= 0 || act < ACT_NONE || act > ACT_RELU) return -1;
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int64_t p = 0; p < k; ++p) acc += a[i * sam + p * sak] * b[p * sbk + j * sbn];
      if (bias) acc += bias[j * sbi];
      c[i * n + j] = act_apply(acc, act);
    }
  }
  return 0;
}

/* Scalar GELU for known-value checks. */
double oracle_act_f64(double x, int act) { return act_apply(x, act); }
