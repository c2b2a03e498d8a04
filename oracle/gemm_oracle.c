/*
 * CPU restatement (plain C, float32) of graph_executor_v2's fused
 * GEMM + bias + activation operator.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and bench.py's cpu_baseline leg
 * as a checker; the product library never links or calls it.
 *
 * What it restates, in the reference's own float32 arithmetic:
 *   - act_apply / act_deriv: backends/cuda/ops/_common/shim/activations.hpp:14-70
 *     (host branch of math_compat.hpp:12-28: std::exp / std::tanh)
 *   - the small-problem forward kernel gemm_bias_act_f32_smoke_ex,
 *     gemm/kernels/regemm_gemm_bias_act.cu:226-252: one output at a time,
 *     acc = fmaf(a, b, acc) for k = 0..K-1, then pre = alpha*acc,
 *     + bias (bias.hpp:155-176), Z = pre, Y = act(pre)
 *   - the backward epilogue bwd_epilogue_kernel, regemm_backward.cu:91-130
 *     (gZ = gY * act'(Z), gC = beta*gZ, gBias accumulated per kind), followed
 *     by gA = alpha*gZ*B^T and gB = alpha*A^T*gZ (regemm_backward.cu:271-291,
 *     there cuBLAS; here a double-accumulated loop, since cuBLAS's order is
 *     unspecified).
 *
 * Build: oracle/Makefile -> oracle/libgemm_oracle.so
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

enum { ACT_NONE = 0, ACT_RELU = 1, ACT_LEAKY = 2, ACT_GELU = 3, ACT_SIGMOID = 4, ACT_TANH = 5 };
enum { BIAS_NONE = 0, BIAS_SCALAR = 1, BIAS_PERM = 2, BIAS_PERN = 3 };

static const float kGeluC = 0.7978845608f;  /* activations.hpp:19 */
static const float kGeluK1 = 0.044715f;     /* activations.hpp:20 */

float gev2o_act(float x, int act, float slope) {
  switch (act) {
    case ACT_RELU: return x > 0.f ? x : 0.f;
    case ACT_LEAKY: return x > 0.f ? x : slope * x;
    case ACT_GELU: {
      float x2 = x * x, x3 = x2 * x;
      float t = fmaf(kGeluC * kGeluK1, x3, kGeluC * x);
      return 0.5f * x * (1.f + tanhf(t));
    }
    case ACT_SIGMOID:
      if (x >= 0.f) { float z = expf(-x); return 1.f / (1.f + z); }
      else { float z = expf(x); return z / (1.f + z); }
    case ACT_TANH: return tanhf(x);
    default: return x;
  }
}

float gev2o_act_deriv(float x, int act, float slope) {
  switch (act) {
    case ACT_RELU: return x > 0.f ? 1.f : 0.f;
    case ACT_LEAKY: return x > 0.f ? 1.f : slope;
    case ACT_GELU: {
      float x2 = x * x, x3 = x2 * x;
      float t = fmaf(kGeluC * kGeluK1, x3, kGeluC * x);
      float th = tanhf(t);
      if (th > 0.999999f) th = 0.999999f;
      if (th < -0.999999f) th = -0.999999f;
      float sech2 = 1.f - th * th;
      float dt = kGeluC * (1.f + 3.f * kGeluK1 * x2);
      return 0.5f * (1.f + th) + 0.5f * x * sech2 * dt;
    }
    case ACT_SIGMOID: {
      float s;
      if (x >= 0.f) { float z = expf(-x); s = 1.f / (1.f + z); }
      else { float z = expf(x); s = z / (1.f + z); }
      return s * (1.f - s);
    }
    case ACT_TANH: { float th = tanhf(x); return 1.f - th * th; }
    default: return 1.f;
  }
}

static float load_bias(const float* bias, int kind, int64_t m, int64_t n) {
  if (!bias) return 0.f;
  switch (kind) {
    case BIAS_SCALAR: return bias[0];
    case BIAS_PERM: return bias[m];
    case BIAS_PERN: return bias[n];
    default: return 0.f;
  }
}

/* Forward, reference small-kernel order.  Z may be NULL.  Row-major, lds given. */
void gev2o_gemm_fwd_f32(int64_t M, int64_t N, int64_t K,
                        const float* A, int64_t lda, const float* B, int64_t ldb,
                        const float* bias, int bias_kind, float alpha,
                        int act, float slope,
                        float* Y, int64_t ldy, float* Z, int64_t ldz) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.f;
      for (int64_t k = 0; k < K; ++k) acc = fmaf(A[m * lda + k], B[k * ldb + n], acc);
      float pre = alpha * acc;
      pre += load_bias(bias, bias_kind, m, n);
      if (Z) Z[m * ldz + n] = pre;
      Y[m * ldy + n] = gev2o_act(pre, act, slope);
    }
  }
}

/* Backward.  Any of gA, gB, gC, gBias may be NULL.  gZ_tmp must hold M*N floats. */
void gev2o_gemm_bwd_f32(int64_t M, int64_t N, int64_t K,
                        const float* A, int64_t lda, const float* B, int64_t ldb,
                        const float* gY, int64_t ldgy, const float* Z, int64_t ldz,
                        int act, float slope, float alpha, float beta,
                        float* gA, int64_t ldga, float* gB, int64_t ldgb,
                        float* gC, int64_t ldgc, float* gBias, int bias_kind,
                        float* gZ_tmp) {
  if (gBias) {
    int64_t nb = bias_kind == BIAS_SCALAR ? 1 : bias_kind == BIAS_PERM ? M
               : bias_kind == BIAS_PERN ? N : 0;
    for (int64_t i = 0; i < nb; ++i) gBias[i] = 0.f;
  }
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float gz = gY[m * ldgy + n] * gev2o_act_deriv(Z[m * ldz + n], act, slope);
      gZ_tmp[m * N + n] = gz;
      if (gC) gC[m * ldgc + n] = beta * gz;
      if (gBias) {
        if (bias_kind == BIAS_PERN) gBias[n] += gz;
        else if (bias_kind == BIAS_PERM) gBias[m] += gz;
        else if (bias_kind == BIAS_SCALAR) gBias[0] += gz;
      }
    }
  }
  if (gA) {
    for (int64_t m = 0; m < M; ++m)
      for (int64_t k = 0; k < K; ++k) {
        double s = 0.0;
        for (int64_t n = 0; n < N; ++n) s += (double)gZ_tmp[m * N + n] * (double)B[k * ldb + n];
        gA[m * ldga + k] = (float)(alpha * s);
      }
  }
  if (gB) {
    for (int64_t k = 0; k < K; ++k)
      for (int64_t n = 0; n < N; ++n) {
        double s = 0.0;
        for (int64_t m = 0; m < M; ++m) s += (double)A[m * lda + k] * (double)gZ_tmp[m * N + n];
        gB[k * ldgb + n] = (float)(alpha * s);
      }
  }
}

/* Vectorised activation helpers over arrays (for the test suite). */
void gev2o_act_array(const float* x, float* y, int64_t n, int act, float slope) {
  for (int64_t i = 0; i < n; ++i) y[i] = gev2o_act(x[i], act, slope);
}

void gev2o_act_deriv_array(const float* x, float* y, int64_t n, int act, float slope) {
  for (int64_t i = 0; i < n; ++i) y[i] = gev2o_act_deriv(x[i], act, slope);
}
