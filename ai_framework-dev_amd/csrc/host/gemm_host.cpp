// Host side of the GEMM + bias + activation op: validation in the reference's
// order and with its Status results (gemm/launcher.cu:147-383), bias-kind
// inference (gemm/launcher.cu:47-102, bias.hpp:70-78), then one call into the
// C ABI of libgev2.so.  No device memory is allocated here.
#include "gemm_host.hpp"

#include <limits>
#include <string>

#include "gev2_gemm.h"

namespace ai::cuda::shim {
namespace {

thread_local std::string t_err;

Status fail(Status s, const char* why) {
  t_err = why;
  return s;
}

bool fits_int32(std::int64_t v) { return v >= 0 && v <= std::numeric_limits<int>::max(); }

bool is_float_dtype(DType d) { return d == DType::F32 || d == DType::F16 || d == DType::BF16; }

// The reference's is_cuda_f32_rowmajor (ai_validate.hpp:137-142), widened to
// the three float storage types this build computes in.
bool is_gpu_rowmajor_2d(const Tensor& t, DType dt) {
  return t.is_cuda() && t.desc.dtype == dt && t.desc.layout == Layout::RowMajor &&
         t.desc.shape.size() == 2;
}

// tensor_layout.hpp:12-19: stride[0] if positive, else the column count.
std::int64_t infer_ld(const Tensor& t) {
  if (t.desc.shape.size() != 2) return 0;
  if (t.desc.stride.size() >= 2 && t.desc.stride[0] > 0) return t.desc.stride[0];
  return t.desc.shape[1];
}

std::int64_t safe_mul_nonneg(std::int64_t a, std::int64_t b) {
  if (a < 0 || b < 0) return -1;
  if (a == 0 || b == 0) return 0;
  return a > std::numeric_limits<std::int64_t>::max() / b ? -1 : a * b;
}

bool lt_ws_ok(const GemmWorkspace* ws) {
  return !ws || !ws->lt_workspace || (reinterpret_cast<std::uintptr_t>(ws->lt_workspace) % 256) == 0;
}

bool scratch_ok(const GemmWorkspace* ws, std::int64_t M, std::int64_t N) {
  if (!ws || !ws->scratch || ws->scratch_bytes == 0) return true;
  return ws->scratch_bytes >= GemmRequiredBackwardScratchBytes(M, N);
}

Status from_abi(int st) {
  if (st != GEV2_OK) t_err = gev2_last_error();
  return static_cast<Status>(st);
}

}  // namespace

const char* GemmLastError() { return t_err.c_str(); }

BiasKind infer_bias_kind_1d_lenMN(const Tensor* Bias, std::int64_t M, std::int64_t N) {
  if (!Bias || !Bias->data || Bias->desc.shape.size() != 1) return BiasKind::None;
  const std::int64_t len = Bias->desc.shape[0];
  if (len == 1) return BiasKind::Scalar;
  if (len == N) return BiasKind::PerN;
  if (len == M) return BiasKind::PerM;
  return BiasKind::None;
}

BiasKind infer_bias_kind_fallback(const Tensor* Bias, std::int64_t M, std::int64_t N) {
  if (!Bias || !Bias->data) return BiasKind::None;
  const auto& s = Bias->desc.shape;
  std::int64_t numel = 1;
  for (auto v : s) {
    if (v < 0) return BiasKind::None;
    numel = safe_mul_nonneg(numel, v);
    if (numel < 0) return BiasKind::None;
  }
  if (numel == 0) return BiasKind::None;
  if (s.size() == 2 && s[0] == 1 && s[1] == N) return BiasKind::PerN;
  if (s.size() == 1 && s[0] == N) return BiasKind::PerN;
  if (s.size() == 2 && s[0] == M && s[1] == 1) return BiasKind::PerM;
  if (s.size() == 1 && s[0] == M) return BiasKind::PerM;
  if ((s.size() == 2 && s[0] == 1 && s[1] == 1) || (s.size() == 1 && s[0] == 1)) return BiasKind::Scalar;
  if (numel == N) return BiasKind::PerN;
  if (numel == M) return BiasKind::PerM;
  if (numel == 1) return BiasKind::Scalar;
  return BiasKind::None;   // e.g. an (M,N) bias: no bias is applied
}

BiasKind decide_bias_kind(const Tensor* Bias, std::int64_t M, std::int64_t N) {
  const BiasKind k = infer_bias_kind_1d_lenMN(Bias, M, N);
  return k != BiasKind::None ? k : infer_bias_kind_fallback(Bias, M, N);
}

bool validate_bias_buffer(const Tensor* Bias, std::int64_t M, std::int64_t N, BiasKind kind) {
  if (!Bias || !Bias->data || kind == BiasKind::None) return true;
  if (Bias->desc.dtype != DType::F32) return false;
  const std::int64_t need = kind == BiasKind::Scalar ? 1 : kind == BiasKind::PerM ? M : N;
  if (need <= 0) return false;
  std::int64_t numel = 1;
  for (auto v : Bias->desc.shape) {
    if (v < 0) return false;
    numel *= v;
  }
  if (numel == need) return true;
  const auto& s = Bias->desc.shape;
  return s.size() == 2 && ((kind == BiasKind::PerN && s[0] == 1 && s[1] == N) ||
                           (kind == BiasKind::PerM && s[0] == M && s[1] == 1) ||
                           (kind == BiasKind::Scalar && s[0] == 1 && s[1] == 1));
}

// ---------------------------------------------------------------------------
// Forward (single and batched share the checks; `batched` admits transposes)
// ---------------------------------------------------------------------------
static Status forward_impl(const Tensor& A, const Tensor& B, const Tensor* Bias, Tensor& Y,
                           const GemmAttrs& attrs, const GemmBatch& bt, bool batched,
                           StreamHandle stream, Tensor* Z_saved, const GemmWorkspace* ws) {
  t_err.clear();
  const DType dt = A.desc.dtype;
  // 1) device / dtype / layout / rank
  if (!is_float_dtype(dt) || !is_gpu_rowmajor_2d(A, dt) || !is_gpu_rowmajor_2d(B, dt) ||
      !is_gpu_rowmajor_2d(Y, dt))
    return fail(Status::DeviceMismatch, "A, B, Y must be GPU row-major 2-D tensors of one float dtype");
  if (!batched && (attrs.trans_a || attrs.trans_b))
    return fail(Status::TransposeNotSupported, "only the non-transposed forward is supported");
  // 2) shapes
  const bool ta = batched && attrs.trans_a, tb = batched && attrs.trans_b;
  const std::int64_t M = ta ? A.desc.shape[1] : A.desc.shape[0];
  const std::int64_t K = ta ? A.desc.shape[0] : A.desc.shape[1];
  const std::int64_t Kb = tb ? B.desc.shape[1] : B.desc.shape[0];
  const std::int64_t N = tb ? B.desc.shape[0] : B.desc.shape[1];
  if (K != Kb || Y.desc.shape[0] != M || Y.desc.shape[1] != N)
    return fail(Status::ShapeMismatch, "shapes do not chain: A[M,K] B[K,N] Y[M,N]");
  // 3) leading dimensions
  const std::int64_t lda = infer_ld(A), ldb = infer_ld(B), ldd = infer_ld(Y);
  if (lda < A.desc.shape[1] || ldb < B.desc.shape[1] || ldd < N)
    return fail(Status::StrideMismatch, "leading dimension smaller than the row length");
  // 4) int32 range
  if (!fits_int32(M) || !fits_int32(N) || !fits_int32(K) || !fits_int32(lda) || !fits_int32(ldb) ||
      !fits_int32(ldd))
    return fail(Status::Invalid, "dimension or leading dimension exceeds int32");
  // 5) pre-activation stash
  if (attrs.save_z && Z_saved == nullptr)
    return fail(Status::MissingOutput, "save_z requires Z_saved");
  const bool want_z = attrs.save_z && Z_saved != nullptr;
  std::int64_t ldz = 0;
  if (want_z) {
    if (!is_gpu_rowmajor_2d(*Z_saved, dt)) return fail(Status::DeviceMismatch, "Z_saved must match Y");
    if (Z_saved->desc.shape[0] != M || Z_saved->desc.shape[1] != N)
      return fail(Status::ShapeMismatch, "Z_saved must be [M,N]");
    ldz = (Z_saved->data == Y.data) ? ldd : infer_ld(*Z_saved);
    if (ldz < N) return fail(Status::StrideMismatch, "ldZ < N");
    if (!fits_int32(ldz)) return fail(Status::Invalid, "ldZ exceeds int32");
  }
  if (!lt_ws_ok(ws)) return fail(Status::Invalid, "lt_workspace must be 256-byte aligned");
  // 6) bias
  const BiasKind bk = decide_bias_kind(Bias, M, N);
  if (!validate_bias_buffer(Bias, M, N, bk)) return fail(Status::Invalid, "bias must be F32 of the kind's length");
  if (bt.count < 1 || !fits_int32(bt.count)) return fail(Status::Invalid, "batch count out of range");

  gev2_gemm_fwd_desc d{};
  d.dtype = static_cast<int32_t>(dt);
  d.act = static_cast<int32_t>(attrs.act);
  d.bias_kind = static_cast<int32_t>(bk);
  d.trans_a = ta ? 1 : 0;
  d.trans_b = tb ? 1 : 0;
  d.leaky_slope = attrs.leaky_slope;
  d.alpha = batched ? attrs.alpha : 1.0f;
  d.M = M; d.N = N; d.K = K; d.batch = bt.count;
  d.A = A.data; d.lda = lda; d.stride_a = bt.stride_a;
  d.B = B.data; d.ldb = ldb; d.stride_b = bt.stride_b;
  d.bias = bk != BiasKind::None ? static_cast<const float*>(Bias->data) : nullptr;
  d.stride_bias = bt.stride_bias;
  d.Y = Y.data; d.ldy = ldd; d.stride_y = bt.stride_y;
  d.Z = want_z ? Z_saved->data : nullptr; d.ldz = ldz; d.stride_z = bt.stride_z;
  if (ws && ws->scratch) {   // split-K partials of skinny problems (gev2_gemm_fwd_workspace_size)
    d.workspace = ws->scratch;
    d.workspace_bytes = static_cast<int64_t>(ws->scratch_bytes);
  }
  return from_abi(gev2_gemm_fwd(&d, stream));
}

Status GemmCudaLaunch(const Tensor& A, const Tensor& B, const Tensor* Bias, Tensor& Y,
                      const GemmAttrs& attrs, StreamHandle stream, Tensor* Z_saved,
                      const GemmWorkspace* ws) {
  return forward_impl(A, B, Bias, Y, attrs, GemmBatch{}, false, stream, Z_saved, ws);
}

Status GemmBatchedLaunch(const Tensor& A, const Tensor& B, const Tensor* Bias, Tensor& Y,
                         const GemmAttrs& attrs, const GemmBatch& batch, StreamHandle stream,
                         Tensor* Z_saved) {
  return forward_impl(A, B, Bias, Y, attrs, batch, true, stream, Z_saved, nullptr);
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
static Status backward_impl(const Tensor& A, const Tensor& B, const Tensor* C, const Tensor& gY,
                            const Tensor& Z, Tensor* gA, Tensor* gB, Tensor* gC, Tensor* gBias,
                            const GemmAttrs& attrs, const GemmBatchBwd& bt, StreamHandle stream,
                            const GemmWorkspace* ws) {
  t_err.clear();
  const DType dt = A.desc.dtype;
  auto ok = [&](const Tensor& t) { return is_gpu_rowmajor_2d(t, dt); };
  if (!is_float_dtype(dt) || !ok(A) || !ok(B) || !ok(gY) || !ok(Z))
    return fail(Status::DeviceMismatch, "A, B, gY, Z must be GPU row-major 2-D tensors of one float dtype");
  if ((gA && !ok(*gA)) || (gB && !ok(*gB)) || (gC && !ok(*gC)) || (C && !ok(*C)))
    return fail(Status::DeviceMismatch, "gA/gB/gC/C must match A");
  if (attrs.trans_a || attrs.trans_b)
    return fail(Status::TransposeNotSupported, "only the non-transposed backward is supported");
  const std::int64_t M = A.desc.shape[0], K = A.desc.shape[1];
  const std::int64_t Kb = B.desc.shape[0], N = B.desc.shape[1];
  if (K != Kb) return fail(Status::ShapeMismatch, "A[M,K] B[K,N]: K differs");
  if (gY.desc.shape[0] != M || gY.desc.shape[1] != N || Z.desc.shape[0] != M || Z.desc.shape[1] != N)
    return fail(Status::ShapeMismatch, "gY and Z must be [M,N]");
  if (gA && (gA->desc.shape[0] != M || gA->desc.shape[1] != K))
    return fail(Status::ShapeMismatch, "gA must be [M,K]");
  if (gB && (gB->desc.shape[0] != K || gB->desc.shape[1] != N))
    return fail(Status::ShapeMismatch, "gB must be [K,N]");
  if (gC) {
    if (!C) return fail(Status::MissingInput, "gC requires C");
    if (gC->desc.shape[0] != M || gC->desc.shape[1] != N) return fail(Status::ShapeMismatch, "gC must be [M,N]");
  }
  const std::int64_t lda = infer_ld(A), ldb = infer_ld(B), ldgy = infer_ld(gY), ldz = infer_ld(Z);
  if (lda < K || ldb < N || ldgy < N || ldz < N)
    return fail(Status::StrideMismatch, "leading dimension smaller than the row length");
  std::int64_t ldga = 0, ldgb = 0, ldgc = 0;
  if (gA && (ldga = infer_ld(*gA)) < K) return fail(Status::StrideMismatch, "ldgA < K");
  if (gB && (ldgb = infer_ld(*gB)) < N) return fail(Status::StrideMismatch, "ldgB < N");
  if (gC && (ldgc = infer_ld(*gC)) < N) return fail(Status::StrideMismatch, "ldgC < N");
  if (!fits_int32(M) || !fits_int32(N) || !fits_int32(K) || !fits_int32(lda) || !fits_int32(ldb) ||
      !fits_int32(ldgy) || !fits_int32(ldz) || (gA && !fits_int32(ldga)) ||
      (gB && !fits_int32(ldgb)) || (gC && !fits_int32(ldgc)))
    return fail(Status::Invalid, "dimension or leading dimension exceeds int32");
  BiasKind bk = BiasKind::None;
  if (gBias && gBias->data) {
    bk = decide_bias_kind(gBias, M, N);
    if (!validate_bias_buffer(gBias, M, N, bk)) return fail(Status::Invalid, "gBias must be F32 of the kind's length");
  }
  if (!lt_ws_ok(ws)) return fail(Status::Invalid, "lt_workspace must be 256-byte aligned");
  if (!scratch_ok(ws, M, N)) return fail(Status::Invalid, "scratch smaller than M*N*4 bytes");
  if (bt.count < 1 || !fits_int32(bt.count)) return fail(Status::Invalid, "batch count out of range");

  gev2_gemm_bwd_desc d{};
  d.dtype = static_cast<int32_t>(dt);
  d.act = static_cast<int32_t>(attrs.act);
  d.bias_kind = static_cast<int32_t>(bk);
  d.leaky_slope = attrs.leaky_slope;
  d.alpha = 1.0f;
  d.beta = (C && gC) ? 1.0f : 0.0f;
  d.M = M; d.N = N; d.K = K; d.batch = bt.count;
  d.A = A.data; d.lda = lda; d.stride_a = bt.stride_a;
  d.B = B.data; d.ldb = ldb; d.stride_b = bt.stride_b;
  d.gY = gY.data; d.ldgy = ldgy; d.stride_gy = bt.stride_gy;
  d.Z = Z.data; d.ldz = ldz; d.stride_z = bt.stride_z;
  d.gA = gA ? gA->data : nullptr; d.ldga = ldga; d.stride_ga = bt.stride_ga;
  d.gB = gB ? gB->data : nullptr; d.ldgb = ldgb; d.stride_gb = bt.stride_gb;
  d.gC = gC ? gC->data : nullptr; d.ldgc = ldgc; d.stride_gc = bt.stride_gc;
  d.gBias = bk != BiasKind::None ? static_cast<float*>(gBias->data) : nullptr;
  d.stride_gbias = bt.stride_gbias;
  if (ws && ws->scratch) {   // the reference's dZ scratch (M*N fp32) doubles as gZ storage
    d.workspace = ws->scratch;
    d.workspace_bytes = static_cast<int64_t>(ws->scratch_bytes ? ws->scratch_bytes
                                                                : GemmRequiredBackwardScratchBytes(M, N));
  }
  return from_abi(gev2_gemm_bwd(&d, stream));
}

Status GemmCudaBackward(const Tensor& A, const Tensor& B, const Tensor* C, const Tensor& gY,
                        const Tensor& Z, Tensor* gA, Tensor* gB, Tensor* gC, Tensor* gBias,
                        const GemmAttrs& attrs, StreamHandle stream, const GemmWorkspace* ws) {
  return backward_impl(A, B, C, gY, Z, gA, gB, gC, gBias, attrs, GemmBatchBwd{}, stream, ws);
}

Status GemmBatchedBackward(const Tensor& A, const Tensor& B, const Tensor* C, const Tensor& gY,
                           const Tensor& Z, Tensor* gA, Tensor* gB, Tensor* gC, Tensor* gBias,
                           const GemmAttrs& attrs, const GemmBatchBwd& batch, StreamHandle stream) {
  return backward_impl(A, B, C, gY, Z, gA, gB, gC, gBias, attrs, batch, stream, nullptr);
}

}  // namespace ai::cuda::shim
