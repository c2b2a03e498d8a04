// C++ operator API of the GEMM + bias + activation op (host side).
//
// Same entry points, argument meaning and Status results as the reference's
// graph_executor_v2/backends/cuda/ops/gemm/api.hpp:97-188 (implemented in
// gemm/launcher.cu:147-383), so its C++ callers (conv2d/launcher.cu:216,429,
// rnn/launcher.cu:194,345) and the pybind module bind unchanged.  The
// implementation validates the views and forwards to the C ABI of
// libgev2.so (include/gev2_gemm.h).  It allocates nothing itself; the
// operator allocates scratch only when the caller's workspace is missing or
// too small, and never while the stream is being captured into a graph.
//
// Differences a caller can observe:
//   - F16 and BF16 tensors are accepted (all of A, B, Y, Z, gY, gA, gB, gC in
//     one dtype; bias / gBias stay F32).  The reference accepts F32 only and
//     reports anything else as DeviceMismatch, which is what other dtypes
//     (I32, I8) and mixed dtypes still give here.
//   - gBias is overwritten with sum(gY * act'(Z)) in a fixed order (the
//     reference zero-fills it and accumulates with float atomics).
//   - GemmBatchedLaunch / GemmBatchedBackward are new: the reference's batched
//     callers loop over slices (conv2d/launcher.cu:180-227, sdpa/launcher.cu:185-270).
#pragma once
#include <cstdint>

#include "shim.hpp"

namespace ai::cuda::shim {

// Bias-kind inference, gemm/launcher.cu:47-77 and bias.hpp:70-78.
BiasKind infer_bias_kind_1d_lenMN(const Tensor* Bias, std::int64_t M, std::int64_t N);
BiasKind infer_bias_kind_fallback(const Tensor* Bias, std::int64_t M, std::int64_t N);
BiasKind decide_bias_kind(const Tensor* Bias, std::int64_t M, std::int64_t N);
// gemm/launcher.cu:79-102 (F32 and element count / 2-D shape of the kind)
bool validate_bias_buffer(const Tensor* Bias, std::int64_t M, std::int64_t N, BiasKind kind);

// Forward: Y = act(A[M,K] B[K,N] + bias); Z_saved = pre-activation when attrs.save_z.
Status GemmCudaLaunch(const Tensor& A, const Tensor& B, const Tensor* Bias, Tensor& Y,
                      const GemmAttrs& attrs, StreamHandle stream, Tensor* Z_saved = nullptr,
                      const GemmWorkspace* ws = nullptr);

inline Status GemmCudaLaunch(const Tensor& A, const Tensor& B, Tensor& Y, const GemmAttrs& attrs,
                             StreamHandle stream, Tensor* Z_saved = nullptr,
                             const GemmWorkspace* ws = nullptr) {
  return GemmCudaLaunch(A, B, nullptr, Y, attrs, stream, Z_saved, ws);
}

// Backward: gA = gZ B^T, gB = A^T gZ, gC = gZ (iff C and gC), gBias = reduce(gZ)
// with gZ = gY * act'(Z).
Status GemmCudaBackward(const Tensor& A, const Tensor& B, const Tensor* C, const Tensor& gY,
                        const Tensor& Z, Tensor* gA, Tensor* gB, Tensor* gC, Tensor* gBias,
                        const GemmAttrs& attrs, StreamHandle stream,
                        const GemmWorkspace* ws = nullptr);

// Capture-safe form (gemm/api.hpp:166-188): the dZ buffer (M*N fp32) is the
// operator's dY' workspace, which always suffices (dY' takes M*N elements and
// the dBias partials are parked in the gA or gB output), so the call never
// allocates.  The cuBLASLt workspace is validated and otherwise unused.
inline Status GemmCudaBackwardInto(const Tensor& A, const Tensor& B, const Tensor* C,
                                   const Tensor& gY, const Tensor& Z, Tensor* gA, Tensor* gB,
                                   Tensor* gC, Tensor* gBias, const GemmAttrs& attrs,
                                   StreamHandle stream, float* dZ, void* lt_ws = nullptr,
                                   std::size_t lt_ws_bytes = 0) {
  GemmWorkspace ws{};
  ws.scratch = static_cast<void*>(dZ);
  ws.scratch_bytes = 0;
  ws.lt_workspace = lt_ws;
  ws.lt_workspace_bytes = lt_ws_bytes;
  return GemmCudaBackward(A, B, C, gY, Z, gA, gB, gC, gBias, attrs, stream, &ws);
}

// Batched / strided form.  The tensors describe ONE slice (2-D, row-major,
// leading dimension from stride[0]); slice b of each operand starts
// b * stride_* elements after its data pointer.  attrs.trans_a / trans_b select
// A stored [K,M] / B stored [N,K]; attrs.alpha scales the product (the SDPA
// 1/sqrt(D) scale, sdpa/launcher.cu:63-66,197).  Bias is per slice.
struct GemmBatch {
  std::int64_t count{1};
  std::int64_t stride_a{0}, stride_b{0}, stride_bias{0}, stride_y{0}, stride_z{0};
};
Status GemmBatchedLaunch(const Tensor& A, const Tensor& B, const Tensor* Bias, Tensor& Y,
                         const GemmAttrs& attrs, const GemmBatch& batch, StreamHandle stream,
                         Tensor* Z_saved = nullptr);

struct GemmBatchBwd {
  std::int64_t count{1};
  std::int64_t stride_a{0}, stride_b{0}, stride_gy{0}, stride_z{0};
  std::int64_t stride_ga{0}, stride_gb{0}, stride_gc{0}, stride_gbias{0};
};
Status GemmBatchedBackward(const Tensor& A, const Tensor& B, const Tensor* C, const Tensor& gY,
                           const Tensor& Z, Tensor* gA, Tensor* gB, Tensor* gC, Tensor* gBias,
                           const GemmAttrs& attrs, const GemmBatchBwd& batch, StreamHandle stream);

// Message of the last failing call on this thread (validation reason or the
// HIP error text), "" after a successful call.
const char* GemmLastError();

}  // namespace ai::cuda::shim
