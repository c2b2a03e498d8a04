// C++ operator API of the Elman RNN on the GEMM operator (host side).
//
// Same entry points, attribute and workspace structs as the reference's
// graph_executor_v2/backends/cuda/ops/rnn/api.hpp:9-79 (implemented in
// rnn/launcher.cu:129-383), so its pybind module and callers bind unchanged.
// The implementation validates the views in the reference's order
// (launcher.cu:39-127) and forwards to gev2_rnn_fwd / gev2_rnn_bwd
// (include/gev2_gemm.h).
//
// Workspaces keep the reference's fields and sizes; this build uses
//   forward:  XH_cat [N, I+H] and W_cat [I+H, H]; Y_rows / Z_rows are not
//             needed (each step's GEMM writes Y[:,t,:] and Z[:,t,:] in place).
//   backward: XH_cat, G_rows, W_cat, dXH_cat and TmpW as in the reference,
//             dWcat as the fp32 sum of dW over steps, Z_rows' first H floats
//             for one step's dB.
// Differences a caller can observe: F16 / BF16 tensors are accepted (one
// dtype for X, Wx, Wh, h0, Y, Z, dY and the gradients; bias and dB stay F32);
// dB is the sum over all steps (the reference's per-step GEMM backward
// zero-fills it, so it keeps step 0's only).
#pragma once

#include "shim.hpp"

namespace ai::cuda::shim {

struct RnnAttrs {
  ActKind act{ActKind::None};
  float leaky_slope{0.01f};
  bool with_bias{false};
  bool save_z{true};
};

struct RnnWorkspaceFwd {
  float* XH_cat{nullptr};  // [N, I+H] (required)
  float* Y_rows{nullptr};  // [N, H]   (required by the reference; unused)
  float* W_cat{nullptr};   // [I+H, H] (required)
  float* Z_rows{nullptr};  // [N, H]   (required with save_z by the reference; unused)
};

struct RnnWorkspaceBwd {
  float* XH_cat{nullptr};   // [N, I+H]
  float* G_rows{nullptr};   // [N, H]
  float* Z_rows{nullptr};   // [N, H]   (first H floats: one step's dB)
  float* W_cat{nullptr};    // [I+H, H]
  float* dXH_cat{nullptr};  // [N, I+H]
  float* dWcat{nullptr};    // [I+H, H] fp32 sum of dW
  float* TmpW{nullptr};     // [I+H, H]
};

Status RnnCudaLaunch(const Tensor& X, const Tensor& Wx, const Tensor& Wh, const Tensor* B, const Tensor& h0,
                     Tensor& Y, const RnnAttrs& attrs, StreamHandle stream, Tensor* Z_saved = nullptr,
                     const RnnWorkspaceFwd* ws_fwd = nullptr);

Status RnnCudaBackwardLaunch(const Tensor& X, const Tensor& Wx, const Tensor& Wh, const Tensor* B, const Tensor& h0,
                             const Tensor& dY_post, const Tensor& Z, Tensor* dWx, Tensor* dWh, Tensor* dB,
                             Tensor* dh0, Tensor* dX, const RnnAttrs& attrs, StreamHandle stream,
                             const RnnWorkspaceBwd* ws_bwd = nullptr);

// Message of the last failing call on this thread.
const char* RnnLastError();

}  // namespace ai::cuda::shim
