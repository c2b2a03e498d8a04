// C++ operator API of conv2d on the GEMM operator (host side).
//
// Same entry points, attribute and workspace structs as the reference's
// graph_executor_v2/backends/cuda/ops/conv2d/api.hpp:5-69 (implemented in
// conv2d/launcher.cu:106-459), so its pybind module and callers bind
// unchanged.  The implementation validates the views and forwards to
// gev2_conv2d_fwd / gev2_conv2d_bwd (include/gev2_gemm.h).
//
// Workspaces: the reference's fields keep their sizes; this build uses
//   forward:  dCol [HWo, K] as the im2col buffer (W_KC, Y_tmp, Z_rows are not
//             needed: the OIHW weights are the GEMM operand as stored and the
//             GEMM writes NCHW directly).  dCol_bytes (additive, 0 = one image)
//             lets one launch cover several images.
//   backward: dCol -> im2col, dTmp -> gradient columns, W_CK -> per-image
//             dW, gy_rows -> fp32 dB sum and per-image dB, dWpack -> fp32 sum
//             of dW, dY_HT -> the dY' scratch; Z_rows unused.  With the
//             reference's sizes that is one image per batched call; the
//             additive *_bytes fields (0 = the reference's size) let one
//             call cover several images.
// Differences a caller can observe: F16 / BF16 tensors are accepted (one
// dtype for X, W, Y, Z, dY, dW, dX; bias and dB stay F32); dB is the sum over
// all images (the reference's per-image GEMM backward zero-fills it, so it
// keeps the last image's only).
#pragma once
#include <cstddef>

#include "shim.hpp"

namespace ai::cuda::shim {

struct Conv2DAttrs {
  int stride_h{1}, stride_w{1};
  int pad_h{0}, pad_w{0};
  int dil_h{1}, dil_w{1};
  int groups{1};
  ActKind act{ActKind::None};
  float leaky_slope{0.01f};
  bool with_bias{false};
  bool save_z{false};
};

struct Conv2DWorkspaceFwd {
  float* dCol{nullptr};     // [HWo, K] (required)
  float* W_KC{nullptr};     // [K, Cout] (accepted, unused)
  float* Y_tmp{nullptr};    // [HWo, Cout] (accepted, unused)
  float* Z_rows{nullptr};   // [HWo, Cout] (accepted, unused)
  std::size_t dCol_bytes{0};   // additive: size of dCol; 0 = one image
};

struct Conv2DWorkspaceBwd {
  float* dCol{nullptr};     // [HWo, K]
  float* dTmp{nullptr};     // max(Cout*K, HWo*K)
  float* W_CK{nullptr};     // [Cout, K]
  float* dY_HT{nullptr};    // [HWo, Cout]
  float* dWpack{nullptr};   // [Cout, K]
  float* gy_rows{nullptr};  // [Cout, HWo]
  float* Z_rows{nullptr};   // [Cout, HWo] (accepted, unused)
  std::size_t dCol_bytes{0};   // additive sizes; 0 = the reference's per-image size
  std::size_t dTmp_bytes{0};
  std::size_t W_CK_bytes{0};
};

Status Conv2DCudaLaunch(const Tensor& X, const Tensor& W, const Tensor* B, Tensor& Y, const Conv2DAttrs& attrs,
                        StreamHandle stream, Tensor* Z_saved = nullptr, const Conv2DWorkspaceFwd* ws_fwd = nullptr);

Status Conv2DCudaBackwardLaunch(const Tensor& X, const Tensor& W, const Tensor& dY, const Tensor& Z, Tensor* dW,
                                Tensor* dB, Tensor* dX, const Conv2DAttrs& attrs, StreamHandle stream,
                                const Conv2DWorkspaceBwd* ws_bwd = nullptr);

// Message of the last failing call on this thread.
const char* Conv2DLastError();

}  // namespace ai::cuda::shim
