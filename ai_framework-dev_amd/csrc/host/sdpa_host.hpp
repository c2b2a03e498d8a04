// C++ operator API of scaled dot-product attention (host side).
//
// Same attribute struct and entry points as the reference's
// graph_executor_v2/backends/cuda/ops/sdpa/api.hpp:8-31 (implemented in
// sdpa/launcher.cu:129-747): Q [B,H,M,D], K / V [B,H,N,D], Y [B,H,M,D], an
// optional mask [B,1,M,N] (I8 / I32: non-zero masks; F32: added).  Like the
// reference these calls take no workspace and allocate what they need for
// the call; callers that cannot allocate use gev2_sdpa_fwd / gev2_sdpa_bwd with
// a workspace instead.
// Differences a caller can observe: F16 / BF16 tensors are accepted (with
// D = 64 or 128 the forward and backward are fused kernels, dropout
// included).
#pragma once
#include <cstdint>

#include "shim.hpp"

namespace ai::cuda::shim {

struct SDPAAttrs {
  float scale{0.f};          // 0: 1/sqrt(D)
  bool causal{false};
  float dropout_p{0.f};
  bool scale_in_train{true};
  std::uint64_t seed{0};
};

Status SDPACudaLaunch(const Tensor& Q, const Tensor& K, const Tensor& V, const Tensor* mask, Tensor& Y,
                      const SDPAAttrs& attrs, StreamHandle stream);

Status SDPACudaBackwardLaunch(const Tensor& Q, const Tensor& K, const Tensor& V, const Tensor& dY, const Tensor* mask,
                              Tensor* dQ, Tensor* dK, Tensor* dV, const SDPAAttrs& attrs, StreamHandle stream);

// Message of the last failing call on this thread.
const char* SDPALastError();

}  // namespace ai::cuda::shim
