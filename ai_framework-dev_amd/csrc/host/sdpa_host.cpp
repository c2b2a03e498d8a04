// Host side of SDPA: the reference's checks and Status results
// (sdpa/launcher.cu:133-156, 333-374), then the C ABI of libgev2.so with a
// workspace allocated for the call (the reference allocates its S / P buffers
// per call as well).
#include "sdpa_host.hpp"

#include <string>

#include "gev2_gemm.h"

namespace ai::cuda::shim {
namespace {

thread_local std::string t_err;

Status fail(Status s, const char* why) {
  t_err = why;
  return s;
}

// is_bhxd_f32_4d_cuda (launcher.cu:28-31), widened to the three float types
bool is_bhxd(const Tensor& t, DType dt) {
  return t.device == Device::CUDA && t.desc.dtype == dt && t.desc.layout == Layout::RowMajor &&
         t.desc.shape.size() == 4;
}

bool is_float(DType d) { return d == DType::F32 || d == DType::F16 || d == DType::BF16; }

int mask_kind(const Tensor* mask) {
  if (!mask) return GEV2_MASK_NONE;
  switch (mask->desc.dtype) {
    case DType::I8: return GEV2_MASK_I8;
    case DType::I32: return GEV2_MASK_I32;
    case DType::F32: return GEV2_MASK_F32;
    default: return -1;
  }
}

bool mask_shape_ok(const Tensor* mask, std::int64_t B, std::int64_t M, std::int64_t N) {
  if (!mask) return true;
  const auto& s = mask->desc.shape;
  return s.size() == 4 && s[0] == B && s[1] == 1 && s[2] == M && s[3] == N;
}

template <typename D>
void fill(D& d, const Tensor& Q, const Tensor& K, const Tensor* mask, const SDPAAttrs& a) {
  d.dtype = static_cast<int32_t>(Q.desc.dtype);
  d.B = static_cast<int32_t>(Q.desc.shape[0]);
  d.H = static_cast<int32_t>(Q.desc.shape[1]);
  d.M = static_cast<int32_t>(Q.desc.shape[2]);
  d.D = static_cast<int32_t>(Q.desc.shape[3]);
  d.N = static_cast<int32_t>(K.desc.shape[2]);
  d.scale = a.scale;
  d.causal = a.causal ? 1 : 0;
  d.dropout_p = a.dropout_p;
  d.seed = a.seed;
  d.scale_in_train = a.scale_in_train ? 1 : 0;
  d.mask_kind = mask_kind(mask);
  d.mask = mask ? mask->data : nullptr;
}

// a workspace for one call, freed on every return path
struct Scratch {
  void* p{nullptr};
  ~Scratch() {
    if (p) {
      (void)gev2_device_synchronize();
      (void)gev2_free(p);
    }
  }
};

Status run(int st) {
  if (st != GEV2_OK) t_err = gev2_sdpa_last_error();
  return static_cast<Status>(st);
}

}  // namespace

const char* SDPALastError() { return t_err.c_str(); }

Status SDPACudaLaunch(const Tensor& Q, const Tensor& K, const Tensor& V, const Tensor* mask, Tensor& Y,
                      const SDPAAttrs& a, StreamHandle stream) {
  t_err.clear();
  const DType dt = Q.desc.dtype;
  if (!is_float(dt) || !is_bhxd(Q, dt) || !is_bhxd(K, dt) || !is_bhxd(V, dt) || !is_bhxd(Y, dt))
    return fail(Status::Invalid, "Q / K / V / Y must be 4-D row-major of one float dtype");
  const auto &q = Q.desc.shape, &k = K.desc.shape, &v = V.desc.shape, &y = Y.desc.shape;
  if (k[0] != q[0] || k[1] != q[1] || k[3] != q[3]) return fail(Status::ShapeMismatch, "K shape");
  if (v[0] != q[0] || v[1] != q[1] || v[2] != k[2] || v[3] != q[3]) return fail(Status::ShapeMismatch, "V shape");
  if (y != q) return fail(Status::ShapeMismatch, "Y shape");
  if (!mask_shape_ok(mask, q[0], q[2], k[2])) return fail(Status::ShapeMismatch, "mask must be [B,1,M,N]");
  if (mask_kind(mask) < 0) return fail(Status::Invalid, "mask dtype must be I8, I32 or F32");
  gev2_sdpa_desc d{};
  fill(d, Q, K, mask, a);
  d.Q = Q.data; d.K = K.data; d.V = V.data; d.Y = Y.data;
  const int64_t wsb = gev2_sdpa_workspace_size(&d, 0);
  if (wsb < 0) return run(gev2_sdpa_fwd(&d, stream));      // reports the descriptor's error
  Scratch ws;
  if (wsb > 0) {
    if (gev2_malloc(&ws.p, static_cast<size_t>(wsb)) != GEV2_OK) return fail(Status::RuntimeError, "workspace allocation");
    d.workspace = ws.p;
    d.workspace_bytes = wsb;
  }
  return run(gev2_sdpa_fwd(&d, stream));
}

Status SDPACudaBackwardLaunch(const Tensor& Q, const Tensor& K, const Tensor& V, const Tensor& dY, const Tensor* mask,
                              Tensor* dQ, Tensor* dK, Tensor* dV, const SDPAAttrs& a, StreamHandle stream) {
  t_err.clear();
  if (!dQ && !dK && !dV) return fail(Status::Invalid, "all outputs null");       // launcher.cu:342
  const DType dt = Q.desc.dtype;
  if (!is_float(dt) || !is_bhxd(Q, dt) || !is_bhxd(K, dt) || !is_bhxd(V, dt) || !is_bhxd(dY, dt))
    return fail(Status::Invalid, "Q / K / V / dY must be 4-D row-major of one float dtype");
  if ((dQ && !is_bhxd(*dQ, dt)) || (dK && !is_bhxd(*dK, dt)) || (dV && !is_bhxd(*dV, dt)))
    return fail(Status::Invalid, "dQ / dK / dV must be 4-D row-major of Q's dtype");
  const auto &q = Q.desc.shape, &k = K.desc.shape, &v = V.desc.shape;
  if (k[0] != q[0] || k[1] != q[1] || k[3] != q[3]) return fail(Status::ShapeMismatch, "K shape");
  if (v[0] != q[0] || v[1] != q[1] || v[2] != k[2] || v[3] != q[3]) return fail(Status::ShapeMismatch, "V shape");
  if (dY.desc.shape != q) return fail(Status::ShapeMismatch, "dY shape");
  if ((dQ && dQ->desc.shape != q) || (dK && dK->desc.shape != k) || (dV && dV->desc.shape != v))
    return fail(Status::ShapeMismatch, "gradient shape");
  if (!mask_shape_ok(mask, q[0], q[2], k[2])) return fail(Status::ShapeMismatch, "mask must be [B,1,M,N]");
  if (mask_kind(mask) < 0) return fail(Status::Invalid, "mask dtype must be I8, I32 or F32");
  gev2_sdpa_bwd_desc d{};
  fill(d, Q, K, mask, a);
  d.Q = Q.data; d.K = K.data; d.V = V.data; d.dY = dY.data;
  d.dQ = dQ ? dQ->data : nullptr;
  d.dK = dK ? dK->data : nullptr;
  d.dV = dV ? dV->data : nullptr;
  gev2_sdpa_desc f{};
  fill(f, Q, K, mask, a);
  const int64_t wsb = gev2_sdpa_workspace_size(&f, 1);
  if (wsb < 0) return run(gev2_sdpa_bwd(&d, stream));
  Scratch ws;
  if (wsb > 0) {
    if (gev2_malloc(&ws.p, static_cast<size_t>(wsb)) != GEV2_OK) return fail(Status::RuntimeError, "workspace allocation");
    d.workspace = ws.p;
    d.workspace_bytes = wsb;
  }
  return run(gev2_sdpa_bwd(&d, stream));
}

}  // namespace ai::cuda::shim
