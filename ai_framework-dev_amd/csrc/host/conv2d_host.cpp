// Host side of conv2d: validation in the reference's order and with its
// Status results (conv2d/launcher.cu:110-144, 241-276), then one call into
// the C ABI of libgev2.so.
#include "conv2d_host.hpp"

#include <string>

#include "gev2_gemm.h"

namespace ai::cuda::shim {
namespace {

thread_local std::string t_err;

Status fail(Status s, const char* why) {
  t_err = why;
  return s;
}

bool is_float(DType d) { return d == DType::F32 || d == DType::F16 || d == DType::BF16; }

// is4_f32_cuda (launcher.cu:31-34), widened to one float storage type
bool is4(const Tensor& t, DType dt) {
  return t.device == Device::CUDA && t.desc.dtype == dt && t.desc.layout == Layout::RowMajor &&
         t.desc.shape.size() == 4;
}

bool is1_f32(const Tensor& t) {
  return t.device == Device::CUDA && t.desc.dtype == DType::F32 && t.desc.layout == Layout::RowMajor &&
         t.desc.shape.size() == 1;
}

Status from_abi(int st) {
  if (st != GEV2_OK) t_err = gev2_conv2d_last_error();
  return static_cast<Status>(st);
}

template <typename D>
void fill_geometry(D& d, const Tensor& X, const Tensor& W, const Conv2DAttrs& a) {
  d.dtype = static_cast<int32_t>(X.desc.dtype);
  d.act = static_cast<int32_t>(a.act);
  d.leaky_slope = a.leaky_slope;
  d.N = static_cast<int32_t>(X.desc.shape[0]);
  d.Cin = static_cast<int32_t>(X.desc.shape[1]);
  d.H = static_cast<int32_t>(X.desc.shape[2]);
  d.W = static_cast<int32_t>(X.desc.shape[3]);
  d.Cout = static_cast<int32_t>(W.desc.shape[0]);
  d.Kh = static_cast<int32_t>(W.desc.shape[2]);
  d.Kw = static_cast<int32_t>(W.desc.shape[3]);
  d.stride_h = a.stride_h; d.stride_w = a.stride_w;
  d.pad_h = a.pad_h; d.pad_w = a.pad_w;
  d.dil_h = a.dil_h; d.dil_w = a.dil_w;
  d.groups = a.groups;
}

bool out_size(const Tensor& X, const Tensor& W, const Conv2DAttrs& a, std::int64_t* Ho, std::int64_t* Wo) {
  if (a.stride_h <= 0 || a.stride_w <= 0 || a.dil_h <= 0 || a.dil_w <= 0) return false;
  *Ho = (X.desc.shape[2] + 2 * a.pad_h - a.dil_h * (W.desc.shape[2] - 1) - 1) / a.stride_h + 1;
  *Wo = (X.desc.shape[3] + 2 * a.pad_w - a.dil_w * (W.desc.shape[3] - 1) - 1) / a.stride_w + 1;
  return true;
}

bool shape4(const Tensor& t, std::int64_t a, std::int64_t b, std::int64_t c, std::int64_t d) {
  const auto& s = t.desc.shape;
  return s[0] == a && s[1] == b && s[2] == c && s[3] == d;
}

}  // namespace

const char* Conv2DLastError() { return t_err.c_str(); }

Status Conv2DCudaLaunch(const Tensor& X, const Tensor& W, const Tensor* B, Tensor& Y, const Conv2DAttrs& a,
                        StreamHandle stream, Tensor* Z_saved, const Conv2DWorkspaceFwd* ws) {
  t_err.clear();
  const DType dt = X.desc.dtype;
  if (!is_float(dt) || !is4(X, dt) || !is4(Y, dt)) return fail(Status::Invalid, "X / Y must be 4-D row-major");
  if (!is4(W, dt)) return fail(Status::Invalid, "W must be 4-D row-major of X's dtype");
  if (a.groups != 1) return fail(Status::Unimplemented, "groups != 1");
  if (!ws || !ws->dCol) return fail(Status::MissingInput, "the dCol workspace is required");
  if (W.desc.shape[1] != X.desc.shape[1]) return fail(Status::ShapeMismatch, "W.Cin != X.Cin");
  std::int64_t Ho = 0, Wo = 0;
  if (!out_size(X, W, a, &Ho, &Wo)) return fail(Status::Invalid, "non-positive stride or dilation");
  if (!shape4(Y, X.desc.shape[0], W.desc.shape[0], Ho, Wo)) return fail(Status::ShapeMismatch, "Y shape");
  for (int i = 0; i < 4; ++i)
    if (X.desc.shape[i] <= 0 || W.desc.shape[i] <= 0) return fail(Status::Invalid, "non-positive dimension");
  if (Ho <= 0 || Wo <= 0) return fail(Status::Invalid, "empty output");
  const bool want_z = a.save_z && Z_saved != nullptr;
  if (want_z) {
    if (!is4(*Z_saved, dt)) return fail(Status::Invalid, "Z_saved must match Y");
    if (!shape4(*Z_saved, X.desc.shape[0], W.desc.shape[0], Ho, Wo)) return fail(Status::ShapeMismatch, "Z shape");
  }
  const bool has_bias = B && B->data && a.with_bias;
  if (has_bias && !(is1_f32(*B) && B->desc.shape[0] == W.desc.shape[0]))
    return fail(Status::ShapeMismatch, "bias must be F32 [Cout]");

  gev2_conv2d_desc d{};
  fill_geometry(d, X, W, a);
  d.save_z = want_z ? 1 : 0;
  d.X = X.data; d.Wt = W.data; d.Y = Y.data;
  d.bias = has_bias ? static_cast<const float*>(B->data) : nullptr;
  d.Z = want_z ? Z_saved->data : nullptr;
  d.col = ws->dCol;
  const std::int64_t per_img = X.desc.shape[1] * W.desc.shape[2] * W.desc.shape[3] * Ho * Wo *
                               static_cast<std::int64_t>(dtype_size(dt));
  d.col_bytes = ws->dCol_bytes ? static_cast<std::int64_t>(ws->dCol_bytes) : per_img;
  return from_abi(gev2_conv2d_fwd(&d, stream));
}

Status Conv2DCudaBackwardLaunch(const Tensor& X, const Tensor& W, const Tensor& dY, const Tensor& Z, Tensor* dW,
                                Tensor* dB, Tensor* dX, const Conv2DAttrs& a, StreamHandle stream,
                                const Conv2DWorkspaceBwd* ws) {
  t_err.clear();
  const DType dt = X.desc.dtype;
  if (!is_float(dt) || !is4(X, dt) || !is4(W, dt) || !is4(dY, dt) || !is4(Z, dt))
    return fail(Status::Invalid, "X / W / dY / Z must be 4-D row-major of one dtype");
  if (a.groups != 1) return fail(Status::Unimplemented, "groups != 1");
  if (!ws || !ws->dCol) return fail(Status::MissingInput, "the dCol workspace is required");
  if (dX && !ws->dTmp) return fail(Status::MissingInput, "dX needs the dTmp workspace");
  if (dW && (!ws->W_CK || !ws->dWpack)) return fail(Status::MissingInput, "dW needs the W_CK and dWpack workspaces");
  if (dB && !ws->gy_rows) return fail(Status::MissingInput, "dB needs the gy_rows workspace");
  if (W.desc.shape[1] != X.desc.shape[1]) return fail(Status::ShapeMismatch, "W.Cin != X.Cin");
  std::int64_t Ho = 0, Wo = 0;
  if (!out_size(X, W, a, &Ho, &Wo)) return fail(Status::Invalid, "non-positive stride or dilation");
  const std::int64_t N = X.desc.shape[0], Cout = W.desc.shape[0];
  if (!shape4(dY, N, Cout, Ho, Wo) || !shape4(Z, N, Cout, Ho, Wo)) return fail(Status::ShapeMismatch, "dY / Z shape");
  if (dW && !(is4(*dW, dt) && shape4(*dW, Cout, X.desc.shape[1], W.desc.shape[2], W.desc.shape[3])))
    return fail(Status::ShapeMismatch, "dW shape");
  if (dB && !(is1_f32(*dB) && dB->desc.shape[0] == Cout)) return fail(Status::ShapeMismatch, "dB shape");
  if (dX && !(is4(*dX, dt) && shape4(*dX, N, X.desc.shape[1], X.desc.shape[2], X.desc.shape[3])))
    return fail(Status::ShapeMismatch, "dX shape");
  for (int i = 0; i < 4; ++i)
    if (X.desc.shape[i] <= 0 || W.desc.shape[i] <= 0) return fail(Status::Invalid, "non-positive dimension");
  if (Ho <= 0 || Wo <= 0) return fail(Status::Invalid, "empty output");

  gev2_conv2d_bwd_desc d{};
  fill_geometry(d, X, W, a);
  d.X = X.data; d.Wt = W.data; d.dY = dY.data; d.Z = Z.data;
  d.dW = dW ? dW->data : nullptr;
  d.dB = dB ? static_cast<float*>(dB->data) : nullptr;
  d.dX = dX ? dX->data : nullptr;
  // the reference's sizes: dCol [HWo,K], dTmp max(Cout*K, HWo*K) floats, W_CK
  // [Cout,K] floats, gy_rows [Cout,HWo] floats, dY_HT [HWo,Cout] floats
  const std::int64_t K = X.desc.shape[1] * W.desc.shape[2] * W.desc.shape[3], HWo = Ho * Wo;
  const std::int64_t es = static_cast<std::int64_t>(dtype_size(dt));
  auto given = [](std::size_t b, std::int64_t dflt) { return b ? static_cast<std::int64_t>(b) : dflt; };
  d.col = ws->dCol;
  d.col_bytes = given(ws->dCol_bytes, K * HWo * es);
  d.dcol = ws->dTmp;
  d.dcol_bytes = given(ws->dTmp_bytes, (Cout * K > HWo * K ? Cout * K : HWo * K) * 4);
  d.gw = ws->W_CK;
  d.gw_bytes = given(ws->W_CK_bytes, Cout * K * 4);
  d.acc_w = ws->dWpack;
  d.acc_b = ws->gy_rows;
  d.acc_b_bytes = ws->gy_rows ? Cout * HWo * 4 : 0;
  d.dz = ws->dY_HT;
  d.dz_bytes = ws->dY_HT ? Cout * HWo * 4 : 0;
  return from_abi(gev2_conv2d_bwd(&d, stream));
}

}  // namespace ai::cuda::shim
