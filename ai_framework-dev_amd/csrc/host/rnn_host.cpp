// Host side of the Elman RNN: the reference's validation order and Status
// results (rnn/launcher.cu:39-127, 143-146, 270-274), then one call into the
// C ABI of libgev2.so.
#include "rnn_host.hpp"

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

// expect_rowmajor_nd (_common/shim/ai_validate.hpp:44-52) with one allowed
// float storage type: device, layout, rank, contiguity, numel > 0, dtype
Status expect(const Tensor& t, std::size_t rank, DType dt) {
  if (t.device != Device::CUDA) return Status::DeviceMismatch;
  if (t.desc.layout != Layout::RowMajor) return Status::LayoutMismatch;
  if (t.desc.shape.size() != rank) return Status::ShapeMismatch;
  if (t.desc.stride.size() != rank) return Status::StrideMismatch;
  std::int64_t want = 1;
  for (std::size_t i = rank; i-- > 0;) {
    if (t.desc.stride[i] != want) return Status::StrideMismatch;
    want *= t.desc.shape[i];
  }
  if (want <= 0) return Status::ShapeMismatch;
  if (t.desc.dtype != dt) return Status::DtypeMismatch;
  return Status::Ok;
}

Status expect2(const Tensor& t, DType dt, std::int64_t d0, std::int64_t d1) {
  Status s = expect(t, 2, dt);
  if (s != Status::Ok) return s;
  return (t.desc.shape[0] == d0 && t.desc.shape[1] == d1) ? Status::Ok : Status::ShapeMismatch;
}

Status expect3(const Tensor& t, DType dt, std::int64_t d0, std::int64_t d1, std::int64_t d2) {
  Status s = expect(t, 3, dt);
  if (s != Status::Ok) return s;
  return (t.desc.shape[0] == d0 && t.desc.shape[1] == d1 && t.desc.shape[2] == d2) ? Status::Ok
                                                                                    : Status::ShapeMismatch;
}

Status bias_ok(const Tensor& b, std::int64_t H) {
  Status s = expect(b, 1, DType::F32);
  if (s != Status::Ok) return s;
  return b.desc.shape[0] == H ? Status::Ok : Status::ShapeMismatch;
}

Status from_abi(int st) {
  if (st != GEV2_OK) t_err = gev2_rnn_last_error();
  return static_cast<Status>(st);
}

#define RNN_TRY(expr, why)                   \
  do {                                       \
    const Status s_ = (expr);                \
    if (s_ != Status::Ok) return fail(s_, why); \
  } while (0)

}  // namespace

const char* RnnLastError() { return t_err.c_str(); }

Status RnnCudaLaunch(const Tensor& X, const Tensor& Wx, const Tensor& Wh, const Tensor* B, const Tensor& h0,
                     Tensor& Y, const RnnAttrs& a, StreamHandle stream, Tensor* Z_saved, const RnnWorkspaceFwd* ws) {
  t_err.clear();
  const DType dt = X.desc.dtype;
  RNN_TRY(expect(X, 3, dt), "X must be [N,T,I] row-major");
  if (!is_float(dt)) return fail(Status::DtypeMismatch, "X must be F32, F16 or BF16");
  RNN_TRY(expect(Wx, 2, dt), "Wx must be 2-D of X's dtype");
  RNN_TRY(expect(Wh, 2, dt), "Wh must be 2-D of X's dtype");
  RNN_TRY(expect(h0, 2, dt), "h0 must be 2-D of X's dtype");
  RNN_TRY(expect(Y, 3, dt), "Y must be 3-D of X's dtype");
  const std::int64_t N = X.desc.shape[0], T = X.desc.shape[1], I = X.desc.shape[2], H = Wx.desc.shape[1];
  if (Wx.desc.shape[0] != I) return fail(Status::ShapeMismatch, "Wx must be [I,H]");
  if (Wh.desc.shape[0] != H || Wh.desc.shape[1] != H) return fail(Status::ShapeMismatch, "Wh must be [H,H]");
  RNN_TRY(expect3(Y, dt, N, T, H), "Y must be [N,T,H]");
  RNN_TRY(expect2(h0, dt, N, H), "h0 must be [N,H]");
  if (a.with_bias) {
    if (!B) return fail(Status::MissingInput, "with_bias needs B");
    RNN_TRY(bias_ok(*B, H), "B must be F32 [H]");
  }
  const bool want_z = a.save_z && Z_saved != nullptr;
  if (want_z) {
    RNN_TRY(expect3(*Z_saved, dt, N, T, H), "Z must be [N,T,H]");
    if (Z_saved->data == Y.data) return fail(Status::Invalid, "Z must not alias Y");
  }
  // the reference requires every workspace field it uses (launcher.cu:143-146)
  if (!ws || !ws->XH_cat || !ws->Y_rows || !ws->W_cat || (want_z && !ws->Z_rows))
    return fail(Status::MissingInput, "workspaces XH_cat, Y_rows, W_cat (and Z_rows with save_z) are required");

  gev2_rnn_desc d{};
  d.dtype = static_cast<int32_t>(dt);
  d.act = static_cast<int32_t>(a.act);
  d.leaky_slope = a.leaky_slope;
  d.save_z = want_z ? 1 : 0;
  d.N = static_cast<int32_t>(N); d.T = static_cast<int32_t>(T);
  d.I = static_cast<int32_t>(I); d.H = static_cast<int32_t>(H);
  d.X = X.data; d.Wx = Wx.data; d.Wh = Wh.data; d.h0 = h0.data;
  d.bias = (a.with_bias && B) ? static_cast<const float*>(B->data) : nullptr;
  d.Y = Y.data;
  d.Z = want_z ? Z_saved->data : nullptr;
  d.xh = ws->XH_cat;
  d.wcat = ws->W_cat;
  return from_abi(gev2_rnn_fwd(&d, stream));
}

Status RnnCudaBackwardLaunch(const Tensor& X, const Tensor& Wx, const Tensor& Wh, const Tensor* /*B*/,
                             const Tensor& h0, const Tensor& dY, const Tensor& Z, Tensor* dWx, Tensor* dWh,
                             Tensor* dB, Tensor* dh0, Tensor* dX, const RnnAttrs& a, StreamHandle stream,
                             const RnnWorkspaceBwd* ws) {
  t_err.clear();
  const DType dt = X.desc.dtype;
  RNN_TRY(expect(X, 3, dt), "X must be [N,T,I] row-major");
  if (!is_float(dt)) return fail(Status::DtypeMismatch, "X must be F32, F16 or BF16");
  RNN_TRY(expect(Wx, 2, dt), "Wx must be 2-D of X's dtype");
  RNN_TRY(expect(Wh, 2, dt), "Wh must be 2-D of X's dtype");
  RNN_TRY(expect(h0, 2, dt), "h0 must be 2-D of X's dtype");
  RNN_TRY(expect(dY, 3, dt), "dY must be 3-D of X's dtype");
  RNN_TRY(expect(Z, 3, dt), "Z must be 3-D of X's dtype");
  const std::int64_t N = X.desc.shape[0], T = X.desc.shape[1], I = X.desc.shape[2], H = Wx.desc.shape[1];
  RNN_TRY(expect3(Z, dt, N, T, H), "Z must be [N,T,H]");
  if (dWx) RNN_TRY(expect2(*dWx, dt, I, H), "dWx must be [I,H]");
  if (dWh) RNN_TRY(expect2(*dWh, dt, H, H), "dWh must be [H,H]");
  if (a.with_bias && dB) RNN_TRY(bias_ok(*dB, H), "dB must be F32 [H]");
  if (dh0) RNN_TRY(expect2(*dh0, dt, N, H), "dh0 must be [N,H]");
  if (dX) RNN_TRY(expect3(*dX, dt, N, T, I), "dX must be [N,T,I]");
  // shapes the reference leaves to the kernels; checked here so that no launch reads out of bounds
  if (Wx.desc.shape[0] != I) return fail(Status::ShapeMismatch, "Wx must be [I,H]");
  RNN_TRY(expect2(Wh, dt, H, H), "Wh must be [H,H]");
  RNN_TRY(expect2(h0, dt, N, H), "h0 must be [N,H]");
  RNN_TRY(expect3(dY, dt, N, T, H), "dY must be [N,T,H]");
  if (!ws || !ws->XH_cat || !ws->G_rows || !ws->Z_rows || !ws->W_cat || !ws->dXH_cat || !ws->dWcat || !ws->TmpW)
    return fail(Status::MissingInput, "all backward workspaces are required");

  gev2_rnn_bwd_desc d{};
  d.dtype = static_cast<int32_t>(dt);
  d.act = static_cast<int32_t>(a.act);
  d.leaky_slope = a.leaky_slope;
  d.N = static_cast<int32_t>(N); d.T = static_cast<int32_t>(T);
  d.I = static_cast<int32_t>(I); d.H = static_cast<int32_t>(H);
  d.X = X.data; d.Wx = Wx.data; d.Wh = Wh.data; d.h0 = h0.data; d.dY = dY.data; d.Z = Z.data;
  d.dWx = dWx ? dWx->data : nullptr;
  d.dWh = dWh ? dWh->data : nullptr;
  d.dB = (a.with_bias && dB) ? static_cast<float*>(dB->data) : nullptr;
  d.dh0 = dh0 ? dh0->data : nullptr;
  d.dX = dX ? dX->data : nullptr;
  d.xh = ws->XH_cat;
  d.g = ws->G_rows;
  d.wcat = ws->W_cat;
  d.dxh = ws->dXH_cat;
  d.dwcat = ws->dWcat;
  d.tmpw = ws->TmpW;
  d.gb = ws->Z_rows;
  return from_abi(gev2_rnn_bwd(&d, stream));
}

}  // namespace ai::cuda::shim
