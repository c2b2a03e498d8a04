// pybind11 module graph_executor_v2.ops._ops_rnn: the reference's Elman RNN
// binding surface (src/bindings/rnn_pybind.cpp:74-283) over this build's
// RnnCudaLaunch / RnnCudaBackwardLaunch: raw pointers plus shapes, an
// RnnAttrs object, an integer stream and the workspace pointers, with the
// reference's binding-level checks.  Additive keyword: dtype (F16 / BF16
// tensors; bias and dB stay F32).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "host/rnn_host.hpp"

namespace py = pybind11;
namespace shim = ai::cuda::shim;

namespace {

shim::Tensor make_tensor(std::uintptr_t ptr, const std::vector<std::int64_t>& shape, shim::DType dt,
                         std::size_t rank) {
  if (shape.size() != rank)
    throw std::invalid_argument(std::string("shape must be ") + std::to_string(rank) + "D");
  shim::Tensor t;
  t.data = reinterpret_cast<void*>(ptr);
  t.device = shim::Device::CUDA;
  t.desc.dtype = dt;
  t.desc.layout = shim::Layout::RowMajor;
  t.desc.shape = shape;
  t.desc.stride.assign(rank, 1);
  for (std::size_t i = rank - 1; i-- > 0;) t.desc.stride[i] = t.desc.stride[i + 1] * shape[i + 1];
  return t;
}

shim::Tensor make_tensor_1d(std::uintptr_t ptr, std::int64_t len) {
  return make_tensor(ptr, {len}, shim::DType::F32, 1);
}

void throw_if_bad(shim::Status st, const char* where) {
  if (st != shim::Status::Ok)
    throw std::runtime_error(std::string("[_ops_rnn::") + where + "] failed with Status=" +
                             std::to_string(static_cast<int>(st)) + ": " + shim::RnnLastError());
}

}  // namespace

PYBIND11_MODULE(_ops_rnn, m) {
  m.attr("__package__") = "graph_executor_v2.ops";
  m.doc() = "Elman RNN on the gfx950 GEMM operator (MI355X build): X [N,T,I], Wx [I,H], Wh [H,H], "
            "h0 [N,H], B [H] (optional), Y/Z [N,T,H].";
  py::module_ common = py::module_::import("graph_executor_v2.ops._ops_common");
  m.attr("ActKind") = common.attr("ActKind");
  m.attr("DType") = common.attr("DType");

  py::class_<shim::RnnAttrs>(m, "RnnAttrs")
      .def(py::init<>())
      .def_readwrite("act", &shim::RnnAttrs::act)
      .def_readwrite("leaky_slope", &shim::RnnAttrs::leaky_slope)
      .def_readwrite("with_bias", &shim::RnnAttrs::with_bias)
      .def_readwrite("save_z", &shim::RnnAttrs::save_z);

  m.def(
      "forward",
      [](std::uintptr_t x_ptr, const std::vector<std::int64_t>& x_shape, std::uintptr_t wx_ptr,
         const std::vector<std::int64_t>& wx_shape, std::uintptr_t wh_ptr, const std::vector<std::int64_t>& wh_shape,
         std::uintptr_t h0_ptr, const std::vector<std::int64_t>& h0_shape, std::uintptr_t y_ptr,
         const std::vector<std::int64_t>& y_shape, py::object b_obj, py::object z_obj, shim::RnnAttrs attrs,
         std::uintptr_t stream_ptr, std::uintptr_t XH_cat_ptr, std::uintptr_t Y_rows_ptr, std::uintptr_t W_cat_ptr,
         std::uintptr_t Z_rows_ptr, shim::DType dtype) {
        shim::Tensor X = make_tensor(x_ptr, x_shape, dtype, 3);
        shim::Tensor Wx = make_tensor(wx_ptr, wx_shape, dtype, 2);
        shim::Tensor Wh = make_tensor(wh_ptr, wh_shape, dtype, 2);
        shim::Tensor h0 = make_tensor(h0_ptr, h0_shape, dtype, 2);
        shim::Tensor Y = make_tensor(y_ptr, y_shape, dtype, 3);
        shim::Tensor B, Zt;
        const shim::Tensor* Bp = nullptr;
        shim::Tensor* Zp = nullptr;
        if (!b_obj.is_none()) {
          B = make_tensor_1d(b_obj.cast<std::uintptr_t>(), wx_shape.at(1));
          Bp = &B;
        }
        if (!z_obj.is_none()) {
          Zt = make_tensor(z_obj.cast<std::uintptr_t>(), y_shape, dtype, 3);
          Zp = &Zt;
        }
        shim::RnnWorkspaceFwd ws{};
        ws.XH_cat = reinterpret_cast<float*>(XH_cat_ptr);
        ws.Y_rows = reinterpret_cast<float*>(Y_rows_ptr);
        ws.W_cat = reinterpret_cast<float*>(W_cat_ptr);
        ws.Z_rows = reinterpret_cast<float*>(Z_rows_ptr);
        // the reference's binding-level checks (rnn_pybind.cpp:144-152)
        if (!ws.XH_cat || !ws.Y_rows || !ws.W_cat)
          throw std::invalid_argument("[_ops_rnn.forward] workspace pointers (XH_cat, Y_rows, W_cat) are required");
        if (attrs.save_z && Zp == nullptr)
          throw std::invalid_argument("[_ops_rnn.forward] attrs.save_z=True requires z_ptr (Z_saved)");
        if (attrs.save_z && !ws.Z_rows)
          throw std::invalid_argument("[_ops_rnn.forward] attrs.save_z=True requires Z_rows workspace");
        shim::Status st;
        {
          py::gil_scoped_release release;
          st = shim::RnnCudaLaunch(X, Wx, Wh, Bp, h0, Y, attrs, reinterpret_cast<shim::StreamHandle>(stream_ptr), Zp,
                                   &ws);
        }
        throw_if_bad(st, "forward");
      },
      py::arg("x_ptr"), py::arg("x_shape"), py::arg("wx_ptr"), py::arg("wx_shape"), py::arg("wh_ptr"),
      py::arg("wh_shape"), py::arg("h0_ptr"), py::arg("h0_shape"), py::arg("y_ptr"), py::arg("y_shape"),
      py::arg("bias_ptr") = py::none(), py::arg("z_ptr") = py::none(), py::arg("attrs") = shim::RnnAttrs{},
      py::arg("stream") = static_cast<std::uintptr_t>(0), py::arg("XH_cat_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("Y_rows_ptr") = static_cast<std::uintptr_t>(0), py::arg("W_cat_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("Z_rows_ptr") = static_cast<std::uintptr_t>(0), py::arg("dtype") = shim::DType::F32);

  m.def(
      "backward",
      [](std::uintptr_t x_ptr, const std::vector<std::int64_t>& x_shape, std::uintptr_t wx_ptr,
         const std::vector<std::int64_t>& wx_shape, std::uintptr_t wh_ptr, const std::vector<std::int64_t>& wh_shape,
         std::uintptr_t h0_ptr, const std::vector<std::int64_t>& h0_shape, std::uintptr_t dy_ptr,
         const std::vector<std::int64_t>& dy_shape, std::uintptr_t z_ptr, const std::vector<std::int64_t>& z_shape,
         py::object dwx_obj, py::object dwh_obj, py::object db_obj, py::object dh0_obj, py::object dx_obj,
         shim::RnnAttrs attrs, std::uintptr_t stream_ptr, std::uintptr_t XH_cat_ptr, std::uintptr_t G_rows_ptr,
         std::uintptr_t Z_rows_ptr, std::uintptr_t W_cat_ptr, std::uintptr_t dXH_cat_ptr, std::uintptr_t dWcat_ptr,
         std::uintptr_t TmpW_ptr, shim::DType dtype) {
        shim::Tensor X = make_tensor(x_ptr, x_shape, dtype, 3);
        shim::Tensor Wx = make_tensor(wx_ptr, wx_shape, dtype, 2);
        shim::Tensor Wh = make_tensor(wh_ptr, wh_shape, dtype, 2);
        shim::Tensor h0 = make_tensor(h0_ptr, h0_shape, dtype, 2);
        shim::Tensor dY = make_tensor(dy_ptr, dy_shape, dtype, 3);
        shim::Tensor Z = make_tensor(z_ptr, z_shape, dtype, 3);
        shim::Tensor dWx_t, dWh_t, dB_t, dh0_t, dX_t;
        shim::Tensor *dWx = nullptr, *dWh = nullptr, *dB = nullptr, *dh0 = nullptr, *dX = nullptr;
        if (!dwx_obj.is_none()) {
          dWx_t = make_tensor(dwx_obj.cast<std::uintptr_t>(), wx_shape, dtype, 2);
          dWx = &dWx_t;
        }
        if (!dwh_obj.is_none()) {
          dWh_t = make_tensor(dwh_obj.cast<std::uintptr_t>(), wh_shape, dtype, 2);
          dWh = &dWh_t;
        }
        if (!db_obj.is_none()) {
          dB_t = make_tensor_1d(db_obj.cast<std::uintptr_t>(), wx_shape.at(1));
          dB = &dB_t;
        }
        if (!dh0_obj.is_none()) {
          dh0_t = make_tensor(dh0_obj.cast<std::uintptr_t>(), h0_shape, dtype, 2);
          dh0 = &dh0_t;
        }
        if (!dx_obj.is_none()) {
          dX_t = make_tensor(dx_obj.cast<std::uintptr_t>(), x_shape, dtype, 3);
          dX = &dX_t;
        }
        shim::RnnWorkspaceBwd ws{};
        ws.XH_cat = reinterpret_cast<float*>(XH_cat_ptr);
        ws.G_rows = reinterpret_cast<float*>(G_rows_ptr);
        ws.Z_rows = reinterpret_cast<float*>(Z_rows_ptr);
        ws.W_cat = reinterpret_cast<float*>(W_cat_ptr);
        ws.dXH_cat = reinterpret_cast<float*>(dXH_cat_ptr);
        ws.dWcat = reinterpret_cast<float*>(dWcat_ptr);
        ws.TmpW = reinterpret_cast<float*>(TmpW_ptr);
        // the reference's binding-level check (rnn_pybind.cpp:255-257)
        if (!ws.XH_cat || !ws.G_rows || !ws.Z_rows || !ws.W_cat || !ws.dXH_cat || !ws.dWcat || !ws.TmpW)
          throw std::invalid_argument(
              "[_ops_rnn.backward] all workspace pointers (XH_cat,G_rows,Z_rows,W_cat,dXH_cat,dWcat,TmpW) are "
              "required");
        shim::Status st;
        {
          py::gil_scoped_release release;
          st = shim::RnnCudaBackwardLaunch(X, Wx, Wh, nullptr, h0, dY, Z, dWx, dWh, dB, dh0, dX, attrs,
                                           reinterpret_cast<shim::StreamHandle>(stream_ptr), &ws);
        }
        throw_if_bad(st, "backward");
      },
      py::arg("x_ptr"), py::arg("x_shape"), py::arg("wx_ptr"), py::arg("wx_shape"), py::arg("wh_ptr"),
      py::arg("wh_shape"), py::arg("h0_ptr"), py::arg("h0_shape"), py::arg("dy_ptr"), py::arg("dy_shape"),
      py::arg("z_ptr"), py::arg("z_shape"), py::arg("dwx_ptr") = py::none(), py::arg("dwh_ptr") = py::none(),
      py::arg("db_ptr") = py::none(), py::arg("dh0_ptr") = py::none(), py::arg("dx_ptr") = py::none(),
      py::arg("attrs") = shim::RnnAttrs{}, py::arg("stream") = static_cast<std::uintptr_t>(0),
      py::arg("XH_cat_ptr") = static_cast<std::uintptr_t>(0), py::arg("G_rows_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("Z_rows_ptr") = static_cast<std::uintptr_t>(0), py::arg("W_cat_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("dXH_cat_ptr") = static_cast<std::uintptr_t>(0), py::arg("dWcat_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("TmpW_ptr") = static_cast<std::uintptr_t>(0), py::arg("dtype") = shim::DType::F32);
}
