// pybind11 module graph_executor_v2.ops._ops_conv2d: the reference's conv2d
// binding surface (src/bindings/conv2d_pybind.cpp:60-258) over this build's
// Conv2DCudaLaunch / Conv2DCudaBackwardLaunch: raw pointers plus shapes, a
// Conv2DAttrs object, an integer stream, and the workspace pointers with the
// reference's binding-level checks.  Additive keywords: dtype (F16 / BF16
// tensors) and the workspace sizes dCol_bytes (forward and backward),
// dTmp_bytes and W_CK_bytes (backward), which let one launch cover several
// images; 0 means the reference's per-image size.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../host/conv2d_host.hpp"

namespace py = pybind11;
namespace shim = ai::cuda::shim;

namespace {

shim::Tensor make_tensor_4d(std::uintptr_t ptr, const std::vector<std::int64_t>& shape, shim::DType dt) {
  if (shape.size() != 4) throw std::invalid_argument("shape must be 4D [N,C,H,W]");
  shim::Tensor t;
  t.data = reinterpret_cast<void*>(ptr);
  t.device = shim::Device::CUDA;
  t.desc.dtype = dt;
  t.desc.layout = shim::Layout::RowMajor;
  t.desc.shape = shape;
  t.desc.stride = {shape[1] * shape[2] * shape[3], shape[2] * shape[3], shape[3], 1};
  return t;
}

shim::Tensor make_tensor_1d(std::uintptr_t ptr, std::int64_t len) {
  shim::Tensor t;
  t.data = reinterpret_cast<void*>(ptr);
  t.device = shim::Device::CUDA;
  t.desc.dtype = shim::DType::F32;
  t.desc.layout = shim::Layout::RowMajor;
  t.desc.shape = {len};
  t.desc.stride = {1};
  return t;
}

void throw_if_bad(shim::Status st, const char* where) {
  if (st != shim::Status::Ok)
    throw std::runtime_error(std::string("[_ops_conv2d::") + where + "] failed with Status=" +
                             std::to_string(static_cast<int>(st)) + ": " + shim::Conv2DLastError());
}

}  // namespace

PYBIND11_MODULE(_ops_conv2d, m) {
  m.attr("__package__") = "graph_executor_v2.ops";
  m.doc() = "conv2d on the gfx950 GEMM operator (MI355X build): X [N,Cin,H,W], W [Cout,Cin,Kh,Kw], "
            "B [Cout], Y/Z [N,Cout,Ho,Wo].";
  py::module_ common = py::module_::import("graph_executor_v2.ops._ops_common");
  m.attr("ActKind") = common.attr("ActKind");
  m.attr("DType") = common.attr("DType");

  py::class_<shim::Conv2DAttrs>(m, "Conv2DAttrs")
      .def(py::init<>())
      .def_readwrite("stride_h", &shim::Conv2DAttrs::stride_h)
      .def_readwrite("stride_w", &shim::Conv2DAttrs::stride_w)
      .def_readwrite("pad_h", &shim::Conv2DAttrs::pad_h)
      .def_readwrite("pad_w", &shim::Conv2DAttrs::pad_w)
      .def_readwrite("dil_h", &shim::Conv2DAttrs::dil_h)
      .def_readwrite("dil_w", &shim::Conv2DAttrs::dil_w)
      .def_readwrite("groups", &shim::Conv2DAttrs::groups)
      .def_readwrite("with_bias", &shim::Conv2DAttrs::with_bias)
      .def_readwrite("act", &shim::Conv2DAttrs::act)
      .def_readwrite("leaky_slope", &shim::Conv2DAttrs::leaky_slope)
      .def_readwrite("save_z", &shim::Conv2DAttrs::save_z);

  m.def(
      "forward",
      [](std::uintptr_t x_ptr, const std::vector<std::int64_t>& x_shape, std::uintptr_t w_ptr,
         const std::vector<std::int64_t>& w_shape, std::uintptr_t y_ptr, const std::vector<std::int64_t>& y_shape,
         py::object b_ptr_obj, py::object z_ptr_obj, shim::Conv2DAttrs attrs, std::uintptr_t stream_ptr,
         std::uintptr_t dCol_ptr, std::uintptr_t W_KC_ptr, std::uintptr_t Y_tmp_ptr, std::uintptr_t Z_rows_ptr,
         shim::DType dtype, std::size_t dCol_bytes) {
        shim::Tensor X = make_tensor_4d(x_ptr, x_shape, dtype);
        shim::Tensor W = make_tensor_4d(w_ptr, w_shape, dtype);
        shim::Tensor Y = make_tensor_4d(y_ptr, y_shape, dtype);
        shim::Tensor B, Zt;
        const shim::Tensor* Bp = nullptr;
        shim::Tensor* Zp = nullptr;
        if (!b_ptr_obj.is_none()) {
          B = make_tensor_1d(b_ptr_obj.cast<std::uintptr_t>(), w_shape.at(0));
          Bp = &B;
        }
        if (!z_ptr_obj.is_none()) {
          Zt = make_tensor_4d(z_ptr_obj.cast<std::uintptr_t>(), y_shape, dtype);
          Zp = &Zt;
        }
        shim::Conv2DWorkspaceFwd ws{};
        ws.dCol = reinterpret_cast<float*>(dCol_ptr);
        ws.W_KC = reinterpret_cast<float*>(W_KC_ptr);
        ws.Y_tmp = reinterpret_cast<float*>(Y_tmp_ptr);
        ws.Z_rows = reinterpret_cast<float*>(Z_rows_ptr);
        ws.dCol_bytes = dCol_bytes;
        // the reference's binding-level checks (conv2d_pybind.cpp:137-145)
        if (!ws.dCol || !ws.W_KC || !ws.Y_tmp)
          throw std::invalid_argument("[_ops_conv2d.forward] workspace pointers (dCol, W_KC, Y_tmp) are required");
        if (attrs.save_z && Zp == nullptr)
          throw std::invalid_argument("[_ops_conv2d.forward] attrs.save_z=True requires z_ptr (Z_saved)");
        if (attrs.save_z && !ws.Z_rows)
          throw std::invalid_argument("[_ops_conv2d.forward] attrs.save_z=True requires Z_rows workspace");
        shim::Status st;
        {
          py::gil_scoped_release release;
          st = shim::Conv2DCudaLaunch(X, W, Bp, Y, attrs, reinterpret_cast<shim::StreamHandle>(stream_ptr), Zp, &ws);
        }
        throw_if_bad(st, "forward");
      },
      py::arg("x_ptr"), py::arg("x_shape"), py::arg("w_ptr"), py::arg("w_shape"), py::arg("y_ptr"),
      py::arg("y_shape"), py::arg("bias_ptr") = py::none(), py::arg("z_ptr") = py::none(),
      py::arg("attrs") = shim::Conv2DAttrs{}, py::arg("stream") = static_cast<std::uintptr_t>(0),
      py::arg("dCol_ptr") = static_cast<std::uintptr_t>(0), py::arg("W_KC_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("Y_tmp_ptr") = static_cast<std::uintptr_t>(0), py::arg("Z_rows_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("dtype") = shim::DType::F32, py::arg("dCol_bytes") = static_cast<std::size_t>(0));

  m.def(
      "backward",
      [](std::uintptr_t x_ptr, const std::vector<std::int64_t>& x_shape, std::uintptr_t w_ptr,
         const std::vector<std::int64_t>& w_shape, std::uintptr_t dy_ptr, const std::vector<std::int64_t>& dy_shape,
         std::uintptr_t z_ptr, const std::vector<std::int64_t>& z_shape, py::object dw_obj, py::object db_obj,
         py::object dx_obj, shim::Conv2DAttrs attrs, std::uintptr_t stream_ptr, std::uintptr_t dCol_ptr,
         std::uintptr_t dTmp_ptr, std::uintptr_t W_CK_ptr, std::uintptr_t dWpack_ptr, std::uintptr_t dY_HT_ptr,
         std::uintptr_t gy_rows_ptr, std::uintptr_t Z_rows_ptr, shim::DType dtype, std::size_t dCol_bytes,
         std::size_t dTmp_bytes, std::size_t W_CK_bytes) {
        shim::Tensor X = make_tensor_4d(x_ptr, x_shape, dtype);
        shim::Tensor W = make_tensor_4d(w_ptr, w_shape, dtype);
        shim::Tensor dY = make_tensor_4d(dy_ptr, dy_shape, dtype);
        shim::Tensor Z = make_tensor_4d(z_ptr, z_shape, dtype);
        shim::Tensor dWt, dBt, dXt;
        shim::Tensor *dW = nullptr, *dB = nullptr, *dX = nullptr;
        if (!dw_obj.is_none()) {
          dWt = make_tensor_4d(dw_obj.cast<std::uintptr_t>(), w_shape, dtype);
          dW = &dWt;
        }
        if (!db_obj.is_none()) {
          dBt = make_tensor_1d(db_obj.cast<std::uintptr_t>(), w_shape.at(0));
          dB = &dBt;
        }
        if (!dx_obj.is_none()) {
          dXt = make_tensor_4d(dx_obj.cast<std::uintptr_t>(), x_shape, dtype);
          dX = &dXt;
        }
        shim::Conv2DWorkspaceBwd ws{};
        ws.dCol = reinterpret_cast<float*>(dCol_ptr);
        ws.dTmp = reinterpret_cast<float*>(dTmp_ptr);
        ws.W_CK = reinterpret_cast<float*>(W_CK_ptr);
        ws.dWpack = reinterpret_cast<float*>(dWpack_ptr);
        ws.dY_HT = reinterpret_cast<float*>(dY_HT_ptr);
        ws.gy_rows = reinterpret_cast<float*>(gy_rows_ptr);
        ws.Z_rows = reinterpret_cast<float*>(Z_rows_ptr);
        ws.dCol_bytes = dCol_bytes;
        ws.dTmp_bytes = dTmp_bytes;
        ws.W_CK_bytes = W_CK_bytes;
        // the reference's binding-level checks (conv2d_pybind.cpp:225-239)
        if (!ws.dCol || !ws.dTmp)
          throw std::invalid_argument("[_ops_conv2d.backward] workspace dCol_ptr and dTmp_ptr are required");
        if (!ws.gy_rows || !ws.Z_rows)
          throw std::invalid_argument("[_ops_conv2d.backward] workspace gy_rows_ptr and Z_rows_ptr are required");
        if (dX && (!ws.W_CK || !ws.dY_HT))
          throw std::invalid_argument("[_ops_conv2d.backward] gX path requires W_CK_ptr and dY_HT_ptr workspaces");
        if (dW && !ws.dWpack)
          throw std::invalid_argument("[_ops_conv2d.backward] gW path requires dWpack_ptr workspace");
        shim::Status st;
        {
          py::gil_scoped_release release;
          st = shim::Conv2DCudaBackwardLaunch(X, W, dY, Z, dW, dB, dX, attrs,
                                              reinterpret_cast<shim::StreamHandle>(stream_ptr), &ws);
        }
        throw_if_bad(st, "backward");
      },
      py::arg("x_ptr"), py::arg("x_shape"), py::arg("w_ptr"), py::arg("w_shape"), py::arg("dy_ptr"),
      py::arg("dy_shape"), py::arg("z_ptr"), py::arg("z_shape"), py::arg("dw_ptr") = py::none(),
      py::arg("db_ptr") = py::none(), py::arg("dx_ptr") = py::none(), py::arg("attrs") = shim::Conv2DAttrs{},
      py::arg("stream") = static_cast<std::uintptr_t>(0), py::arg("dCol_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("dTmp_ptr") = static_cast<std::uintptr_t>(0), py::arg("W_CK_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("dWpack_ptr") = static_cast<std::uintptr_t>(0), py::arg("dY_HT_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("gy_rows_ptr") = static_cast<std::uintptr_t>(0), py::arg("Z_rows_ptr") = static_cast<std::uintptr_t>(0),
      py::arg("dtype") = shim::DType::F32, py::arg("dCol_bytes") = static_cast<std::size_t>(0),
      py::arg("dTmp_bytes") = static_cast<std::size_t>(0), py::arg("W_CK_bytes") = static_cast<std::size_t>(0));
}
