// graph_executor_v2.ops._ops_common: the operator types shared by the op
// modules (reference: src/bindings/ops_common_pybind.cpp:25-145).  Same
// names, enum values, fields and make_tensor_2d signature; GemmAttrs also
// exposes alpha (used by the batched entry points only).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <vector>

#include "host/shim.hpp"

namespace py = pybind11;
namespace shim = ::ai::cuda::shim;

PYBIND11_MODULE(_ops_common, m) {
  m.attr("__package__") = "graph_executor_v2.ops";
  m.doc() = "Shared operator types: ActKind, GemmAttrs, Device, DType, Layout, TensorDesc, "
            "Tensor, make_tensor_2d (MI355X build).";

  py::enum_<shim::ActKind>(m, "ActKind", py::arithmetic())
      .value("None", shim::ActKind::None)
      .value("ReLU", shim::ActKind::ReLU)
      .value("LeakyReLU", shim::ActKind::LeakyReLU)
      .value("GELU", shim::ActKind::GELU)
      .value("Sigmoid", shim::ActKind::Sigmoid)
      .value("Tanh", shim::ActKind::Tanh)
      .export_values();

  py::class_<shim::GemmAttrs>(m, "GemmAttrs")
      .def(py::init<>())
      .def_readwrite("trans_a", &shim::GemmAttrs::trans_a)
      .def_readwrite("trans_b", &shim::GemmAttrs::trans_b)
      .def_readwrite("act", &shim::GemmAttrs::act)
      .def_readwrite("with_bias", &shim::GemmAttrs::with_bias)
      .def_readwrite("leaky_slope", &shim::GemmAttrs::leaky_slope)
      .def_readwrite("save_z", &shim::GemmAttrs::save_z)
      .def_readwrite("alpha", &shim::GemmAttrs::alpha);

  py::enum_<shim::Device>(m, "Device", py::arithmetic())
      .value("CPU", shim::Device::CPU)
      .value("CUDA", shim::Device::CUDA)
      .export_values();

  py::enum_<shim::DType>(m, "DType", py::arithmetic())
      .value("F32", shim::DType::F32)
      .value("F16", shim::DType::F16)
      .value("BF16", shim::DType::BF16)
      .value("I32", shim::DType::I32)
      .value("I8", shim::DType::I8)
      .export_values();

  py::enum_<shim::Layout>(m, "Layout", py::arithmetic())
      .value("RowMajor", shim::Layout::RowMajor)
      .value("ColMajor", shim::Layout::ColMajor)
      .export_values();

  py::class_<shim::TensorDesc>(m, "TensorDesc")
      .def(py::init<>())
      .def_readwrite("dtype", &shim::TensorDesc::dtype)
      .def_readwrite("layout", &shim::TensorDesc::layout)
      .def_readwrite("shape", &shim::TensorDesc::shape)
      .def_readwrite("stride", &shim::TensorDesc::stride)
      .def("dim", &shim::TensorDesc::dim);

  py::class_<shim::Tensor>(m, "Tensor")
      .def(py::init<>())
      .def_property(
          "data_u64",
          [](const shim::Tensor& t) { return reinterpret_cast<std::uintptr_t>(t.data); },
          [](shim::Tensor& t, std::uintptr_t p) { t.data = reinterpret_cast<void*>(p); })
      .def_readwrite("desc", &shim::Tensor::desc)
      .def_readwrite("device", &shim::Tensor::device)
      .def_readwrite("device_index", &shim::Tensor::device_index)
      .def("is_cuda", &shim::Tensor::is_cuda)
      .def("is_contiguous_rowmajor_2d", &shim::Tensor::is_contiguous_rowmajor_2d);

  m.def(
      "make_tensor_2d",
      [](std::uintptr_t ptr_u64, const std::vector<std::int64_t>& shape, shim::DType dtype,
         shim::Device device, int device_index) {
        if (shape.size() != 2) throw std::invalid_argument("make_tensor_2d: shape must be 2D");
        shim::Tensor t = shim::make_tensor2d(reinterpret_cast<void*>(ptr_u64), shape[0], shape[1], dtype);
        t.device = device;
        t.device_index = device_index;
        return t;
      },
      py::arg("ptr_u64"), py::arg("shape"), py::arg("dtype") = shim::DType::F32,
      py::arg("device") = shim::Device::CUDA, py::arg("device_index") = 0);

  m.attr("__all__") = py::make_tuple("ActKind", "GemmAttrs", "Device", "DType", "Layout",
                                     "TensorDesc", "Tensor", "make_tensor_2d");
}
