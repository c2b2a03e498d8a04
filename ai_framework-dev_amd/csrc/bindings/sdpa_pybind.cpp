// pybind11 module graph_executor_v2.ops._ops_sdpa (additive: the reference
// declares SDPACudaLaunch / SDPACudaBackwardLaunch, sdpa/api.hpp:19-31, but
// builds no Python module for them).  Raw pointers plus shapes, an SDPAAttrs
// object and an integer stream, in the style of the other _ops_* modules.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "host/sdpa_host.hpp"

namespace py = pybind11;
namespace shim = ai::cuda::shim;

namespace {

shim::Tensor make4(std::uintptr_t ptr, const std::vector<std::int64_t>& s, shim::DType dt) {
  if (s.size() != 4) throw std::invalid_argument("shape must be 4D [B,H,rows,D]");
  shim::Tensor t;
  t.data = reinterpret_cast<void*>(ptr);
  t.device = shim::Device::CUDA;
  t.desc.dtype = dt;
  t.desc.layout = shim::Layout::RowMajor;
  t.desc.shape = s;
  t.desc.stride = {s[1] * s[2] * s[3], s[2] * s[3], s[3], 1};
  return t;
}

void throw_if_bad(shim::Status st, const char* where) {
  if (st != shim::Status::Ok)
    throw std::runtime_error(std::string("[_ops_sdpa::") + where + "] failed with Status=" +
                             std::to_string(static_cast<int>(st)) + ": " + shim::SDPALastError());
}

}  // namespace

PYBIND11_MODULE(_ops_sdpa, m) {
  m.attr("__package__") = "graph_executor_v2.ops";
  m.doc() = "Scaled dot-product attention on gfx950 (MI355X build): Q [B,H,M,D], K/V [B,H,N,D], Y [B,H,M,D], "
            "mask [B,1,M,N] (I8/I32/F32, optional).";
  py::module_ common = py::module_::import("graph_executor_v2.ops._ops_common");
  m.attr("DType") = common.attr("DType");

  py::class_<shim::SDPAAttrs>(m, "SDPAAttrs")
      .def(py::init<>())
      .def_readwrite("scale", &shim::SDPAAttrs::scale)
      .def_readwrite("causal", &shim::SDPAAttrs::causal)
      .def_readwrite("dropout_p", &shim::SDPAAttrs::dropout_p)
      .def_readwrite("scale_in_train", &shim::SDPAAttrs::scale_in_train)
      .def_readwrite("seed", &shim::SDPAAttrs::seed);

  m.def(
      "forward",
      [](std::uintptr_t q, const std::vector<std::int64_t>& qs, std::uintptr_t k, const std::vector<std::int64_t>& ks,
         std::uintptr_t v, const std::vector<std::int64_t>& vs, std::uintptr_t y, const std::vector<std::int64_t>& ys,
         py::object mask_ptr, shim::DType mask_dtype, shim::SDPAAttrs attrs, std::uintptr_t stream,
         shim::DType dtype) {
        shim::Tensor Q = make4(q, qs, dtype), K = make4(k, ks, dtype), V = make4(v, vs, dtype), Y = make4(y, ys, dtype);
        shim::Tensor Mt;
        const shim::Tensor* Mp = nullptr;
        if (!mask_ptr.is_none()) {
          Mt = make4(mask_ptr.cast<std::uintptr_t>(), {qs.at(0), 1, qs.at(2), ks.at(2)}, mask_dtype);
          Mp = &Mt;
        }
        shim::Status st;
        {
          py::gil_scoped_release release;
          st = shim::SDPACudaLaunch(Q, K, V, Mp, Y, attrs, reinterpret_cast<shim::StreamHandle>(stream));
        }
        throw_if_bad(st, "forward");
      },
      py::arg("q_ptr"), py::arg("q_shape"), py::arg("k_ptr"), py::arg("k_shape"), py::arg("v_ptr"), py::arg("v_shape"),
      py::arg("y_ptr"), py::arg("y_shape"), py::arg("mask_ptr") = py::none(), py::arg("mask_dtype") = shim::DType::I8,
      py::arg("attrs") = shim::SDPAAttrs{}, py::arg("stream") = static_cast<std::uintptr_t>(0),
      py::arg("dtype") = shim::DType::F32);

  m.def(
      "backward",
      [](std::uintptr_t q, const std::vector<std::int64_t>& qs, std::uintptr_t k, const std::vector<std::int64_t>& ks,
         std::uintptr_t v, const std::vector<std::int64_t>& vs, std::uintptr_t dy, py::object dq_ptr,
         py::object dk_ptr, py::object dv_ptr, py::object mask_ptr, shim::DType mask_dtype, shim::SDPAAttrs attrs,
         std::uintptr_t stream, shim::DType dtype) {
        shim::Tensor Q = make4(q, qs, dtype), K = make4(k, ks, dtype), V = make4(v, vs, dtype), dY = make4(dy, qs, dtype);
        shim::Tensor dQt, dKt, dVt, Mt;
        shim::Tensor *dQ = nullptr, *dK = nullptr, *dV = nullptr;
        const shim::Tensor* Mp = nullptr;
        if (!dq_ptr.is_none()) { dQt = make4(dq_ptr.cast<std::uintptr_t>(), qs, dtype); dQ = &dQt; }
        if (!dk_ptr.is_none()) { dKt = make4(dk_ptr.cast<std::uintptr_t>(), ks, dtype); dK = &dKt; }
        if (!dv_ptr.is_none()) { dVt = make4(dv_ptr.cast<std::uintptr_t>(), vs, dtype); dV = &dVt; }
        if (!mask_ptr.is_none()) {
          Mt = make4(mask_ptr.cast<std::uintptr_t>(), {qs.at(0), 1, qs.at(2), ks.at(2)}, mask_dtype);
          Mp = &Mt;
        }
        shim::Status st;
        {
          py::gil_scoped_release release;
          st = shim::SDPACudaBackwardLaunch(Q, K, V, dY, Mp, dQ, dK, dV, attrs,
                                            reinterpret_cast<shim::StreamHandle>(stream));
        }
        throw_if_bad(st, "backward");
      },
      py::arg("q_ptr"), py::arg("q_shape"), py::arg("k_ptr"), py::arg("k_shape"), py::arg("v_ptr"), py::arg("v_shape"),
      py::arg("dy_ptr"), py::arg("dq_ptr") = py::none(), py::arg("dk_ptr") = py::none(),
      py::arg("dv_ptr") = py::none(), py::arg("mask_ptr") = py::none(), py::arg("mask_dtype") = shim::DType::I8,
      py::arg("attrs") = shim::SDPAAttrs{}, py::arg("stream") = static_cast<std::uintptr_t>(0),
      py::arg("dtype") = shim::DType::F32);
}
