// graph_executor_v2.ops._ops_gemm: the Python surface of the GEMM + bias +
// activation op (reference: src/bindings/gemm_pybind.cpp:101-687).
//
// Same functions, keyword names, defaults and argument checks:
//   forward, backward, forward_ex, backward_ex, backward_into,
//   forward_ex_attrs, backward_ex_attrs, forward_raw, backward_raw
// plus forward_batched / backward_batched (new: one launch over a strided
// batch, the form the conv2d and SDPA callers need) and a trailing `dtype`
// keyword on the raw-pointer entry points (F32 by default, as in the reference).
// The GIL is released for each native call; calls are stream-ordered and
// asynchronous.  A Status other than Ok becomes RuntimeError("[_ops_gemm::fn]
// ..."), except InvalidArgument, which is a ValueError like the reference's
// std::invalid_argument from its backward (regemm_backward.cu:160-171).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <cctype>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "host/gemm_host.hpp"

namespace py = pybind11;
namespace shim = ::ai::cuda::shim;
using namespace pybind11::literals;

namespace {

void raise_if_not_ok(shim::Status st, const char* where) {
  using S = shim::Status;
  if (st == S::Ok) return;
  const char* msg = "GEMM op failed";
  switch (st) {
    case S::DeviceMismatch: msg = "DeviceMismatch: not a GPU tensor, not row-major 2-D, or dtype mismatch"; break;
    case S::DtypeMismatch: msg = "DtypeMismatch: F32, F16 and BF16 are supported"; break;
    case S::LayoutMismatch: msg = "LayoutMismatch: only row-major is supported"; break;
    case S::TransposeNotSupported: msg = "TransposeNotSupported: only non-transposed path supported"; break;
    case S::ShapeMismatch: msg = "ShapeMismatch: check M,K / K,N / Y(M,N)"; break;
    case S::StrideMismatch: msg = "StrideMismatch: invalid leading dimensions (lda/ldb/ldd)"; break;
    case S::MissingInput: msg = "MissingInput: required input missing (e.g., C for gC)"; break;
    case S::MissingOutput: msg = "MissingOutput: required output missing (e.g., save_z=True but Z_saved is None)"; break;
    case S::Invalid: msg = "Invalid: argument range/validity error (e.g., int32 overflow)"; break;
    case S::InvalidArgument: msg = "InvalidArgument"; break;
    case S::CUDA_ERROR: msg = "HIP error"; break;
    default: msg = "Unknown error";
  }
  std::string full = std::string("[_ops_gemm::") + where + "] " + msg;
  const std::string detail = shim::GemmLastError();
  if (!detail.empty()) full += " (" + detail + ")";
  if (st == S::InvalidArgument) throw std::invalid_argument(full);
  throw std::runtime_error(full);
}

shim::ActKind parse_act(const std::string& s) {
  std::string k(s);
  std::transform(k.begin(), k.end(), k.begin(), [](unsigned char c) { return static_cast<char>(std::tolower(c)); });
  if (k == "none") return shim::ActKind::None;
  if (k == "relu") return shim::ActKind::ReLU;
  if (k == "leakyrelu" || k == "leaky_relu" || k == "lrelu") return shim::ActKind::LeakyReLU;
  if (k == "gelu") return shim::ActKind::GELU;
  if (k == "sigmoid") return shim::ActKind::Sigmoid;
  if (k == "tanh") return shim::ActKind::Tanh;
  throw std::invalid_argument("unknown act: " + s);
}

const shim::Tensor* as_const_tensor_ptr(const py::object& o) {
  return o.is_none() ? nullptr : &o.cast<const shim::Tensor&>();
}
shim::Tensor* as_tensor_ptr(const py::object& o) { return o.is_none() ? nullptr : &o.cast<shim::Tensor&>(); }

// None -> null stream; a PyCapsule holding a hipStream_t (the reference's
// form); an int address is accepted as well.
shim::StreamHandle as_stream(const py::object& o) {
  if (o.is_none()) return nullptr;
  if (PyCapsule_CheckExact(o.ptr())) {
    void* p = PyCapsule_GetPointer(o.ptr(), PyCapsule_GetName(o.ptr()));
    if (!p && PyErr_Occurred()) throw py::error_already_set();
    return p;
  }
  if (py::isinstance<py::int_>(o)) return reinterpret_cast<void*>(o.cast<std::uintptr_t>());
  throw py::type_error("stream must be None, a PyCapsule or an int");
}

shim::Tensor raw2d(std::uintptr_t p, std::int64_t r, std::int64_t c, shim::DType dt) {
  return shim::make_tensor2d(reinterpret_cast<void*>(p), r, c, dt);
}

shim::Tensor raw2d_f32(std::uintptr_t p, std::int64_t r, std::int64_t c) {
  return shim::make_tensor2d(reinterpret_cast<void*>(p), r, c, shim::DType::F32);
}

// gemm_pybind.cpp:190-203: a gBias shaped like a PerM reduction is refused for Dense.
void check_gbias_pern(const shim::Tensor* gBias, std::int64_t M, const char* where, const char* text) {
  if (!gBias || !gBias->data) return;
  const auto& sh = gBias->desc.shape;
  if ((sh.size() == 1 && sh[0] == M) || (sh.size() == 2 && sh[0] == M && sh[1] == 1))
    throw std::invalid_argument(std::string("[_ops_gemm::") + where + "] " + text);
}

const char* kPerMText =
    "gBias shape suggests PerM (len==M). Bias grad for Dense must be PerN; allocate gBias as (1,N) or (N,).";

void forward_attrs(const char* where, const shim::Tensor& A, const shim::Tensor& B, const py::object& bias_obj,
                   shim::Tensor& Y, shim::GemmAttrs attrs, const py::object& z_obj, const py::object& stream_obj,
                   const char* save_z_text) {
  const shim::Tensor* Bias = as_const_tensor_ptr(bias_obj);
  shim::Tensor* Z = as_tensor_ptr(z_obj);
  shim::StreamHandle s = as_stream(stream_obj);
  py::gil_scoped_release release;
  if (Z && Z->data && !attrs.save_z) attrs.save_z = true;
  if (attrs.save_z && (!Z || !Z->data)) throw std::invalid_argument(save_z_text);
  raise_if_not_ok(shim::GemmCudaLaunch(A, B, Bias, Y, attrs, s, Z), where);
}

void backward_attrs(const char* where, const shim::Tensor& A, const shim::Tensor& B, const py::object& C_obj,
                    const shim::Tensor& gY, const shim::Tensor& Z, const py::object& gA_obj,
                    const py::object& gB_obj, const py::object& gC_obj, const py::object& gBias_obj,
                    const shim::GemmAttrs& attrs, const py::object& stream_obj, const char* perm_text,
                    const shim::GemmWorkspace* ws) {
  const shim::Tensor* C = as_const_tensor_ptr(C_obj);
  shim::Tensor* gA = as_tensor_ptr(gA_obj);
  shim::Tensor* gB = as_tensor_ptr(gB_obj);
  shim::Tensor* gC = as_tensor_ptr(gC_obj);
  shim::Tensor* gBias = as_tensor_ptr(gBias_obj);
  shim::StreamHandle s = as_stream(stream_obj);
  py::gil_scoped_release release;
  check_gbias_pern(gBias, A.desc.shape.at(0), where, perm_text);
  raise_if_not_ok(shim::GemmCudaBackward(A, B, C, gY, Z, gA, gB, gC, gBias, attrs, s, ws), where);
}

}  // namespace

PYBIND11_MODULE(_ops_gemm, m) {
  m.attr("__package__") = "graph_executor_v2.ops";
  m.doc() = "GEMM + bias + activation (fused epilogue) on MI355X: F32, F16, BF16; row-major; "
            "bias priority Scalar > PerN(len==N) > PerM(len==M); optional pre-activation stash.";

  py::module_ common = py::module_::import("graph_executor_v2.ops._ops_common");
  for (const char* n : {"ActKind", "GemmAttrs", "Device", "DType", "Layout", "TensorDesc", "Tensor", "make_tensor_2d"})
    m.attr(n) = common.attr(n);

  // ---- shim::Tensor entry points -------------------------------------------------
  m.def(
      "forward",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object bias, shim::Tensor& Y, shim::GemmAttrs attrs,
         py::object Z_saved, py::object stream) {
        forward_attrs("forward", A, B, bias, Y, attrs, Z_saved, stream,
                      "[_ops_gemm::forward] save_z=True requires a valid Z_saved Tensor");
      },
      "A"_a, "B"_a, "bias"_a = py::none(), "Y"_a, "attrs"_a, "Z_saved"_a = py::none(), "stream"_a = py::none(),
      "Run fused GEMM(+bias+activation). Optionally saves pre-activation Z into Z_saved.");

  m.def(
      "backward",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object C, const shim::Tensor& gY, const shim::Tensor& Z,
         py::object gA, py::object gB, py::object gC, py::object gBias, const shim::GemmAttrs& attrs,
         py::object stream) {
        backward_attrs("backward", A, B, C, gY, Z, gA, gB, gC, gBias, attrs, stream, kPerMText, nullptr);
      },
      "A"_a, "B"_a, "C"_a = py::none(), "gY"_a, "Z"_a, "gA"_a = py::none(), "gB"_a = py::none(),
      "gC"_a = py::none(), "gBias"_a = py::none(), "attrs"_a, "stream"_a = py::none(),
      "Compute gradients for fused GEMM(+bias+activation) using pre-activation Z.");

  m.def(
      "forward_ex",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object bias_obj, shim::Tensor& Y, bool trans_a,
         bool trans_b, std::string act, bool with_bias, double leaky_slope, bool save_z, py::object Z_obj,
         py::object stream_obj) {
        const shim::Tensor* Bias = as_const_tensor_ptr(bias_obj);
        shim::Tensor* Z = as_tensor_ptr(Z_obj);
        shim::StreamHandle s = as_stream(stream_obj);
        shim::GemmAttrs attrs{};
        attrs.trans_a = trans_a;
        attrs.trans_b = trans_b;
        attrs.act = parse_act(act);
        attrs.with_bias = with_bias;
        attrs.leaky_slope = static_cast<float>(leaky_slope);
        attrs.save_z = save_z;
        py::gil_scoped_release release;
        if (attrs.with_bias && Bias == nullptr) throw std::invalid_argument("with_bias=True but bias is None");
        if (attrs.save_z) {
          if (!Z || !Z->data) throw std::invalid_argument("save_z=True requires Z_saved Tensor");
        } else if (Z && Z->data) {
          attrs.save_z = true;
        }
        raise_if_not_ok(shim::GemmCudaLaunch(A, B, Bias, Y, attrs, s, Z), "forward_ex");
      },
      "A"_a, "B"_a, "bias"_a = py::none(), "Y"_a, "trans_a"_a = false, "trans_b"_a = false, "act"_a = "none",
      "with_bias"_a = false, "leaky_slope"_a = 0.01, "save_z"_a = false, "Z_saved"_a = py::none(),
      "stream"_a = py::none(), "Fused GEMM with epilogue parameters given as Python primitives.");

  m.def(
      "backward_ex",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object C, const shim::Tensor& gY, const shim::Tensor& Z,
         py::object gA, py::object gB, py::object gC, py::object gBias, bool trans_a, bool trans_b, std::string act,
         bool with_bias, double leaky_slope, py::object stream) {
        shim::GemmAttrs attrs{};
        attrs.trans_a = trans_a;
        attrs.trans_b = trans_b;
        attrs.act = parse_act(act);
        attrs.with_bias = with_bias;
        attrs.leaky_slope = static_cast<float>(leaky_slope);
        backward_attrs("backward_ex", A, B, C, gY, Z, gA, gB, gC, gBias, attrs, stream, kPerMText, nullptr);
      },
      "A"_a, "B"_a, "C"_a = py::none(), "gY"_a, "Z"_a, "gA"_a = py::none(), "gB"_a = py::none(),
      "gC"_a = py::none(), "gBias"_a = py::none(), "trans_a"_a = false, "trans_b"_a = false, "act"_a = "none",
      "with_bias"_a = false, "leaky_slope"_a = 0.01, "stream"_a = py::none(),
      "Backward for fused GEMM with epilogue parameters given as Python primitives.");

  m.def(
      "backward_into",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object C, const shim::Tensor& gY, const shim::Tensor& Z,
         py::object gA, py::object gB, py::object gC, py::object gBias, const shim::GemmAttrs& attrs,
         py::object stream, std::uintptr_t dZ_ptr, std::uintptr_t lt_ws_ptr, std::size_t lt_ws_bytes) {
        if (!dZ_ptr)
          throw std::invalid_argument("[_ops_gemm::backward_into] dZ_ptr is required for capture-safe path");
        if ((lt_ws_ptr == 0) != (lt_ws_bytes == 0))
          throw std::invalid_argument(
              "[_ops_gemm::backward_into] lt_workspace ptr/bytes must be both zero or both non-zero");
        shim::GemmWorkspace ws{};
        ws.scratch = reinterpret_cast<void*>(dZ_ptr);
        ws.scratch_bytes = shim::GemmRequiredBackwardScratchBytes(A.desc.shape.at(0), B.desc.shape.at(1));
        ws.lt_workspace = reinterpret_cast<void*>(lt_ws_ptr);
        ws.lt_workspace_bytes = lt_ws_bytes;
        backward_attrs("backward_into", A, B, C, gY, Z, gA, gB, gC, gBias, attrs, stream,
                       "gBias must be PerN (shape (1,N) or (N,))", &ws);
      },
      "A"_a, "B"_a, "C"_a = py::none(), "gY"_a, "Z"_a, "gA"_a = py::none(), "gB"_a = py::none(),
      "gC"_a = py::none(), "gBias"_a = py::none(), "attrs"_a, "stream"_a = py::none(), "dZ_ptr"_a,
      "lt_ws_ptr"_a = static_cast<std::uintptr_t>(0), "lt_ws_bytes"_a = static_cast<std::size_t>(0),
      "Capture-safe backward: the dZ buffer (M*N fp32) is the dY' workspace whenever one is needed, so nothing "
      "is allocated.");

  m.def(
      "forward_ex_attrs",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object bias, shim::Tensor& Y, shim::GemmAttrs attrs,
         py::object Z_saved, py::object stream) {
        forward_attrs("forward_ex_attrs", A, B, bias, Y, attrs, Z_saved, stream,
                      "[_ops_gemm::forward_ex_attrs] save_z=True requires Z_saved");
      },
      "A"_a, "B"_a, "bias"_a = py::none(), "Y"_a, "attrs"_a, "Z_saved"_a = py::none(), "stream"_a = py::none(),
      "Alias of `forward`.");

  m.def(
      "backward_ex_attrs",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object C, const shim::Tensor& gY, const shim::Tensor& Z,
         py::object gA, py::object gB, py::object gC, py::object gBias, const shim::GemmAttrs& attrs,
         py::object stream) {
        backward_attrs("backward_ex_attrs", A, B, C, gY, Z, gA, gB, gC, gBias, attrs, stream,
                       "gBias must be PerN (1,N) or (N,)", nullptr);
      },
      "A"_a, "B"_a, "C"_a = py::none(), "gY"_a, "Z"_a, "gA"_a = py::none(), "gB"_a = py::none(),
      "gC"_a = py::none(), "gBias"_a = py::none(), "attrs"_a, "stream"_a = py::none(), "Alias of `backward`.");

  // ---- raw-pointer entry points ----------------------------------------------------
  m.def(
      "forward_raw",
      [](std::uintptr_t A_ptr, std::uintptr_t B_ptr, std::uintptr_t Bias_ptr, std::uintptr_t Y_ptr, std::int64_t M,
         std::int64_t K, std::int64_t N, bool trans_a, bool trans_b, std::string act, bool with_bias,
         double leaky_slope, bool save_z, std::uintptr_t Z_ptr, py::object stream_obj, shim::DType dtype) {
        shim::StreamHandle s = as_stream(stream_obj);
        shim::GemmAttrs attrs{};
        attrs.trans_a = trans_a;
        attrs.trans_b = trans_b;
        attrs.act = parse_act(act);
        attrs.with_bias = with_bias;
        attrs.leaky_slope = static_cast<float>(leaky_slope);
        attrs.save_z = save_z;
        py::gil_scoped_release release;
        shim::Tensor A = raw2d(A_ptr, M, K, dtype), B = raw2d(B_ptr, K, N, dtype), Y = raw2d(Y_ptr, M, N, dtype);
        shim::Tensor bias_t{}, z_t{};
        shim::Tensor* Bias = nullptr;
        shim::Tensor* Z = nullptr;
        if (with_bias) {
          if (!Bias_ptr) throw std::invalid_argument("[_ops_gemm::forward_raw] with_bias=True but Bias_ptr==0");
          bias_t = raw2d_f32(Bias_ptr, 1, N);
          Bias = &bias_t;
        }
        if (save_z) {
          if (!Z_ptr) throw std::invalid_argument("[_ops_gemm::forward_raw] save_z=True but Z_ptr==0");
          z_t = raw2d(Z_ptr, M, N, dtype);
          Z = &z_t;
        }
        raise_if_not_ok(shim::GemmCudaLaunch(A, B, Bias, Y, attrs, s, Z), "forward_raw");
      },
      "A_ptr"_a, "B_ptr"_a, "Bias_ptr"_a, "Y_ptr"_a, "M"_a, "K"_a, "N"_a, "trans_a"_a = false, "trans_b"_a = false,
      "act"_a = "none", "with_bias"_a = false, "leaky_slope"_a = 0.01, "save_z"_a = false,
      "Z_ptr"_a = static_cast<std::uintptr_t>(0), "stream"_a = py::none(), "dtype"_a = shim::DType::F32,
      "Raw-pointer fused GEMM(+bias+activation), row-major; bias is (1,N) F32.");

  m.def(
      "backward_raw",
      [](std::uintptr_t A_ptr, std::uintptr_t B_ptr, std::uintptr_t C_ptr, std::uintptr_t gY_ptr,
         std::uintptr_t Z_ptr, std::uintptr_t gA_ptr, std::uintptr_t gB_ptr, std::uintptr_t gC_ptr,
         std::uintptr_t gBias_ptr, std::int64_t M, std::int64_t K, std::int64_t N, bool trans_a, bool trans_b,
         std::string act, bool with_bias, double leaky_slope, py::object stream_obj, shim::DType dtype) {
        shim::StreamHandle s = as_stream(stream_obj);
        shim::GemmAttrs attrs{};
        attrs.trans_a = trans_a;
        attrs.trans_b = trans_b;
        attrs.act = parse_act(act);
        attrs.with_bias = with_bias;
        attrs.leaky_slope = static_cast<float>(leaky_slope);
        py::gil_scoped_release release;
        shim::Tensor A = raw2d(A_ptr, M, K, dtype), B = raw2d(B_ptr, K, N, dtype);
        shim::Tensor gY = raw2d(gY_ptr, M, N, dtype), Z = raw2d(Z_ptr, M, N, dtype);
        shim::Tensor c_t = raw2d(C_ptr, M, N, dtype), ga_t = raw2d(gA_ptr, M, K, dtype);
        shim::Tensor gb_t = raw2d(gB_ptr, K, N, dtype), gc_t = raw2d(gC_ptr, M, N, dtype);
        shim::Tensor gbias_t = raw2d_f32(gBias_ptr, 1, N);
        raise_if_not_ok(shim::GemmCudaBackward(A, B, C_ptr ? &c_t : nullptr, gY, Z, gA_ptr ? &ga_t : nullptr,
                                               gB_ptr ? &gb_t : nullptr, gC_ptr ? &gc_t : nullptr,
                                               gBias_ptr ? &gbias_t : nullptr, attrs, s),
                        "backward_raw");
      },
      "A_ptr"_a, "B_ptr"_a, "C_ptr"_a = static_cast<std::uintptr_t>(0), "gY_ptr"_a, "Z_ptr"_a,
      "gA_ptr"_a = static_cast<std::uintptr_t>(0), "gB_ptr"_a = static_cast<std::uintptr_t>(0),
      "gC_ptr"_a = static_cast<std::uintptr_t>(0), "gBias_ptr"_a = static_cast<std::uintptr_t>(0), "M"_a, "K"_a,
      "N"_a, "trans_a"_a = false, "trans_b"_a = false, "act"_a = "none", "with_bias"_a = false,
      "leaky_slope"_a = 0.01, "stream"_a = py::none(), "dtype"_a = shim::DType::F32,
      "Raw-pointer backward for fused GEMM(+bias+activation); gBias is (1,N) F32.");

  // ---- batched / strided (new) -----------------------------------------------------
  m.def(
      "forward_batched",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object bias_obj, shim::Tensor& Y,
         shim::GemmAttrs attrs, std::int64_t batch, std::int64_t stride_a, std::int64_t stride_b,
         std::int64_t stride_y, std::int64_t stride_bias, py::object Z_obj, std::int64_t stride_z,
         py::object stream_obj) {
        const shim::Tensor* Bias = as_const_tensor_ptr(bias_obj);
        shim::Tensor* Z = as_tensor_ptr(Z_obj);
        shim::StreamHandle s = as_stream(stream_obj);
        py::gil_scoped_release release;
        if (Z && Z->data) attrs.save_z = true;
        if (attrs.save_z && (!Z || !Z->data))
          throw std::invalid_argument("[_ops_gemm::forward_batched] save_z=True requires Z_saved");
        shim::GemmBatch bt{batch, stride_a, stride_b, stride_bias, stride_y, stride_z};
        raise_if_not_ok(shim::GemmBatchedLaunch(A, B, Bias, Y, attrs, bt, s, Z), "forward_batched");
      },
      "A"_a, "B"_a, "bias"_a = py::none(), "Y"_a, "attrs"_a, "batch"_a, "stride_a"_a, "stride_b"_a, "stride_y"_a,
      "stride_bias"_a = 0, "Z_saved"_a = py::none(), "stride_z"_a = 0, "stream"_a = py::none(),
      "One launch over `batch` slices: Y_b = act(alpha*op(A_b) op(B_b) + bias_b). Tensors describe one "
      "slice; slice b starts b*stride_* elements after the data pointer. attrs.trans_a/trans_b/alpha apply.");

  m.def(
      "backward_batched",
      [](const shim::Tensor& A, const shim::Tensor& B, py::object C_obj, const shim::Tensor& gY,
         const shim::Tensor& Z, py::object gA_obj, py::object gB_obj, py::object gC_obj, py::object gBias_obj,
         const shim::GemmAttrs& attrs, std::int64_t batch, std::int64_t stride_a, std::int64_t stride_b,
         std::int64_t stride_gy, std::int64_t stride_z, std::int64_t stride_ga, std::int64_t stride_gb,
         std::int64_t stride_gc, std::int64_t stride_gbias, py::object stream_obj) {
        const shim::Tensor* C = as_const_tensor_ptr(C_obj);
        shim::Tensor* gA = as_tensor_ptr(gA_obj);
        shim::Tensor* gB = as_tensor_ptr(gB_obj);
        shim::Tensor* gC = as_tensor_ptr(gC_obj);
        shim::Tensor* gBias = as_tensor_ptr(gBias_obj);
        shim::StreamHandle s = as_stream(stream_obj);
        py::gil_scoped_release release;
        shim::GemmBatchBwd bt{batch, stride_a, stride_b, stride_gy, stride_z, stride_ga, stride_gb, stride_gc,
                              stride_gbias};
        raise_if_not_ok(shim::GemmBatchedBackward(A, B, C, gY, Z, gA, gB, gC, gBias, attrs, bt, s),
                        "backward_batched");
      },
      "A"_a, "B"_a, "C"_a = py::none(), "gY"_a, "Z"_a, "gA"_a = py::none(), "gB"_a = py::none(),
      "gC"_a = py::none(), "gBias"_a = py::none(), "attrs"_a, "batch"_a, "stride_a"_a, "stride_b"_a,
      "stride_gy"_a, "stride_z"_a, "stride_ga"_a = 0, "stride_gb"_a = 0, "stride_gc"_a = 0, "stride_gbias"_a = 0,
      "stream"_a = py::none(), "Backward of forward_batched (no transposes), one launch per gradient.");

  m.attr("__all__") = py::make_tuple("ActKind", "GemmAttrs", "Device", "DType", "Layout", "TensorDesc", "Tensor",
                                     "make_tensor_2d", "forward", "backward", "forward_ex", "backward_ex",
                                     "backward_into", "forward_ex_attrs", "backward_ex_attrs", "forward_raw",
                                     "backward_raw", "forward_batched", "backward_batched");
}
