// Host-side operator types of the GEMM + bias + activation op.
//
// These are the types the reference's C++ callers and Python binding pass
// around (graph_executor_v2/backends/cuda/ops/_common/shim/): a non-owning 2-D
// tensor view, the enums with their ABI values, the GEMM attributes, the
// workspace descriptor and the Status codes.  Names, field names and enum
// values are kept identical because they are the drop-in interface: the
// conv2d / rnn launchers and the pybind modules are written against them.
//   Device/DType/Layout      ai_device.hpp:14-27
//   ActKind/BiasKind         enums.hpp:10-24
//   Status                   ai_status.hpp:14-43
//   TensorDesc/Tensor        ai_tensor.hpp:13-63, make_tensor2d ai_tensor.hpp:93-100
//   GemmAttrs                ai_ops_base.hpp:9-18
//   GemmWorkspace            gemm/api.hpp:97-104
// "CUDA" in Device::CUDA means "the GPU" (here: the MI355X through HIP).
// Nothing in this header includes a GPU runtime header.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace ai::cuda::shim {

enum class Device : int { CPU = 0, CUDA = 1 };
enum class DType : int { F32 = 0, F16 = 1, BF16 = 2, I32 = 3, I8 = 4 };
enum class Layout : int { RowMajor = 0, ColMajor = 1 };
enum class ActKind : int { None = 0, ReLU = 1, LeakyReLU = 2, GELU = 3, Sigmoid = 4, Tanh = 5 };
enum class BiasKind : int { None = 0, Scalar = 1, PerM = 2, PerN = 3 };

enum class Status : int {
  Ok = 0,
  Invalid = 1,
  Unimplemented = 2,
  RuntimeError = 3,
  InvalidArgument = 4,
  MissingInput = 10,
  MissingOutput = 11,
  DeviceMismatch = 100,
  DtypeMismatch = 101,
  LayoutMismatch = 102,
  ShapeMismatch = 103,
  StrideMismatch = 104,
  TransposeNotSupported = 105,
  CUDA_ERROR = 130,   // HIP runtime / launch failures
  Unknown = 999
};

static_assert(static_cast<int>(Device::CUDA) == 1 && static_cast<int>(DType::BF16) == 2 &&
                  static_cast<int>(ActKind::Tanh) == 5 && static_cast<int>(BiasKind::PerN) == 3 &&
                  static_cast<int>(Status::CUDA_ERROR) == 130,
              "operator enum values are ABI anchors");

// hipStream_t (or nullptr for the null stream), carried as an opaque pointer.
using StreamHandle = void*;

inline std::size_t dtype_size(DType dt) {
  switch (dt) {
    case DType::F32: case DType::I32: return 4;
    case DType::F16: case DType::BF16: return 2;
    case DType::I8: return 1;
  }
  return 0;
}

struct TensorDesc {
  DType dtype{DType::F32};
  Layout layout{Layout::RowMajor};
  std::vector<std::int64_t> shape;    // dims
  std::vector<std::int64_t> stride;   // element strides
  std::int64_t dim(int i) const { return shape.at(static_cast<std::size_t>(i)); }
};

struct Tensor {
  void* data{nullptr};
  TensorDesc desc{};
  Device device{Device::CUDA};
  int device_index{0};

  bool is_cuda() const { return device == Device::CUDA; }
  bool is_defined() const { return data != nullptr; }
  bool is_contiguous_rowmajor_2d() const {
    if (desc.layout != Layout::RowMajor || desc.shape.size() != 2 || desc.stride.size() != 2)
      return false;
    if (desc.shape[0] < 0 || desc.shape[1] < 0) return false;
    return desc.stride[1] == 1 && desc.stride[0] == desc.shape[1];
  }
};

// 2-D row-major view with dense strides {cols, 1} on the GPU, device 0.
inline Tensor make_tensor2d(void* ptr, std::int64_t rows, std::int64_t cols,
                            DType dt = DType::F32) {
  Tensor t;
  t.data = ptr;
  t.device = Device::CUDA;
  t.device_index = 0;
  t.desc.dtype = dt;
  t.desc.layout = Layout::RowMajor;
  t.desc.shape = {rows, cols};
  t.desc.stride = {cols, 1};
  return t;
}

struct GemmAttrs {
  bool trans_a{false};
  bool trans_b{false};
  ActKind act{ActKind::None};
  bool with_bias{false};
  float leaky_slope{0.01f};
  bool save_z{false};
  float alpha{1.0f};   // honoured by the batched launcher only (the 2-D launcher uses 1)
  float beta{0.0f};    // unused, as in the reference
};

// Workspaces of a call (gemm/api.hpp:97-104), validated like the reference's
// (alignment of lt_workspace, size of scratch).  `scratch` is the operator's
// workspace: the backward's dY' (M*N elements suffice) and, in the forward,
// the split-K partials of skinny 16-bit problems; lt_workspace is unused.
struct alignas(256) GemmWorkspace {
  void* lt_workspace = nullptr;
  std::size_t lt_workspace_bytes = 0;
  void* scratch = nullptr;
  std::size_t scratch_bytes = 0;
};

constexpr std::size_t GemmRequiredBackwardScratchBytes(std::int64_t M, std::int64_t N) noexcept {
  return (M <= 0 || N <= 0) ? 0u : static_cast<std::size_t>(M) * static_cast<std::size_t>(N) * 4u;
}

}  // namespace ai::cuda::shim
