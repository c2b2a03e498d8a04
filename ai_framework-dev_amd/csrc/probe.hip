// Measurement helper (no counterpart in the reference): the sustained rate of
// back-to-back v_mfma_f32_32x32x16_bf16 with one wave on every SIMD and
// operands that are either zero or random bf16 values.  The benchmark reports
// it beside the GEMM's roofline fraction: with random data the part runs its
// matrix cores at a lower clock than with zeros, so the published dense peak
// is not reachable by any kernel on such inputs.
#include <hip/hip_runtime.h>

#include "../../include/gev2_gemm.h"
#include "gev2_device.hpp"

namespace gev2 {

// externally visible, so the compiler cannot drop the stores (and with them
// the MFMAs that feed them)
__device__ float gev2_probe_sink[1];

__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
  return x;
}

// two bf16 values with random sign and mantissa, exponent in [120, 127]
__device__ __forceinline__ uint32_t probe_bf16x2(uint32_t h) {
  const uint32_t g = probe_hash(h);
  const uint32_t lo = (h & 0x807fu) | ((120u + ((h >> 7) & 7u)) << 7);
  const uint32_t hi = (g & 0x807fu) | ((120u + ((g >> 7) & 7u)) << 7);
  return (lo & 0xffffu) | (hi << 16);
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
probe_mfma_kernel(int random_operands, int iters) {
  f32x16_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  u32x4 ua = {0u, 0u, 0u, 0u}, ub = {0u, 0u, 0u, 0u};
  if (random_operands) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ua[i] = probe_bf16x2(probe_hash(t * 8 + i));
      ub[i] = probe_bf16x2(probe_hash(t * 8 + 4 + i));
    }
  }
  const bf16x8_t a = __builtin_bit_cast(bf16x8_t, ua), b = __builtin_bit_cast(bf16x8_t, ub);
  const bf16x8_t a2 = __builtin_bit_cast(bf16x8_t, ub), b2 = __builtin_bit_cast(bf16x8_t, ua);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16((i & 1) ? a2 : a, (i & 2) ? b2 : b, acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += acc[i][0] + acc[i][15];
  if (s == 1234.5f) gev2_probe_sink[0] = s;   // keeps the MFMAs live; never true in practice
}

// Streaming read: workgroup w reads chunks w, w + grid, ... of
// 256 threads x U x 16 bytes, every thread with its U 16-byte loads in flight
// at once, and folds them into one word.
template <int U>
__global__ void __launch_bounds__(256) probe_read_kernel(const u32x4* __restrict__ src, int64_t chunks) {
  uint32_t x = 0u;
  for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const u32x4* p = src + c * (256 * U) + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + u * 256);
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (x == 0x9e3779b9u) gev2_probe_sink[0] = static_cast<float>(x);   // keeps the loads live
}

// Streaming write: workgroup w writes chunks w, w + grid, ... of
// 256 threads x U x 16 bytes with 16-byte vector stores.
template <int U>
__global__ void __launch_bounds__(256) probe_write_kernel(u32x4* __restrict__ dst, int64_t chunks) {
  for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    u32x4* p = dst + c * (256 * U) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < U; ++u) p[u * 256] = u32x4{static_cast<uint32_t>(c), static_cast<uint32_t>(u), 0u, 0u};
  }
}

}  // namespace gev2

extern "C" int gev2_probe_hbm_write(void* buf, size_t bytes, int sets, int reps, int workgroups, int unroll,
                                    void* stream) {
  const size_t chunk = static_cast<size_t>(256) * 16 * static_cast<size_t>(unroll);
  if (!buf || sets < 1 || reps < 1 || workgroups < 1) return GEV2_INVALID_ARGUMENT;
  if (unroll != 8 && unroll != 16) return GEV2_INVALID_ARGUMENT;
  if (bytes == 0 || bytes % chunk != 0 || (reinterpret_cast<uintptr_t>(buf) & 15u) != 0) return GEV2_INVALID_ARGUMENT;
  const int64_t chunks = static_cast<int64_t>(bytes / chunk);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int r = 0; r < reps; ++r) {
    auto* dst = reinterpret_cast<gev2::u32x4*>(static_cast<char*>(buf) + (r % sets) * bytes);
    if (unroll == 8)
      hipLaunchKernelGGL(gev2::probe_write_kernel<8>, dim3(workgroups), dim3(256), 0, s, dst, chunks);
    else
      hipLaunchKernelGGL(gev2::probe_write_kernel<16>, dim3(workgroups), dim3(256), 0, s, dst, chunks);
    if (hipGetLastError() != hipSuccess) return GEV2_HIP_ERROR;
  }
  return GEV2_OK;
}

extern "C" int gev2_probe_hbm_read(const void* buf, size_t bytes, int sets, int reps, int workgroups, int unroll,
                                   void* stream) {
  const size_t chunk = static_cast<size_t>(256) * 16 * static_cast<size_t>(unroll);
  if (!buf || sets < 1 || reps < 1 || workgroups < 1) return GEV2_INVALID_ARGUMENT;
  if (unroll != 8 && unroll != 16 && unroll != 32) return GEV2_INVALID_ARGUMENT;
  if (bytes == 0 || bytes % chunk != 0 || (reinterpret_cast<uintptr_t>(buf) & 15u) != 0) return GEV2_INVALID_ARGUMENT;
  const int64_t chunks = static_cast<int64_t>(bytes / chunk);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int r = 0; r < reps; ++r) {
    const auto* src = reinterpret_cast<const gev2::u32x4*>(static_cast<const char*>(buf) + (r % sets) * bytes);
    if (unroll == 8)
      hipLaunchKernelGGL(gev2::probe_read_kernel<8>, dim3(workgroups), dim3(256), 0, s, src, chunks);
    else if (unroll == 16)
      hipLaunchKernelGGL(gev2::probe_read_kernel<16>, dim3(workgroups), dim3(256), 0, s, src, chunks);
    else
      hipLaunchKernelGGL(gev2::probe_read_kernel<32>, dim3(workgroups), dim3(256), 0, s, src, chunks);
    if (hipGetLastError() != hipSuccess) return GEV2_HIP_ERROR;
  }
  return GEV2_OK;
}

extern "C" int gev2_probe_mfma_bf16(int random_operands, int iters, void* stream) {
  if (iters < 1) return GEV2_INVALID_ARGUMENT;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return GEV2_HIP_ERROR;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return GEV2_HIP_ERROR;
  hipLaunchKernelGGL(gev2::probe_mfma_kernel, dim3(cus), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     random_operands, iters);
  return hipGetLastError() == hipSuccess ? GEV2_OK : GEV2_HIP_ERROR;
}
