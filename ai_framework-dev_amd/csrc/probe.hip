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

}  // namespace gev2

extern "C" int gev2_probe_mfma_bf16(int random_operands, int iters, void* stream) {
  if (iters < 1) return GEV2_INVALID_ARGUMENT;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return GEV2_HIP_ERROR;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return GEV2_HIP_ERROR;
  hipLaunchKernelGGL(gev2::probe_mfma_kernel, dim3(cus), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     random_operands, iters);
  return hipGetLastError() == hipSuccess ? GEV2_OK : GEV2_HIP_ERROR;
}
