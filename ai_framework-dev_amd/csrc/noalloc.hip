// The forward entry point that allocates nothing: gev2_gemm_fwd_noalloc.
//
// gev2_gemm_fwd takes the split-K partial sums of skinny 16-bit problems from
// the caller's workspace or, failing that, from a buffer the library
// allocates per stream.  Callers that may not allocate at all (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc) use
// this variant instead: the partials go to `scratch`, a fixed device array of
// kNoAllocScratchBytes that every GPU holds from module load until the
// process ends.  Everything else (validation, kernel choice, the kernels) is
// gev2_gemm_fwd's.
//
// The array's host-side name is only a stand-in for the symbol: its device
// address is looked up once per device with hipGetSymbolAddress (with that
// device current) and only that address is ever handed to a kernel.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/gev2_gemm.h"
#include "gev2_kernels.hpp"

namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[gev2::kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's copy of `scratch` (looked up on first use).
hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

extern "C" {

int gev2_gemm_fwd_noalloc(const gev2_gemm_fwd_desc* desc, void* stream) {
  void* ptr = nullptr;
  const hipError_t e = scratch_address(&ptr);
  if (e != hipSuccess) return gev2::report_hip_error(e, "hipGetSymbolAddress(scratch)");
  return gev2::gemm_fwd_run(desc, stream, ptr, gev2::kNoAllocScratchBytes);
}

}  // extern "C"
