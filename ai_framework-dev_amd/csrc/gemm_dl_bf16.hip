// Instantiations of the direct-to-LDS MFMA tile GEMM for one element type
// (__bf16); split per type so the three compile in parallel.
#include "gemm_dl_impl.hpp"

namespace gev2 {
hipError_t launch_dl_bf16(int cfg, bool ta, bool tb, const TileArgs& a, int batch, hipStream_t s) {
  return launch_dl_cfg<__bf16>(cfg, ta, tb, a, batch, s);
}
}  // namespace gev2
