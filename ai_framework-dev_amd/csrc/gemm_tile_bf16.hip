// Instantiations of the MFMA tile GEMM for one element type (__bf16); split per
// type so the three compile in parallel.
#include "gemm_tile_impl.hpp"

namespace gev2 {
hipError_t launch_tile_bf16(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                          int batch, hipStream_t s) {
  return launch_cfg<__bf16>(cfg, ta, tb, pro, vec, a, batch, s);
}
}  // namespace gev2
