// Instantiations of the MFMA tile GEMM for one element type (float); split per
// type so the three compile in parallel.
#include "gemm_tile_impl.hpp"

namespace gev2 {
hipError_t launch_tile_f32(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                          int batch, hipStream_t s) {
  return launch_cfg<float>(cfg, ta, tb, pro, vec, a, batch, s);
}
}  // namespace gev2
