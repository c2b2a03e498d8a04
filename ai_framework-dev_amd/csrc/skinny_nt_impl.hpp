// The dot-product core of the skinny NT product (M <= 16):
//   sum[m] = sum_n G[m][n] * (Z ? act'(Z[m][n]) : 1) * B[k][n]
// for one output column k, computed by one wave: the wave reads row k of B
// once in 16-byte chunks (lanes stride over n, two passes' loads in flight at
// once), keeps M partial sums per lane and adds them across the wave in a
// fixed butterfly order, so that every lane returns all M sums.  Shared by
// skinny_nt_kernel and the RNN's fused backward step.
#pragma once

#include "gev2_device.hpp"
#include "gev2_kernels.hpp"

namespace gev2 {

template <typename T>
__device__ __forceinline__ void skinny_nt_column(const SkinnyNtArgs& p, int k, int lane, float* sum) {
  constexpr int EPC = Elem<T>::kPerChunk;
  const T* G = reinterpret_cast<const T*>(p.G);
  const T* Z = reinterpret_cast<const T*>(p.Z);
  const T* brow = reinterpret_cast<const T*>(p.B) + (int64_t)k * p.ldb;
  float acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0.f;
  // two passes of 64 chunks at a time, so that both passes' loads are in
  // flight together; a second pass past N reloads the first and adds nothing
  for (int n0 = lane * EPC; n0 < p.N; n0 += 128 * EPC) {
    const int n1 = n0 + 64 * EPC;
    const bool two = n1 < p.N;
    const int nb = two ? n1 : n0;
    u32x4 braw[2], graw[2][16];
    braw[0] = *reinterpret_cast<const u32x4*>(brow + n0);
    braw[1] = *reinterpret_cast<const u32x4*>(brow + nb);
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if (m >= p.M) continue;
      graw[0][m] = *reinterpret_cast<const u32x4*>(G + (int64_t)m * p.ldg + n0);
      graw[1][m] = *reinterpret_cast<const u32x4*>(G + (int64_t)m * p.ldg + nb);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1 && !two) break;
      const int n = h == 0 ? n0 : nb;
      float bv[EPC];
      chunk_to_f32<T>(braw[h], bv);
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        if (m >= p.M) continue;
        float gv[EPC];
        chunk_to_f32<T>(graw[h][m], gv);
        if (Z) {
          float zv[EPC];
          chunk_to_f32<T>(*reinterpret_cast<const u32x4*>(Z + (int64_t)m * p.ldz + n), zv);
#pragma unroll
          for (int e = 0; e < EPC; ++e) gv[e] *= act_grad(zv[e], p.act, p.slope);
        }
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[m] = fmaf(gv[e], bv[e], acc[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    if (m >= p.M) continue;
    float v = acc[m];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    sum[m] = v;
  }
}

}  // namespace gev2
