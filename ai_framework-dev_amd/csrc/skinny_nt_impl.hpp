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

template <typename T, int MAXM = 16, int P = 2>
__device__ __forceinline__ void skinny_nt_column(const SkinnyNtArgs& p, int k, int lane, float* sum) {
  constexpr int EPC = Elem<T>::kPerChunk;
  const T* G = reinterpret_cast<const T*>(p.G);
  const T* Z = reinterpret_cast<const T*>(p.Z);
  const T* brow = reinterpret_cast<const T*>(p.B) + (int64_t)k * p.ldb;
  float acc[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; ++m) acc[m] = 0.f;
  // P passes of 64 chunks at a time, so that all their loads are in flight
  // together; a pass past N reloads the first and adds nothing.  A lane adds
  // its chunks in increasing n whatever P is.
  for (int n0 = lane * EPC; n0 < p.N; n0 += P * 64 * EPC) {
    int nn[P];
    bool ok[P];
#pragma unroll
    for (int h = 0; h < P; ++h) {
      const int nh = n0 + h * 64 * EPC;
      ok[h] = nh < p.N;
      nn[h] = ok[h] ? nh : n0;
    }
    u32x4 braw[P], graw[P][MAXM];
#pragma unroll
    for (int h = 0; h < P; ++h) braw[h] = *reinterpret_cast<const u32x4*>(brow + nn[h]);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m >= p.M) continue;
#pragma unroll
      for (int h = 0; h < P; ++h) graw[h][m] = *reinterpret_cast<const u32x4*>(G + (int64_t)m * p.ldg + nn[h]);
    }
#pragma unroll
    for (int h = 0; h < P; ++h) {
      if (!ok[h]) break;
      const int n = nn[h];
      float bv[EPC];
      chunk_to_f32<T>(braw[h], bv);
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
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
  for (int m = 0; m < MAXM; ++m) {
    if (m >= p.M) continue;
    float v = acc[m];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    sum[m] = v;
  }
}

// Rows and passes for a problem: up to 8 rows keep four passes of fp32
// chunks in flight (graw: 4 x 8 chunks), 16 rows two.
template <typename T>
constexpr int skinny_nt_passes(int maxm) { return (maxm == 8 && sizeof(T) == 4) ? 4 : 2; }

}  // namespace gev2
