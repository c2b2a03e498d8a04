// Small fp32 problems in one launch.
//
// A GEMM whose output covers only a few CUs' worth of tiles (the MLP layer
// X[64,784] . W[784,256] is 64 tiles of 16x16) is bound by the latency of its
// launches and memory round trips, not by the matrix cores.  The reference
// runs such a layer through the same tile kernel as a large one
// (regemm_epilogue.cu; the backward's dY' pass and two GEMMs,
// regemm_backward.cu:151-301, launcher.cu:279-383).  Here one launch does the
// whole forward (GEMM, bias, activation, Z) and one the whole backward (dX, dW
// and the PerN dBias, with dY' = dY (.) act'(Z) formed as the operands are
// loaded):
//
//   - a workgroup owns one 16x16 output tile; its W waves take interleaved
//     blocks of 16 along the reduction (wave w: blocks w, w + W, ...), load
//     their operands straight into registers (4 blocks in flight per wave,
//     16-byte loads where the operand is contiguous along the reduction) and
//     accumulate with v_mfma_f32_16x16x4f32;
//   - the W partial tiles meet in LDS and are added in wave order, then the
//     epilogue writes the tile; a backward job with a reduction of at most 64
//     (the dW of a 64-row batch, a rank-8 dW) instead gives each wave a
//     tile of its own;
//   - in the backward, workgroups past the dX and dW tiles each sum 64
//     columns of dY' over the rows, split over their waves (PerN dBias).
//
// Every sum has a fixed order, so results repeat bit for bit.
#include "gev2_device.hpp"
#include "gev2_kernels.hpp"

namespace gev2 {

// elements (i, k0 .. k0 + 3) of an operand, zero past the reduction length,
// times act'(Z) when it is dY' (HASZ).  VEC operands (k contiguous, rows and
// base 16-byte aligned) take one 16-byte load per array when all four are in
// range.
template <bool VEC, bool HASZ, int ACT, bool TWO = false>
__device__ __forceinline__ f32x4_t small_load4(const SmallOperand& o, int i, int k0, int red, float slope) {
  f32x4_t v;
  // TWO: the part holding k0 .. k0+3 (k0 and k1 are multiples of 4, so the
  // four never straddle k1); element k of it is pb[ob + k * ks]
  const bool second = TWO && k0 >= o.k1;
  const float* pb = second ? o.p2 : o.p;
  const int64_t ob = second ? (int64_t)i * o.rs2 - (int64_t)o.k1 * o.ks : (int64_t)i * o.rs;
  if constexpr (VEC) {
    if (k0 + 3 < red) {
      v = *reinterpret_cast<const f32x4_t*>(pb + (ob + k0));
      if constexpr (HASZ) {
        const f32x4_t z = *reinterpret_cast<const f32x4_t*>(o.z + (int64_t)i * o.zrs + k0);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= act_grad_t<ACT>(z[e], slope);
      }
      return v;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int k = k0 + e;
    float x = 0.f;
    if (k < red) {
      x = pb[ob + (int64_t)k * o.ks];
      if constexpr (HASZ) x *= act_grad_t<ACT>(o.z[(int64_t)i * o.zrs + (int64_t)k * o.zks], slope);
    }
    v[e] = x;
  }
  return v;
}

// One 16x16 output tile t of job J; red: W x 256 floats of LDS.
template <int W, bool AV, bool BV, bool AZ, bool BZ, int ACT, bool FWD, bool TWO = false>
__device__ __forceinline__ void small_tile(const SmallArgs& p, const SmallJob& J, int t, float* red) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tr = t / J.tiles_c, tc = t - tr * J.tiles_c;
  // MFMA operand lanes: A row / B column lane % 16.  Reduction blocks of 16:
  // lane quarter q = lane / 16 holds k = 16 j + 4 q + e (e < 4) of block j, and
  // MFMA e of the block sums those four k (one per quarter).
  const int r = tr * 16 + (lane & 15), c = tc * 16 + (lane & 15), kq = lane >> 4;
  const bool rin = r < J.rows, cin = c < J.cols;
  const int blocks = (J.red + 15) >> 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = wave; j0 < blocks; j0 += 4 * W) {
    f32x4_t av[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k0 = 16 * (j0 + u * W) + 4 * kq;
      av[u] = rin ? small_load4<AV, AZ, ACT, TWO>(J.a, r, k0, J.red, p.slope) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      bv[u] = cin ? small_load4<BV, BZ, ACT>(J.b, c, k0, J.red, p.slope) : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][e], bv[u][e], acc, 0, 0, 0);
  }
  // D[4 (lane / 16) + v][lane % 16] = acc[v]
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave * 256 + v * 64 + lane] = acc[v];
  __syncthreads();
  if (tid < 256) {
    float s = red[tid];
#pragma unroll
    for (int w = 1; w < W; ++w) s += red[w * 256 + tid];
    const int v = tid >> 6, l = tid & 63;
    const int row = tr * 16 + 4 * (l >> 4) + v, col = tc * 16 + (l & 15);
    if (row < J.rows && col < J.cols) {
      const float pre = J.scale == 1.f ? s : J.scale * s;
      if constexpr (FWD) {
        const float z = p.bias ? pre + load_bias(p.bias, p.bias_kind, row, col) : pre;
        if (p.Z) p.Z[(int64_t)row * p.ldz + col] = z;
        J.out[(int64_t)row * J.ldo + col] = act_fwd(z, p.act, p.slope);
      } else {
        J.out[(int64_t)row * J.ldo + col] = pre;
      }
    }
  }
}

// Short reductions (at most 64): each wave of workgroup g owns tile W g + wave
// and runs the whole reduction itself; no LDS, no barrier.
template <int W, bool AV, bool BV, bool AZ, bool BZ, int ACT>
__device__ __forceinline__ void small_tile_own(const SmallArgs& p, const SmallJob& J, int g) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int t = g * W + wave;
  if (t >= J.tiles) return;
  const int tr = t / J.tiles_c, tc = t - tr * J.tiles_c;
  const int r = tr * 16 + (lane & 15), c = tc * 16 + (lane & 15), kq = lane >> 4;
  const bool rin = r < J.rows, cin = c < J.cols;
  const int blocks = (J.red + 15) >> 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < blocks; j0 += 4) {
    f32x4_t av[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k0 = 16 * (j0 + u) + 4 * kq;
      av[u] = rin ? small_load4<AV, AZ, ACT>(J.a, r, k0, J.red, p.slope) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      bv[u] = cin ? small_load4<BV, BZ, ACT>(J.b, c, k0, J.red, p.slope) : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][e], bv[u][e], acc, 0, 0, 0);
  }
  const int col = tc * 16 + (lane & 15);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = tr * 16 + 4 * (lane >> 4) + v;
    if (row < J.rows && col < J.cols) J.out[(int64_t)row * J.ldo + col] = J.scale == 1.f ? acc[v] : J.scale * acc[v];
  }
}

// PerN dBias: workgroup b sums columns 64 b + lane; wave w adds rows
// w, w + W, ... in order (16 loads of each array in flight), then wave 0 adds
// the W wave sums in order.
template <int W, int ACT>
__device__ __forceinline__ void small_dbias(const SmallArgs& p, int b, float* part) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int n = b * 64 + lane;
  float s = 0.f;
  if (n < p.N) {
    for (int m0 = wave; m0 < p.M; m0 += 16 * W) {
      float g[16], z[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int m = m0 + u * W;
        g[u] = m < p.M ? p.gY[(int64_t)m * p.ldgy + n] : 0.f;
        z[u] = m < p.M ? p.Zin[(int64_t)m * p.ldzin + n] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (m0 + u * W < p.M) s += g[u] * act_grad_t<ACT>(z[u], p.slope);
    }
  }
  part[wave * 64 + lane] = s;
  __syncthreads();
  if (wave == 0 && n < p.N) {
    float t = part[lane];
#pragma unroll
    for (int w = 1; w < W; ++w) t += part[w * 64 + lane];
    p.gbias[n] = t;
  }
}

// Forward: job 0, A / B contiguous along K (AV / BV) or not.
// TWO: the X operand comes in two parts (SmallOperand::p2)
template <int W, bool AV, bool BV, bool TWO = false>
__global__ void __launch_bounds__(W * 64) small_fwd_kernel(SmallArgs p) {
  __shared__ float red[W * 256];
  small_tile<W, AV, BV, false, false, kActNone, true, TWO>(p, p.job[0], blockIdx.x, red);
}

// Backward: tiles of the jobs (kind 1: dX, dY' on the left; kind 2: dW, dY'
// on the right), then the dBias columns.  GAV: both dX operands contiguous
// along the reduction.
template <int W, int ACT, bool GAV>
__device__ __forceinline__ void small_bwd_job(const SmallArgs& p, const SmallJob& J, int t, float* red) {
  if (J.kind == 1) {
    if (J.own) small_tile_own<W, GAV, GAV, true, false, ACT>(p, J, t);
    else small_tile<W, GAV, GAV, true, false, ACT, false>(p, J, t, red);
  } else {
    if (J.own) small_tile_own<W, false, false, false, true, ACT>(p, J, t);
    else small_tile<W, false, false, false, true, ACT, false>(p, J, t, red);
  }
}

template <int W, int ACT, bool GAV>
__global__ void __launch_bounds__(W * 64) small_bwd_kernel(SmallArgs p) {
  __shared__ float red[W * 256];
  const int t = blockIdx.x;
  const int t0 = p.njobs > 0 ? p.job[0].wgs : 0;
  const int t1 = p.njobs > 1 ? p.job[1].wgs : 0;
  if (t < t0) small_bwd_job<W, ACT, GAV>(p, p.job[0], t, red);
  else if (t < t0 + t1) small_bwd_job<W, ACT, GAV>(p, p.job[1], t - t0, red);
  else small_dbias<W, ACT>(p, t - t0 - t1, red);
}

template <int W>
static hipError_t launch_small_w(const SmallArgs& a, int wgs, hipStream_t s) {
  if (a.fwd) {
    const bool av = a.job[0].a.vec, bv = a.job[0].b.vec;
    if (a.job[0].a.p2) {
      if (av && bv) hipLaunchKernelGGL((small_fwd_kernel<W, true, true, true>), dim3(wgs), dim3(W * 64), 0, s, a);
      else if (av) hipLaunchKernelGGL((small_fwd_kernel<W, true, false, true>), dim3(wgs), dim3(W * 64), 0, s, a);
      else if (bv) hipLaunchKernelGGL((small_fwd_kernel<W, false, true, true>), dim3(wgs), dim3(W * 64), 0, s, a);
      else hipLaunchKernelGGL((small_fwd_kernel<W, false, false, true>), dim3(wgs), dim3(W * 64), 0, s, a);
    } else if (av && bv) hipLaunchKernelGGL((small_fwd_kernel<W, true, true>), dim3(wgs), dim3(W * 64), 0, s, a);
    else if (av) hipLaunchKernelGGL((small_fwd_kernel<W, true, false>), dim3(wgs), dim3(W * 64), 0, s, a);
    else if (bv) hipLaunchKernelGGL((small_fwd_kernel<W, false, true>), dim3(wgs), dim3(W * 64), 0, s, a);
    else hipLaunchKernelGGL((small_fwd_kernel<W, false, false>), dim3(wgs), dim3(W * 64), 0, s, a);
    return hipGetLastError();
  }
  bool gav = false;
  for (int j = 0; j < a.njobs; ++j)
    if (a.job[j].kind == 1) gav = a.job[j].a.vec && a.job[j].b.vec;
  const auto go = [&]<int ACT>() {
    if (gav) hipLaunchKernelGGL((small_bwd_kernel<W, ACT, true>), dim3(wgs), dim3(W * 64), 0, s, a);
    else hipLaunchKernelGGL((small_bwd_kernel<W, ACT, false>), dim3(wgs), dim3(W * 64), 0, s, a);
  };
  switch (a.act) {
    case kActRelu: go.template operator()<kActRelu>(); break;
    case kActLeaky: go.template operator()<kActLeaky>(); break;
    case kActGelu: go.template operator()<kActGelu>(); break;
    case kActSigmoid: go.template operator()<kActSigmoid>(); break;
    case kActTanh: go.template operator()<kActTanh>(); break;
    default: go.template operator()<kActNone>(); break;
  }
  return hipGetLastError();
}

int small_waves_for(int64_t red) { return red >= 512 ? 16 : 4; }

hipError_t launch_small(const SmallArgs& a, int waves, hipStream_t s) {
  int wgs = 0;
  for (int j = 0; j < a.njobs; ++j) {
    if (a.job[j].wgs != (a.job[j].own ? (a.job[j].tiles + waves - 1) / waves : a.job[j].tiles) ||
        (a.fwd && a.job[j].own))
      return hipErrorInvalidValue;
    wgs += a.job[j].wgs;
  }
  if (!a.fwd && a.gbias) wgs += (a.N + 63) / 64;
  if (wgs <= 0) return hipSuccess;
  return waves == 16 ? launch_small_w<16>(a, wgs, s) : launch_small_w<4>(a, wgs, s);
}

}  // namespace gev2
