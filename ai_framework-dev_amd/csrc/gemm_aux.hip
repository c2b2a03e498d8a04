// Small backward helpers for the cases the fused MFMA passes do not cover:
//   - gC = beta * gY (.) act'(Z), and gC = 0 when beta = 0 (the reference
//     zero-fills gC when C is absent or beta = 0: regemm_backward.cu:115-117,
//     :183-189)
//   - bias gradient when it cannot ride the dW pass: PerM (row sums), Scalar,
//     or PerN without a dW output.  (regemm_backward.cu:120-129 accumulates
//     these with fp32 atomics; here every sum has a fixed order.)
#include "gev2_device.hpp"
#include "gev2_kernels.hpp"
#include "skinny_nt_impl.hpp"

namespace gev2 {

template <typename T>
__global__ void __launch_bounds__(256) grad_elementwise_kernel(GradArgs p) {
  const int bz = blockIdx.y;
  const T* gY = reinterpret_cast<const T*>(p.gY) + (int64_t)bz * p.sgY;
  const T* Z = reinterpret_cast<const T*>(p.Z) + (int64_t)bz * p.sZ;
  T* out = reinterpret_cast<T*>(p.out) + (int64_t)bz * p.sOut;
  const int64_t total = (int64_t)p.M * p.N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int m = static_cast<int>(i / p.N), n = static_cast<int>(i - (int64_t)m * p.N);
    if (p.beta == 0.f) {
      // beta = 0: gC is zero, whatever dY holds (no 0 * inf)
      Elem<T>::store1(out + (int64_t)m * p.ldout + n, 0.f);
      continue;
    }
    const float g = Elem<T>::load1(gY + (int64_t)m * p.ldgy + n);
    const float z = Elem<T>::load1(Z + (int64_t)m * p.ldz + n);
    Elem<T>::store1(out + (int64_t)m * p.ldout + n, p.beta * (g * act_grad(z, p.act, p.slope)));
  }
}

// PerN: 64 columns x 4 row lanes per workgroup; each thread walks its rows in
// order, then the 4 lanes are added in order.
template <typename T>
__global__ void __launch_bounds__(256) bias_grad_cols_kernel(GradArgs p) {
  __shared__ float red[4][64];
  const int bz = blockIdx.y;
  const T* gY = reinterpret_cast<const T*>(p.gY) + (int64_t)bz * p.sgY;
  const T* Z = reinterpret_cast<const T*>(p.Z) + (int64_t)bz * p.sZ;
  const int c = threadIdx.x & 63, r = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + c;
  float s = 0.f;
  if (n < p.N) {
    for (int m = r; m < p.M; m += 4) {
      const float g = Elem<T>::load1(gY + (int64_t)m * p.ldgy + n);
      const float z = Elem<T>::load1(Z + (int64_t)m * p.ldz + n);
      s += g * act_grad(z, p.act, p.slope);
    }
  }
  red[r][c] = s;
  __syncthreads();
  if (r == 0 && n < p.N) p.gbias[(int64_t)bz * p.sGbias + n] = red[0][c] + red[1][c] + red[2][c] + red[3][c];
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// PerM: one wave per row.  VEC: rows are read in 16-byte chunks (every row and
// slice start 16-byte aligned, N a multiple of the chunk).
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) bias_grad_rows_kernel(GradArgs p) {
  const int bz = blockIdx.y;
  const T* gY = reinterpret_cast<const T*>(p.gY) + (int64_t)bz * p.sgY;
  const T* Z = reinterpret_cast<const T*>(p.Z) + (int64_t)bz * p.sZ;
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= p.M) return;
  float s = 0.f;
  const T* grow = gY + (int64_t)m * p.ldgy;
  const T* zrow = Z + (int64_t)m * p.ldz;
  dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
    if constexpr (VEC) {
      constexpr int EPC = Elem<T>::kPerChunk;
      for (int n = lane * EPC; n < p.N; n += 64 * EPC) {
        float gv[EPC], zv[EPC];
        chunk_to_f32<T>(*reinterpret_cast<const u32x4*>(grow + n), gv);
        chunk_to_f32<T>(*reinterpret_cast<const u32x4*>(zrow + n), zv);
#pragma unroll
        for (int e = 0; e < EPC; ++e) s += gv[e] * act_grad_t<ACT>(zv[e], p.slope);
      }
    } else {
      for (int n = lane; n < p.N; n += 64) s += Elem<T>::load1(grow + n) * act_grad_t<ACT>(Elem<T>::load1(zrow + n), p.slope);
    }
  });
  s = wave_sum(s);
  if (lane == 0) p.gbias[(int64_t)bz * p.sGbias + m] = s;
}

// Scalar: one workgroup per slice sums everything.
template <typename T>
__global__ void __launch_bounds__(256) bias_grad_all_kernel(GradArgs p) {
  __shared__ float red[4];
  const int bz = blockIdx.y;
  const T* gY = reinterpret_cast<const T*>(p.gY) + (int64_t)bz * p.sgY;
  const T* Z = reinterpret_cast<const T*>(p.Z) + (int64_t)bz * p.sZ;
  const int64_t total = (int64_t)p.M * p.N;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < total; i += 256) {
    const int m = static_cast<int>(i / p.N), n = static_cast<int>(i - (int64_t)m * p.N);
    const float g = Elem<T>::load1(gY + (int64_t)m * p.ldgy + n);
    const float z = Elem<T>::load1(Z + (int64_t)m * p.ldz + n);
    s += g * act_grad(z, p.act, p.slope);
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) p.gbias[(int64_t)bz * p.sGbias] = red[0] + red[1] + red[2] + red[3];
}

// grad_prep: 256 threads = 32 chunk columns x 8 row lanes; a workgroup covers
// kPrepRows rows x (32 * EPC) columns.  Each thread walks its rows in order,
// the 8 row lanes are then added in order: the partial sums are deterministic.
template <typename T>
__global__ void __launch_bounds__(256) grad_prep_kernel(PrepArgs p) {
  constexpr int EPC = Elem<T>::kPerChunk;
  constexpr int COLS = 32 * EPC;
  __shared__ float red[8][COLS];
  const int bz = blockIdx.z;
  const T* gY = reinterpret_cast<const T*>(p.gY) + (int64_t)bz * p.sgY;
  const T* Z = reinterpret_cast<const T*>(p.Z) + (int64_t)bz * p.sZ;
  T* out = reinterpret_cast<T*>(p.out) + (int64_t)bz * p.sOut;
  const int cc = threadIdx.x & 31, rl = threadIdx.x >> 5;
  const int n = blockIdx.x * COLS + cc * EPC;
  const int r0 = blockIdx.y * kPrepRows;
  const bool nok = n < p.N;
  float sum[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) sum[e] = 0.f;
  // every load of the thread's rows is issued before the first store (the
  // output may not be assumed disjoint from the inputs, so stores would
  // otherwise hold back the next row's loads)
  constexpr int RPT = kPrepRows / 8;
  u32x4 g[RPT], z[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int m = r0 + rl + 8 * i;
    if (nok && m < p.M) {
      g[i] = *reinterpret_cast<const u32x4*>(gY + (int64_t)m * p.ldgy + n);
      z[i] = *reinterpret_cast<const u32x4*>(Z + (int64_t)m * p.ldz + n);
    }
  }
  dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int m = r0 + rl + 8 * i;
      if (!nok || m >= p.M) continue;
      float gv[EPC], zv[EPC];
      chunk_to_f32<T>(g[i], gv);
      chunk_to_f32<T>(z[i], zv);
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        gv[e] *= act_grad_t<ACT>(zv[e], p.slope);
        sum[e] += gv[e];
      }
      *reinterpret_cast<u32x4*>(out + (int64_t)m * p.N + n) = f32_to_chunk<T>(gv);
    }
  });
  if (!p.partial) return;
#pragma unroll
  for (int e = 0; e < EPC; ++e) red[rl][cc * EPC + e] = sum[e];
  __syncthreads();
  const int c = threadIdx.x;
  if (c < COLS && blockIdx.x * COLS + c < p.N) {
    float s = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) s += red[l][c];
    p.partial[(int64_t)bz * p.sPartial + (int64_t)blockIdx.y * p.N + blockIdx.x * COLS + c] = s;
  }
}

// grad_prep for a PerM bias: one wave per row writes that row of dY' and its
// sum, so the bias gradient needs no second pass over dY and Z.  Lanes take
// chunks lane, lane + 64, ... (four per round, their loads issued together)
// and add them in that order; the wave's butterfly then adds the lanes.
template <typename T>
__global__ void __launch_bounds__(256) grad_prep_rows_kernel(PrepArgs p) {
  constexpr int EPC = Elem<T>::kPerChunk;
  constexpr int U = 4;
  const int bz = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= p.M) return;                              // wave-uniform; no barrier below
  const T* grow = reinterpret_cast<const T*>(p.gY) + (int64_t)bz * p.sgY + (int64_t)m * p.ldgy;
  const T* zrow = reinterpret_cast<const T*>(p.Z) + (int64_t)bz * p.sZ + (int64_t)m * p.ldz;
  T* orow = reinterpret_cast<T*>(p.out) + (int64_t)bz * p.sOut + (int64_t)m * p.N;
  float s = 0.f;
  dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
    for (int n0 = lane * EPC; n0 < p.N; n0 += U * 64 * EPC) {
      u32x4 g[U], z[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int n = n0 + u * 64 * EPC;
        if (n < p.N) {
          g[u] = *reinterpret_cast<const u32x4*>(grow + n);
          z[u] = *reinterpret_cast<const u32x4*>(zrow + n);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int n = n0 + u * 64 * EPC;
        if (n < p.N) {
          float gv[EPC], zv[EPC];
          chunk_to_f32<T>(g[u], gv);
          chunk_to_f32<T>(z[u], zv);
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            gv[e] *= act_grad_t<ACT>(zv[e], p.slope);
            s += gv[e];
          }
          *reinterpret_cast<u32x4*>(orow + n) = f32_to_chunk<T>(gv);
        }
      }
    }
  });
  s = wave_sum(s);
  if (lane == 0) p.rowsum[(int64_t)bz * p.sRowsum + m] = s;
}

// 64 columns x 4 row-block lanes per workgroup: lane g adds row blocks
// g, g+4, ... in order (independent loads, unrolled), then the 4 lanes are
// added in order.
__global__ void __launch_bounds__(256) finish_col_sums_kernel(const float* partial, int64_t sPartial,
                                                              int row_blocks, int N, float* gbias,
                                                              int64_t sGbias) {
  __shared__ float red[4][64];
  const int c = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + c;
  const int bz = blockIdx.y;
  float s = 0.f;
  if (n < N) {
    const float* pp = partial + (int64_t)bz * sPartial + n;
#pragma unroll 8
    for (int rb = g; rb < row_blocks; rb += 4) s += pp[(int64_t)rb * N];
  }
  red[g][c] = s;
  __syncthreads();
  if (g == 0 && n < N) gbias[(int64_t)bz * sGbias + n] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
}

// Skinny NT product for the backward's gA when M <= 16:
//   D[m][k] = alpha * sum_n G[m][n] * (Z ? act'(Z[m][n]) : 1) * B[k][n].
// Every output column k is a dot product of one contiguous row of B with the
// M rows of G: one wave per k (skinny_nt_column); G (and Z) are small and come
// from L2.
template <typename T, int MAXM>
__global__ void __launch_bounds__(256) skinny_nt_kernel(SkinnyNtArgs p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.x * 4 + wave;
  if (k >= p.K) return;                              // wave-uniform; no barrier below
  float v[16];
  skinny_nt_column<T, MAXM, skinny_nt_passes<T>(MAXM)>(p, k, lane, v);
  T* D = reinterpret_cast<T*>(p.D);
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    if (m >= p.M) continue;
    if (lane == 0) Elem<T>::store1(D + (int64_t)m * p.ldd + k, p.alpha * v[m]);
  }
}

hipError_t launch_skinny_nt(int dtype, const SkinnyNtArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.K + 3) / 4));
  switch (dtype) {
    case kF32:
      if (a.M <= 8) hipLaunchKernelGGL((skinny_nt_kernel<float, 8>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((skinny_nt_kernel<float, 16>), grid, dim3(256), 0, s, a);
      break;
    case kBF16:
      if (a.M <= 8) hipLaunchKernelGGL((skinny_nt_kernel<__bf16, 8>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((skinny_nt_kernel<__bf16, 16>), grid, dim3(256), 0, s, a);
      break;
    case kF16:
      if (a.M <= 8) hipLaunchKernelGGL((skinny_nt_kernel<_Float16, 8>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((skinny_nt_kernel<_Float16, 16>), grid, dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// fp32 split-K reduction: one thread per output element (64 threads per
// workgroup, so even a 64x256 output spreads over 256 workgroups); the ks
// slices are added in order s = 0, 1, ... with 16 loads in flight, then alpha,
// bias, Z and act.
__global__ void __launch_bounds__(64) splitk_reduce_kernel(SplitkReduceArgs p) {
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (i >= (int64_t)p.M * p.N) return;
  const int m = static_cast<int>(i / p.N), n = static_cast<int>(i - (int64_t)m * p.N);
  const int64_t slice = (int64_t)p.M * p.N;
  const float* src = p.part + i;
  float acc = src[0];
  for (int s0 = 1; s0 < p.ks; s0 += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = s0 + u < p.ks ? src[(s0 + u) * slice] : 0.f;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (s0 + u < p.ks) acc += v[u];
  }
  const float b = p.bias ? load_bias(p.bias, p.bias_kind, m, n) : 0.f;
  const float z = fmaf(p.alpha, acc, b);
  if (p.Z) p.Z[(int64_t)m * p.ldz + n] = z;
  p.Y[(int64_t)m * p.ldy + n] = act_fwd(z, p.act, p.slope);
}

hipError_t launch_splitk_reduce(const SplitkReduceArgs& a, hipStream_t s) {
  const int64_t threads = (int64_t)a.M * a.N;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>((threads + 63) / 64)), dim3(64), 0, s, a);
  return hipGetLastError();
}

template <typename T>
static hipError_t grad_prep_t(const PrepArgs& a, int batch, hipStream_t s) {
  if (a.rowsum) {
    hipLaunchKernelGGL(grad_prep_rows_kernel<T>, dim3((a.M + 3) / 4, batch), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  constexpr int COLS = 32 * Elem<T>::kPerChunk;
  dim3 grid((a.N + COLS - 1) / COLS, (a.M + kPrepRows - 1) / kPrepRows, batch);
  hipLaunchKernelGGL(grad_prep_kernel<T>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_grad_prep(int dtype, const PrepArgs& a, int batch, hipStream_t s) {
  switch (dtype) {
    case kF32: return grad_prep_t<float>(a, batch, s);
    case kBF16: return grad_prep_t<__bf16>(a, batch, s);
    case kF16: return grad_prep_t<_Float16>(a, batch, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_finish_col_sums(const float* partial, int64_t sPartial, int row_blocks, int N,
                                  float* gbias, int64_t sGbias, int batch, hipStream_t s) {
  hipLaunchKernelGGL(finish_col_sums_kernel, dim3((N + 63) / 64, batch), dim3(256), 0, s, partial, sPartial,
                     row_blocks, N, gbias, sGbias);
  return hipGetLastError();
}

template <typename T>
static hipError_t grad_elementwise_t(const GradArgs& a, int batch, hipStream_t s) {
  const int64_t total = (int64_t)a.M * a.N;
  int64_t nb = (total + 255) / 256;
  int blocks = static_cast<int>(nb < 4096 ? nb : 4096);
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(grad_elementwise_kernel<T>, dim3(blocks, batch), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <typename T>
static hipError_t bias_grad_t(const GradArgs& a, int batch, hipStream_t s) {
  switch (a.bias_kind) {
    case kBiasPerN:
      hipLaunchKernelGGL(bias_grad_cols_kernel<T>, dim3((a.N + 63) / 64, batch), dim3(256), 0, s, a);
      break;
    case kBiasPerM: {
      constexpr int EPC = Elem<T>::kPerChunk;
      const auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
      const bool vec = al(a.gY) && al(a.Z) && a.N % EPC == 0 && a.ldgy % EPC == 0 && a.ldz % EPC == 0 &&
                       (batch == 1 || (a.sgY % EPC == 0 && a.sZ % EPC == 0));
      if (vec) hipLaunchKernelGGL((bias_grad_rows_kernel<T, true>), dim3((a.M + 3) / 4, batch), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((bias_grad_rows_kernel<T, false>), dim3((a.M + 3) / 4, batch), dim3(256), 0, s, a);
      break;
    }
    case kBiasScalar:
      hipLaunchKernelGGL(bias_grad_all_kernel<T>, dim3(1, batch), dim3(256), 0, s, a);
      break;
    default: return hipSuccess;
  }
  return hipGetLastError();
}

hipError_t launch_grad_elementwise(int dtype, const GradArgs& a, int batch, hipStream_t s) {
  switch (dtype) {
    case kF32: return grad_elementwise_t<float>(a, batch, s);
    case kBF16: return grad_elementwise_t<__bf16>(a, batch, s);
    case kF16: return grad_elementwise_t<_Float16>(a, batch, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bias_grad(int dtype, const GradArgs& a, int batch, hipStream_t s) {
  switch (dtype) {
    case kF32: return bias_grad_t<float>(a, batch, s);
    case kBF16: return bias_grad_t<__bf16>(a, batch, s);
    case kF16: return bias_grad_t<_Float16>(a, batch, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
