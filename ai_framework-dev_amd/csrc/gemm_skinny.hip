// Bandwidth-bound forward for skinny shapes, Y[M,N] = act(alpha * X[M,K] W[K,N] + b)
// with M <= 16.  The reference runs these through its 128x128 FFMA tile and
// leaves almost every workgroup idle (regemm_gemm_bias_act.cu:254-395 with a
// (N/128, 1) grid).
//
// W dominates the traffic (K*N elements, read exactly once), so the kernel is
// built around streaming it:
//   - one workgroup per slab of 32 bytes of every W row (16 bf16/f16 columns or
//     8 fp32 columns), covering all of K: no cross-workgroup reduction, hence
//     no device-scope fence (which on an 8-XCD part writes back L2);
//   - slabs are assigned so that the workgroups of one XCD take adjacent slabs
//     and share each 128-byte line of W through that XCD's L2;
//   - each lane pair reads one row's 32 bytes with 16-byte loads, a thread's
//     rows of a K chunk are all in flight at once;
//   - X[:, chunk] sits in LDS as k-pairs (x[k][m], x[k+1][m]), so 16-bit data
//     uses v_dot2_f32_{bf16,f16} on W row pairs; fp32 uses FMA;
//   - the 128 row lanes are summed by a fixed shuffle tree and a fixed-order
//     LDS pass (deterministic), then bias / activation / Z / Y.
#include "gev2_device.hpp"
#include "gev2_kernels.hpp"

namespace gev2 {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (__is_same(T, __bf16)) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
  }
}

constexpr int kOobOffsetSk = static_cast<int>(0x80000000u);
constexpr int kSkThreads = 256;
constexpr int kSkRowLanes = kSkThreads / 2;   // lane pairs

template <typename T> constexpr int sk_cols() { return 2 * Elem<T>::kPerChunk; }

// K rows per LDS chunk of X: the whole of K = 4096 for 16-bit data with
// M <= 8, so that a thread has all of its W rows in flight at once.
template <typename T, int MAXM>
constexpr int sk_chunk() { return (sizeof(T) == 2 && MAXM == 8) ? 4096 : 2048; }

template <typename T, int MAXM>
__global__ void __launch_bounds__(kSkThreads) gemm_skinny_kernel(SkinnyArgs p) {
  constexpr int kSkChunk = sk_chunk<T, MAXM>();
  constexpr bool kHalf = sizeof(T) == 2;
  constexpr int EPC = Elem<T>::kPerChunk;
  constexpr int COLS = sk_cols<T>();
  // rows each thread handles per chunk: 16-bit data in k pairs
  constexpr int RSTEP = kHalf ? 2 : 1;
  constexpr int RPT = kSkChunk / (kSkRowLanes * RSTEP);
  // X chunk: 16-bit -> dwords (x[k][m], x[k+1][m]) at [k/2][m]; fp32 -> [k][m]
  // X chunk, reused for the final reduction (MH * EPC * 256 floats)
  constexpr int MH = MAXM < 8 ? MAXM : 8;
  constexpr int XS = (kSkChunk / RSTEP) * MAXM, RS = MH * EPC * kSkThreads;
  __shared__ uint32_t xs[XS > RS ? XS : RS];

  const int tid = threadIdx.x;
  const int h = tid & 1, rl = tid >> 1;
  // XCD-aware slab order: workgroup i runs on XCD i % 8
  int slab = blockIdx.x;
  const int nslab = gridDim.x;
  if ((nslab & 7) == 0) slab = (slab & 7) * (nslab >> 3) + (slab >> 3);
  const int n = slab * COLS + h * EPC;
  const bool nok = n < p.N;   // N % EPC == 0 (host)
  const int M = p.M;

  const T* X = reinterpret_cast<const T*>(p.A);
  const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.B), static_cast<short>(0),
                                                                      0x7fffffff, 0x00020000);
  float acc[MAXM][EPC];
#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[m][e] = 0.f;

  for (int kc0 = 0; kc0 < p.K; kc0 += kSkChunk) {
    // W rows of this thread: k = kc0 + (rl + kSkRowLanes * i) * RSTEP (+1)
    u32x4 w[RPT][RSTEP];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int r = 0; r < RSTEP; ++r) {
        const int k = kc0 + (rl + kSkRowLanes * i) * RSTEP + r;
        const int off = (nok && k < p.K) ? static_cast<int>(((int64_t)k * p.ldb + n) * sizeof(T)) : kOobOffsetSk;
        w[i][r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, off, 0, 0));
      }
    // stage X[:, kc0 : kc0 + kSkChunk) (zero beyond M and K); with x_vec each
    // thread reads 16 bytes (EPC consecutive k of one row m)
    __syncthreads();
    if (p.x_vec) {
      for (int idx = tid; idx < (kSkChunk / EPC) * MAXM; idx += kSkThreads) {
        const int m = idx % MAXM, j = idx / MAXM;
        const int k = kc0 + j * EPC;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (m < M && k < p.K) v = *reinterpret_cast<const u32x4*>(X + (int64_t)m * p.lda + k);
        if constexpr (kHalf) {
#pragma unroll
          for (int q = 0; q < 4; ++q) xs[(4 * j + q) * MAXM + m] = v[q];   // (x[k+2q], x[k+2q+1])
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) xs[(4 * j + q) * MAXM + m] = v[q];
        }
      }
    } else if constexpr (kHalf) {
      for (int idx = tid; idx < (kSkChunk / 2) * MAXM; idx += kSkThreads) {
        const int m = idx % MAXM, j = idx / MAXM;
        const int k = kc0 + 2 * j;
        uint32_t lo = 0, hi = 0;
        if (m < M && k < p.K) lo = *reinterpret_cast<const uint16_t*>(X + (int64_t)m * p.lda + k);
        if (m < M && k + 1 < p.K) hi = *reinterpret_cast<const uint16_t*>(X + (int64_t)m * p.lda + k + 1);
        xs[j * MAXM + m] = lo | (hi << 16);
      }
    } else {
      for (int idx = tid; idx < kSkChunk * MAXM; idx += kSkThreads) {
        const int m = idx % MAXM, j = idx / MAXM;
        const int k = kc0 + j;
        xs[j * MAXM + m] = (m < M && k < p.K) ? __float_as_uint(X[(int64_t)m * p.lda + k]) : 0u;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int j = rl + kSkRowLanes * i;   // k pair (16-bit) or k (fp32) within the chunk
      const u32x4* xv = reinterpret_cast<const u32x4*>(xs + j * MAXM);
      if constexpr (kHalf) {
        uint32_t pr[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pr[2 * q] = (w[i][0][q] & 0xffffu) | (w[i][1][q] << 16);
          pr[2 * q + 1] = (w[i][0][q] >> 16) | (w[i][1][q] & 0xffff0000u);
        }
#pragma unroll
        for (int mq = 0; mq < MAXM / 4; ++mq) {
          const u32x4 x4 = xv[mq];
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[mq * 4 + t][e] = dot2<T>(pr[e], x4[t], acc[mq * 4 + t][e]);
        }
      } else {
#pragma unroll
        for (int mq = 0; mq < MAXM / 4; ++mq) {
          const u32x4 x4 = xv[mq];
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[mq * 4 + t][e] = fmaf(__uint_as_float(x4[t]), __uint_as_float(w[i][0][e]), acc[mq * 4 + t][e]);
        }
      }
    }
  }

  // Sum over the 128 row lanes in a fixed order, MH rows of X at a time: each
  // thread stores its sums at red[v][rl][h] (v = m * EPC + e), then two
  // threads per output each add 64 row lanes in order and the pair is added.
  float* red = reinterpret_cast<float*>(xs);
  T* Y = reinterpret_cast<T*>(p.D);
  T* Zo = reinterpret_cast<T*>(p.Zo);
#pragma unroll
  for (int m0 = 0; m0 < MAXM; m0 += MH) {
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < MH; ++mm)
#pragma unroll
      for (int e = 0; e < EPC; ++e) red[(mm * EPC + e) * kSkThreads + tid] = acc[m0 + mm][e];
    __syncthreads();
    // output o = (mm, c) for c < COLS; threads 2o, 2o+1
    const int o = tid >> 1, part = tid & 1;
    float s = 0.f;
    const int mm = o / COLS, c = o % COLS;
    if (mm < MH) {
      const int hh = c / EPC, e = c % EPC;
      const float* col = red + (mm * EPC + e) * kSkThreads + hh;
      for (int r = part * 64; r < part * 64 + 64; ++r) s += col[2 * r];
    }
    const float s_hi = __shfl_xor(s, 1, 64);
    const int m = m0 + mm;
    const int nn = slab * COLS + c;
    if (part == 0 && mm < MH && m < M && nn < p.N) {
      const float tot = s + s_hi;
      float pre = p.alpha == 1.f ? tot : p.alpha * tot;
      if (p.bias) pre += load_bias(p.bias, p.bias_kind, m, nn);
      if (Zo) Elem<T>::store1(Zo + (int64_t)m * p.ldzo + nn, pre);
      Elem<T>::store1(Y + (int64_t)m * p.ldd + nn, act_fwd(pre, p.act, p.slope));
    }
  }
}

template <typename T>
static hipError_t launch_skinny_t(const SkinnyArgs& a, hipStream_t s) {
  constexpr int COLS = sk_cols<T>();
  dim3 grid((a.N + COLS - 1) / COLS);
  if (a.M <= 8)
    hipLaunchKernelGGL((gemm_skinny_kernel<T, 8>), grid, dim3(kSkThreads), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<T, 16>), grid, dim3(kSkThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_skinny(int dtype, const SkinnyArgs& a, hipStream_t s) {
  switch (dtype) {
    case kF32: return launch_skinny_t<float>(a, s);
    case kBF16: return launch_skinny_t<__bf16>(a, s);
    case kF16: return launch_skinny_t<_Float16>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
