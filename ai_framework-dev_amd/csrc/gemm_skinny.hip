// Bandwidth-bound forward for skinny shapes, Y[M,N] = act(alpha * X[M,K] W[K,N] + b)
// with M <= 16 (the reference runs these through its 128x128 FFMA tile and
// leaves almost every workgroup idle: regemm_gemm_bias_act.cu:254-395 with a
// (N/128, 1) grid).
//
// W dominates the traffic (K*N elements, read exactly once).  The grid is
// (N / slab) x splits: each workgroup streams a [K/splits, slab] block of W
// with 16-byte loads (16 lanes cover one slab row, 16 row groups per
// workgroup), keeps its slice of X in LDS, and accumulates M x (8 or 4)
// fp32 sums per lane -- v_dot2_f32_{bf16,f16} on row pairs for 16-bit data,
// FMA for fp32.  Row-group sums are reduced in LDS and written as one fp32
// partial per (split, m, n).  The last workgroup of a slab to arrive (an
// arrival counter per slab) adds the partials in split order, applies
// bias/activation/Z and stores Y, then resets the counter: deterministic and
// single-launch.
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

constexpr int kSkLanesPerRow = 16;  // lanes covering one slab row
constexpr int kSkRowGroups = 16;    // 256 threads
constexpr int kSkThreads = kSkLanesPerRow * kSkRowGroups;
static_assert(kSkLanesPerRow * 8 <= kSkThreads, "one thread per slab column in the reduction");
constexpr int kSkMaxKs = 1024;      // max K rows per split (LDS X slice)
constexpr int kSkStep = 128;        // K rows per main-loop iteration (both variants)

// Slab width in columns: 16 lanes x one 16-byte chunk each.
template <typename T> constexpr int slab_cols() { return kSkLanesPerRow * Elem<T>::kPerChunk; }

template <typename T, int MAXM>
__global__ void __launch_bounds__(kSkThreads) gemm_skinny_kernel(SkinnyArgs p) {
  constexpr int EPC = Elem<T>::kPerChunk;
  constexpr int NS = slab_cols<T>();
  constexpr bool kHalf = sizeof(T) == 2;
  // X slice: for 16-bit, dword (x[m][k], x[m][k+1]) pairs; for fp32, floats.
  __shared__ uint32_t xs[MAXM * kSkMaxKs / (kHalf ? 2 : 1)];
  __shared__ float red[kSkRowGroups][NS];
  __shared__ unsigned last_flag;

  const int tid = threadIdx.x;
  const int ln = tid % kSkLanesPerRow, rg = tid / kSkLanesPerRow;
  const int slab = blockIdx.x, split = blockIdx.y;
  const int n0 = slab * NS;
  const int ncol = n0 + ln * EPC;
  const int kbeg = split * p.k_per_split;
  const int kend = min(p.K, kbeg + p.k_per_split);
  const int M = p.M;

  const T* X = reinterpret_cast<const T*>(p.A);
  const T* W = reinterpret_cast<const T*>(p.B);

  // stage X[:, kbeg:kbeg+ks) into LDS, zero beyond kend; ks is padded to the
  // main loop's full step (128 rows) so that every LDS entry the loop reads was
  // written in this launch
  {
    const int ks = (p.k_per_split + kSkStep - 1) / kSkStep * kSkStep;
    if constexpr (kHalf) {
      const int pairs = ks / 2;
      for (int idx = tid; idx < MAXM * pairs; idx += kSkThreads) {
        const int m = idx / pairs, j = idx - m * pairs;
        const int k = kbeg + 2 * j;
        uint32_t lo = 0, hi = 0;
        if (m < M && k < kend) lo = *reinterpret_cast<const uint16_t*>(X + (int64_t)m * p.lda + k);
        if (m < M && k + 1 < kend) hi = *reinterpret_cast<const uint16_t*>(X + (int64_t)m * p.lda + k + 1);
        xs[m * (kSkMaxKs / 2) + j] = lo | (hi << 16);
      }
    } else {
      for (int idx = tid; idx < MAXM * ks; idx += kSkThreads) {
        const int m = idx / ks, j = idx - m * ks;
        const int k = kbeg + j;
        xs[m * kSkMaxKs + j] = (m < M && k < kend) ? __float_as_uint(X[(int64_t)m * p.lda + k]) : 0u;
      }
    }
  }
  __syncthreads();

  float acc[MAXM][EPC];
#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int c = 0; c < EPC; ++c) acc[m][c] = 0.f;

  const bool col_ok = ncol < p.N;   // N % EPC == 0 is required by the host
  const T* wcol = W + ncol;
  if constexpr (kHalf) {
    // rows kbeg + 2*rg + 32*i (+1)
    constexpr int U = 4;
    static_assert(2 * kSkRowGroups * U == kSkStep, "loop step");
    for (int kb = kbeg + 2 * rg; kb < kend; kb += 2 * kSkRowGroups * U) {
      u32x4 w0[U], w1[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb + u * 2 * kSkRowGroups;
        const bool ok0 = col_ok && k < kend, ok1 = col_ok && k + 1 < kend;
        w0[u] = ok0 ? *reinterpret_cast<const u32x4*>(wcol + (int64_t)k * p.ldb) : u32x4{0, 0, 0, 0};
        w1[u] = ok1 ? *reinterpret_cast<const u32x4*>(wcol + (int64_t)(k + 1) * p.ldb) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb + u * 2 * kSkRowGroups;
        const int j = (k - kbeg) >> 1;
        uint32_t pr[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pr[2 * q] = (w0[u][q] & 0xffffu) | (w1[u][q] << 16);
          pr[2 * q + 1] = (w0[u][q] >> 16) | (w1[u][q] & 0xffff0000u);
        }
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          const uint32_t xm = xs[m * (kSkMaxKs / 2) + min(j, kSkMaxKs / 2 - 1)];
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[m][c] = dot2<T>(pr[c], xm, acc[m][c]);
        }
      }
    }
  } else {
    constexpr int U = 8;
    static_assert(kSkRowGroups * U == kSkStep, "loop step");
    for (int kb = kbeg + rg; kb < kend; kb += kSkRowGroups * U) {
      u32x4 w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb + u * kSkRowGroups;
        w[u] = (col_ok && k < kend) ? *reinterpret_cast<const u32x4*>(wcol + (int64_t)k * p.ldb)
                                    : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = min(kb + u * kSkRowGroups - kbeg, kSkMaxKs - 1);
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          const float xm = __uint_as_float(xs[m * kSkMaxKs + j]);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(xm, __uint_as_float(w[u][c]), acc[m][c]);
        }
      }
    }
  }

  // reduce the 16 row groups, one output row at a time
  float* part = p.partial + (int64_t)split * M * p.N;
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    if (m < M) {   // uniform across the workgroup
#pragma unroll
      for (int c = 0; c < EPC; ++c) red[rg][ln * EPC + c] = acc[m][c];
      __syncthreads();
      if (tid < NS) {
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < kSkRowGroups; ++g) s += red[g][tid];
        const int n = n0 + tid;
        if (n < p.N) part[(int64_t)m * p.N + n] = s;
      }
      __syncthreads();
    }
  }

  // arrival: the last workgroup of this slab finishes it
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&p.counters[slab], 1u);
    last_flag = (prev == static_cast<unsigned>(p.splits - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();

  T* Y = reinterpret_cast<T*>(p.D);
  T* Zo = reinterpret_cast<T*>(p.Zo);
  for (int idx = tid; idx < M * NS; idx += kSkThreads) {
    const int m = idx / NS, c = idx - m * NS;
    const int n = n0 + c;
    if (n >= p.N) continue;
    float s = 0.f;
    for (int sp = 0; sp < p.splits; ++sp) s += p.partial[((int64_t)sp * M + m) * p.N + n];
    float pre = p.alpha == 1.f ? s : p.alpha * s;
    if (p.bias) pre += load_bias(p.bias, p.bias_kind, m, n);
    if (Zo) Elem<T>::store1(Zo + (int64_t)m * p.ldzo + n, pre);
    Elem<T>::store1(Y + (int64_t)m * p.ldd + n, act_fwd(pre, p.act, p.slope));
  }
  if (tid == 0) p.counters[slab] = 0u;
}

template <typename T>
static hipError_t launch_skinny_t(const SkinnyArgs& a, hipStream_t s) {
  constexpr int NS = slab_cols<T>();
  dim3 grid((a.N + NS - 1) / NS, a.splits);
  if (a.M <= 8)
    hipLaunchKernelGGL((gemm_skinny_kernel<T, 8>), grid, dim3(kSkThreads), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<T, 16>), grid, dim3(kSkThreads), 0, s, a);
  return hipGetLastError();
}

int skinny_slab_cols(int dtype) { return dtype == kF32 ? slab_cols<float>() : slab_cols<__bf16>(); }
int skinny_max_ks() { return kSkMaxKs; }

hipError_t launch_skinny(int dtype, const SkinnyArgs& a, int, hipStream_t s) {
  switch (dtype) {
    case kF32: return launch_skinny_t<float>(a, s);
    case kBF16: return launch_skinny_t<__bf16>(a, s);
    case kF16: return launch_skinny_t<_Float16>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
