// Elman RNN on the GEMM operator: the rnn launcher of graph_executor_v2
// (backends/cuda/ops/rnn/launcher.cu:129-383, kernels.cu) rebuilt around it.
//
//   h_t = act(X_t Wx + h_{t-1} Wh + b),  Y[:,t,:] = h_t,  Z[:,t,:] = pre-activation,
//   X [N,T,I], Wx [I,H], Wh [H,H], h0 [N,H], b [H] fp32, Y / Z [N,T,H].
//
// Forward, per step: one gather kernel writes XH = [X_t, h_{t-1}] ([N, I+H]),
// then ONE operator forward XH . [Wx; Wh] (+ b, act) writes h_t and Z_t
// straight into Y[:,t,:] and Z[:,t,:] through their row stride T*H, and the
// next step reads h_t from Y.  For 16-bit batches of at most 16 rows with I a
// whole number of 256-row K blocks (and the operator scratch in the
// descriptor), the skinny split-K kernel reads X_t and h_{t-1} in place
// instead, and the gather launch goes.  The reference copies X_t and h_{t-1} in with
// two 2-D copies and Y_rows / Z_rows out with two more per step.
// Backward (BPTT), per step from T-1 down to 0: one gather kernel rebuilds
// XH = [X_t, act(Z_{t-1}) or h0], forms G = dY_t + dh_next (dh_next = the
// h-columns of the previous step's dXH) and stores the previous step's dX;
// then ONE operator backward with gY = G, Z = Z[:,t,:] (stride T*H) gives
// dXH = G' [Wx; Wh]^T, dWcat_t = XH^T G' and dB_t; one kernel adds dWcat_t
// and dB_t to fp32 sums in step order.  dB is the sum over all steps (the
// reference's per-step GEMM backward zero-fills it, so it keeps step 0's only).
// With N <= 16 and N*T <= I+H (rnn_bwd_gathered) the step is one kernel:
// G'_t = G * act'(Z_t) is kept for all steps in an [N, T, H] buffer, step t
// computes dXH_t = G'_t Wcat^T column by column and turns each column into
// dX_t or G'_{t-1} at once; dWx = X^T G', dWh = Hprev^T G' and dB are formed
// once after the loop, each a sum of depth N*T rounded once.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <list>
#include <mutex>
#include <set>
#include <string>

#include "../../include/gev2_gemm.h"
#include "gev2_device.hpp"
#include "gev2_kernels.hpp"
#include "skinny_nt_impl.hpp"

namespace gev2 {

struct RnnDims {
  int N, T, I, H;
};

// xh[n, :I] = X[n, t, :];  xh[n, I:] = hprev[n * ldh + :]
template <typename T>
__global__ void __launch_bounds__(256) rnn_fwd_gather_kernel(const T* __restrict__ X, const T* __restrict__ hprev,
                                                             int64_t ldh, T* __restrict__ xh, RnnDims d, int t) {
  const int IH = d.I + d.H;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)d.N * IH) return;
  const int n = static_cast<int>(idx / IH), j = static_cast<int>(idx - (int64_t)n * IH);
  xh[idx] = j < d.I ? X[((int64_t)n * d.T + t) * d.I + j] : hprev[n * ldh + (j - d.I)];
}

// Step t of the backward (T > t >= 0):
//   xh[n, :I]  = X[n, t, :]
//   xh[n, I:]  = t > 0 ? act(Z[n, t-1, :]) : h0[n, :]
//   g[n, :]    = dY[n, t, :] + (t < T-1 ? dxh[n, I:] : 0)
//   dX[n, t+1, :] = dxh[n, :I]            (t < T-1, dX requested)
template <typename T>
__global__ void __launch_bounds__(256) rnn_bwd_gather_kernel(const T* __restrict__ X, const T* __restrict__ Z,
                                                             const T* __restrict__ h0, const T* __restrict__ dY,
                                                             const T* __restrict__ dxh, T* __restrict__ xh,
                                                             T* __restrict__ g, T* __restrict__ dX, RnnDims d, int t,
                                                             int act, float slope) {
  const int IH = d.I + d.H;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)d.N * IH) return;
  const int n = static_cast<int>(idx / IH), j = static_cast<int>(idx - (int64_t)n * IH);
  const bool last = t == d.T - 1;
  if (j < d.I) {
    xh[idx] = X[((int64_t)n * d.T + t) * d.I + j];
    if (dX && !last) dX[((int64_t)n * d.T + t + 1) * d.I + j] = dxh[idx];
  } else {
    const int h = j - d.I;
    if (t > 0)
      Elem<T>::store1(xh + idx, act_fwd(Elem<T>::load1(Z + ((int64_t)n * d.T + t - 1) * d.H + h), act, slope));
    else
      xh[idx] = h0[(int64_t)n * d.H + h];
    float gy = Elem<T>::load1(dY + ((int64_t)n * d.T + t) * d.H + h);
    if (!last) gy += Elem<T>::load1(dxh + idx);
    Elem<T>::store1(g + (int64_t)n * d.H + h, gy);
  }
}

// Step t of the backward in the gathered-G' form (N <= 16; used for the first
// step, t = T-1, whose G' needs no dh_next):
//   G'[n, t, :] = (dY[n, t, :] + (t < T-1 ? dxh[n, I:] : 0)) * act'(Z[n, t, :])
//   dX[n, t+1, :] = dxh[n, :I]            (t < T-1, dX requested)
// G' ([N, T, H], row stride T*H) is kept for the weight gradients after the loop.
template <typename T>
__global__ void __launch_bounds__(256) rnn_bwd_gather_g_kernel(const T* __restrict__ Z, const T* __restrict__ dY,
                                                               const T* __restrict__ dxh, T* __restrict__ gall,
                                                               T* __restrict__ dX, RnnDims d, int t, int act,
                                                               float slope) {
  const int IH = d.I + d.H;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)d.N * IH) return;
  const int n = static_cast<int>(idx / IH), j = static_cast<int>(idx - (int64_t)n * IH);
  const bool last = t == d.T - 1;
  if (j < d.I) {
    if (dX && !last) dX[((int64_t)n * d.T + t + 1) * d.I + j] = dxh[idx];
  } else {
    const int h = j - d.I;
    const int64_t o = ((int64_t)n * d.T + t) * d.H + h;
    float gy = Elem<T>::load1(dY + o);
    if (!last) gy += Elem<T>::load1(dxh + idx);
    Elem<T>::store1(gall + o, gy * act_grad(Elem<T>::load1(Z + o), act, slope));
  }
}

// Backward step t >= 1 of the gathered-G' form in one kernel: wave k forms
// column k of dXH_t = G'_t Wcat^T (skinny_nt_column) and consumes it at once,
// lane m taking row m: a column k < I is dX[m, t, k]; a column I + h is
// dh_next[m, h], from which the lane forms
//   G'[m, t-1, h] = (dY[m, t-1, h] + dh_next[m, h]) * act'(Z[m, t-1, h]).
// dXH itself is never stored.
template <typename T, int MAXM>
__global__ void __launch_bounds__(256) rnn_step_nt_kernel(SkinnyNtArgs p, const T* __restrict__ dY,
                                                          const T* __restrict__ Z, T* __restrict__ gall,
                                                          T* __restrict__ dX, RnnDims d, int t, int act, float slope) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.x * 4 + wave;
  if (k >= p.K) return;                              // wave-uniform; no barrier below
  float v[16];
  skinny_nt_column<T, MAXM, skinny_nt_passes<T>(MAXM)>(p, k, lane, v);
  if (lane >= p.M) return;
  float x = 0.f;
#pragma unroll
  for (int m = 0; m < 16; ++m)
    if (lane == m) x = v[m];
  const int m = lane;
  if (k < d.I) {
    if (dX) Elem<T>::store1(dX + ((int64_t)m * d.T + t) * d.I + k, x);
  } else {
    const int64_t o = ((int64_t)m * d.T + t - 1) * d.H + (k - d.I);
    const float gy = Elem<T>::load1(dY + o) + x;
    Elem<T>::store1(gall + o, gy * act_grad(Elem<T>::load1(Z + o), act, slope));
  }
}

// hprev[n, t, :] = t > 0 ? act(Z[n, t-1, :]) : h0[n, :]   ([N, T, H])
template <typename T>
__global__ void __launch_bounds__(256) rnn_hprev_kernel(const T* __restrict__ Z, const T* __restrict__ h0,
                                                        T* __restrict__ hprev, RnnDims d, int act, float slope) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)d.N * d.T * d.H) return;
  const int h = static_cast<int>(idx % d.H);
  const int64_t nt = idx / d.H;
  const int t = static_cast<int>(nt % d.T), n = static_cast<int>(nt / d.T);
  if (t > 0)
    Elem<T>::store1(hprev + idx, act_fwd(Elem<T>::load1(Z + idx - d.H), act, slope));
  else
    hprev[idx] = h0[(int64_t)n * d.H + h];
}

// dB[h] = sum over the rows r = 0 .. rows-1 of g[r, h], in row order (fp32).
template <typename T>
__global__ void __launch_bounds__(256) rnn_colsum_kernel(const T* __restrict__ g, int64_t rows, int H,
                                                         float* __restrict__ dB) {
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float s = 0.f;
#pragma unroll 8
  for (int64_t r = 0; r < rows; ++r) s += Elem<T>::load1(g + r * H + h);
  dB[h] = s;
}

// dwcat[i] = (first ? 0 : dwcat[i]) + tmpw[i];  dB[h] likewise from gb
template <typename T>
__global__ void __launch_bounds__(256) rnn_acc_kernel(float* __restrict__ dwcat, const T* __restrict__ tmpw,
                                                      int64_t nw, float* __restrict__ dB, const float* __restrict__ gb,
                                                      int H, int first) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nw) {
    const float v = Elem<T>::load1(tmpw + i);
    dwcat[i] = first ? v : dwcat[i] + v;
  }
  if (dB && i < H) dB[i] = first ? gb[i] : dB[i] + gb[i];
}

// The same sum four elements per thread (16-byte fp32 accesses, 8- or 16-byte
// loads of tmpw): nw % 4 == 0 and 16-byte aligned dwcat and tmpw.
template <typename T>
__global__ void __launch_bounds__(256) rnn_acc4_kernel(float* __restrict__ dwcat, const T* __restrict__ tmpw,
                                                       int64_t nw4, float* __restrict__ dB,
                                                       const float* __restrict__ gb, int H, int first) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nw4) {
    f4 v;
    if constexpr (sizeof(T) == 4) {
      v = reinterpret_cast<const f4*>(tmpw)[i];
    } else {
      const uint2 raw = reinterpret_cast<const uint2*>(tmpw)[i];
      const T* e = reinterpret_cast<const T*>(&raw);
      v = f4{Elem<T>::load1(e), Elem<T>::load1(e + 1), Elem<T>::load1(e + 2), Elem<T>::load1(e + 3)};
    }
    f4* w = reinterpret_cast<f4*>(dwcat) + i;
    *w = first ? v : *w + v;
  }
  if (dB && i < H) dB[i] = first ? gb[i] : dB[i] + gb[i];
}

// After step 0: dX[n, 0, :] = dxh[n, :I]; dh0 = dxh[n, I:]; dWx / dWh = dwcat
// split and converted to the tensor dtype.
template <typename T>
__global__ void __launch_bounds__(256) rnn_bwd_finish_kernel(const T* __restrict__ dxh, const float* __restrict__ dwcat,
                                                             T* __restrict__ dX, T* __restrict__ dh0,
                                                             T* __restrict__ dWx, T* __restrict__ dWh, RnnDims d) {
  const int IH = d.I + d.H;
  const int64_t nx = (int64_t)d.N * IH, nw = (int64_t)IH * d.H;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx < nx) {
    const int n = static_cast<int>(idx / IH), j = static_cast<int>(idx - (int64_t)n * IH);
    if (j < d.I) {
      if (dX) dX[(int64_t)n * d.T * d.I + j] = dxh[idx];
    } else if (dh0) {
      dh0[(int64_t)n * d.H + (j - d.I)] = dxh[idx];
    }
  } else if (idx < nx + nw) {
    const int64_t w = idx - nx;
    const int64_t split = (int64_t)d.I * d.H;
    if (w < split) {
      if (dWx) Elem<T>::store1(dWx + w, dwcat[w]);
    } else if (dWh) {
      Elem<T>::store1(dWh + (w - split), dwcat[w]);
    }
  }
}

// T == 0: the gradients are zero (the reference zero-fills them first).
template <typename T>
__global__ void __launch_bounds__(256) rnn_zero_kernel(T* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = T{};
}

inline unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

template <typename T>
hipError_t launch_fwd_gather(const void* X, const void* hprev, int64_t ldh, void* xh, const RnnDims& d, int t,
                             hipStream_t s) {
  hipLaunchKernelGGL((rnn_fwd_gather_kernel<T>), dim3(blocks_for((int64_t)d.N * (d.I + d.H))), dim3(256), 0, s,
                     static_cast<const T*>(X), static_cast<const T*>(hprev), ldh, static_cast<T*>(xh), d, t);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd_gather(const void* X, const void* Z, const void* h0, const void* dY, const void* dxh, void* xh,
                             void* g, void* dX, const RnnDims& d, int t, int act, float slope, hipStream_t s) {
  hipLaunchKernelGGL((rnn_bwd_gather_kernel<T>), dim3(blocks_for((int64_t)d.N * (d.I + d.H))), dim3(256), 0, s,
                     static_cast<const T*>(X), static_cast<const T*>(Z), static_cast<const T*>(h0),
                     static_cast<const T*>(dY), static_cast<const T*>(dxh), static_cast<T*>(xh), static_cast<T*>(g),
                     static_cast<T*>(dX), d, t, act, slope);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_acc(float* dwcat, const void* tmpw, int64_t nw, float* dB, const float* gb, int H, bool first,
                      hipStream_t s) {
  if (nw % 4 == 0 && (reinterpret_cast<uintptr_t>(dwcat) & 15) == 0 && (reinterpret_cast<uintptr_t>(tmpw) & 15) == 0) {
    hipLaunchKernelGGL((rnn_acc4_kernel<T>), dim3(blocks_for(std::max<int64_t>(nw / 4, H))), dim3(256), 0, s, dwcat,
                       static_cast<const T*>(tmpw), nw / 4, dB, gb, H, first ? 1 : 0);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((rnn_acc_kernel<T>), dim3(blocks_for(std::max<int64_t>(nw, H))), dim3(256), 0, s, dwcat,
                     static_cast<const T*>(tmpw), nw, dB, gb, H, first ? 1 : 0);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd_gather_g(const void* Z, const void* dY, const void* dxh, void* gall, void* dX,
                               const RnnDims& d, int t, int act, float slope, hipStream_t s) {
  hipLaunchKernelGGL((rnn_bwd_gather_g_kernel<T>), dim3(blocks_for((int64_t)d.N * (d.I + d.H))), dim3(256), 0, s,
                     static_cast<const T*>(Z), static_cast<const T*>(dY), static_cast<const T*>(dxh),
                     static_cast<T*>(gall), static_cast<T*>(dX), d, t, act, slope);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_step_nt(const SkinnyNtArgs& a, const void* dY, const void* Z, void* gall, void* dX,
                          const RnnDims& d, int t, int act, float slope, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.K + 3) / 4));
  if (a.M <= 8)
    hipLaunchKernelGGL((rnn_step_nt_kernel<T, 8>), grid, dim3(256), 0, s, a, static_cast<const T*>(dY),
                       static_cast<const T*>(Z), static_cast<T*>(gall), static_cast<T*>(dX), d, t, act, slope);
  else
    hipLaunchKernelGGL((rnn_step_nt_kernel<T, 16>), grid, dim3(256), 0, s, a, static_cast<const T*>(dY),
                       static_cast<const T*>(Z), static_cast<T*>(gall), static_cast<T*>(dX), d, t, act, slope);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_hprev(const void* Z, const void* h0, void* hprev, const RnnDims& d, int act, float slope,
                        hipStream_t s) {
  hipLaunchKernelGGL((rnn_hprev_kernel<T>), dim3(blocks_for((int64_t)d.N * d.T * d.H)), dim3(256), 0, s,
                     static_cast<const T*>(Z), static_cast<const T*>(h0), static_cast<T*>(hprev), d, act, slope);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_colsum(const void* g, int64_t rows, int H, float* dB, hipStream_t s) {
  hipLaunchKernelGGL((rnn_colsum_kernel<T>), dim3((H + 255) / 256), dim3(256), 0, s, static_cast<const T*>(g),
                     rows, H, dB);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd_finish(const void* dxh, const float* dwcat, void* dX, void* dh0, void* dWx, void* dWh,
                             const RnnDims& d, hipStream_t s) {
  const int64_t n = (int64_t)d.N * (d.I + d.H) + (int64_t)(d.I + d.H) * d.H;
  hipLaunchKernelGGL((rnn_bwd_finish_kernel<T>), dim3(blocks_for(n)), dim3(256), 0, s, static_cast<const T*>(dxh),
                     dwcat, static_cast<T*>(dX), static_cast<T*>(dh0), static_cast<T*>(dWx), static_cast<T*>(dWh), d);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_zero(void* p, int64_t n, hipStream_t s) {
  if (!p || n == 0) return hipSuccess;
  hipLaunchKernelGGL((rnn_zero_kernel<T>), dim3(blocks_for(n)), dim3(256), 0, s, static_cast<T*>(p), n);
  return hipGetLastError();
}

#define GEV2_RNN_DISPATCH(dtype, F, ...)                          \
  ((dtype) == GEV2_F32 ? F<float>(__VA_ARGS__)                    \
   : (dtype) == GEV2_BF16 ? F<__bf16>(__VA_ARGS__)                \
                          : F<_Float16>(__VA_ARGS__))

}  // namespace gev2

namespace {

thread_local std::string t_rnn_error;

int rnn_fail(int st, const char* msg) {
  t_rnn_error = msg;
  return st;
}

int64_t esize(int dtype) { return dtype == GEV2_F32 ? 4 : 2; }

template <typename D>
int rnn_check(const D* d) {
  if (!d) return rnn_fail(GEV2_INVALID_ARGUMENT, "null descriptor");
  if (d->dtype != GEV2_F32 && d->dtype != GEV2_F16 && d->dtype != GEV2_BF16)
    return rnn_fail(GEV2_DTYPE_MISMATCH, "dtype must be F32, F16 or BF16");
  if (d->act < GEV2_ACT_NONE || d->act > GEV2_ACT_TANH) return rnn_fail(GEV2_INVALID_ARGUMENT, "bad act kind");
  if (d->N <= 0 || d->T < 0 || d->I <= 0 || d->H <= 0)
    return rnn_fail(GEV2_INVALID, "N, I, H must be positive and T non-negative");
  if ((int64_t)d->N * d->T * std::max(d->I, d->H) > 0x7fffffffLL ||
      (int64_t)d->N * (d->I + d->H) > 0x7fffffffLL || (int64_t)(d->I + d->H) * d->H > 0x7fffffffLL)
    return rnn_fail(GEV2_INVALID, "sizes must fit int32");
  return GEV2_OK;
}

// 16-byte vector rows whose byte offsets from the base stay below 2^31 (the
// split kernel's 32-bit buffer offsets).
bool rows16(const void* p, int64_t ld, int64_t rows, int64_t cols, int64_t es) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (ld * es) % 16 == 0 && (cols * es) % 16 == 0 &&
         ((rows - 1) * ld + cols) * es <= 0x7fffff00LL;
}

// The skinny split kernel reads XH = [X_t | h_{t-1}] from its two places, so
// a step needs no gather launch, when: 16-bit data, N <= 16, I a whole number
// of the kernel's 256-row K blocks, 16-byte rows of X, h0, Y and wcat within
// 2^31 bytes, and the caller's 256-byte aligned workspace holds the partials.
// Otherwise a step gathers XH and calls the operator.
bool rnn_fwd_two_part(const gev2_rnn_desc* d) {
  if (d->dtype == GEV2_F32 || d->N > gev2::kSkinnyMaxM || d->I % 256 != 0 || d->H % 8 != 0) return false;
  if (std::getenv("GEV2_RNN_GATHER") || std::getenv("GEV2_NO_SKINNY")) return false;
  const int64_t es = 2, T = d->T, IH = d->I + d->H;
  if (!rows16(d->X, T * d->I, d->N, T * d->I, es) || !rows16(d->h0, d->H, d->N, d->H, es) ||
      !rows16(d->Y, T * d->H, d->N, T * d->H, es) || !rows16(d->wcat, d->H, IH, d->H, es))
    return false;
  const int64_t need = gev2::skinny_split_workspace_bytes(d->N, d->H, static_cast<int>(IH));
  return d->ws && (reinterpret_cast<uintptr_t>(d->ws) & 255) == 0 && d->ws_bytes >= need;
}

// The backward's gathered-G' form: G' of every step is kept in an [N, T, H]
// buffer (tmpw), and a step is one kernel (rnn_step_nt_kernel: dXH_t = G'_t
// Wcat^T, each column turned at once into dX_t or G'_{t-1}); after the loop
// dWx = X^T G' and dWh = Hprev^T G' are one operator forward each (depth N*T,
// one rounding), Hprev staged in dwcat, and dB is a column sum of G'.  Needs N <= 16, 16-byte rows of G' and wcat, and N*T <= I+H (so
// that G' fits tmpw and Hprev fits dwcat).  GEV2_RNN_STEP_DW=1 keeps the
// per-step form (one operator backward and one accumulation per step).
bool rnn_bwd_gathered(const gev2_rnn_bwd_desc* d) {
  const int64_t es = esize(d->dtype);
  if (d->N > gev2::kSkinnyMaxM || (int64_t)d->N * d->T > (int64_t)d->I + d->H || (d->H * es) % 16 != 0) return false;
  if (std::getenv("GEV2_RNN_STEP_DW")) return false;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return al(d->tmpw) && al(d->wcat) && al(d->dwcat);
}

// dW = A^T G' over the N*T rows (A: X or the staged Hprev), as an operator forward
gev2_gemm_fwd_desc rnn_wgrad_desc(const gev2_rnn_bwd_desc* d, const void* A, int64_t lda, int M, void* out) {
  gev2_gemm_fwd_desc f{};
  f.dtype = d->dtype; f.act = GEV2_ACT_NONE; f.alpha = 1.f; f.bias_kind = GEV2_BIAS_NONE;
  f.M = M; f.N = d->H; f.K = (int64_t)d->N * d->T; f.batch = 1;
  f.A = A; f.lda = lda; f.trans_a = 1;
  f.B = d->tmpw; f.ldb = d->H;
  f.Y = out; f.ldy = d->H;
  f.workspace = d->ws; f.workspace_bytes = d->ws_bytes;
  return f;
}

// fp32: the one-launch small kernel takes XH = [X_t | h_{t-1}] as a two-part
// operand (no gather) within its limits (at most 512 16x16 output tiles, a
// reduction I+H of 128-2048, 2^26 multiply-adds) and with I a multiple of 4.
bool rnn_fwd_small_two_part(const gev2_rnn_desc* d) {
  const int64_t IH = (int64_t)d->I + d->H;
  if (d->dtype != GEV2_F32 || d->I % 4 != 0 || std::getenv("GEV2_RNN_GATHER") || std::getenv("GEV2_NO_SMALL"))
    return false;
  const int64_t tiles = ((int64_t)(d->N + 15) / 16) * ((d->H + 15) / 16);
  return tiles <= 512 && IH >= 128 && IH <= 2048 && static_cast<double>(d->N) * d->H * IH <= 67108864.0;
}

int gemm_status(int st) {
  if (st != GEV2_OK) t_rnn_error = std::string("gemm: ") + gev2_last_error();
  return st;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return GEV2_OK;
  t_rnn_error = std::string(where) + ": " + hipGetErrorString(e);
  return GEV2_HIP_ERROR;
}

// The step loops are T serial launches of small kernels, which the launch rate
// bounds.  On a created stream each distinct (descriptor, stream) is run
// eagerly the first time (which also creates the operator's per-stream
// scratch), recorded into a HIP graph the second time, and replayed from then
// on.  A replay reads the buffers the descriptor names, as they are at launch.
// GEV2_RNN_GRAPH=0 turns this off.  At most kMaxGraphs executables are kept.
constexpr size_t kMaxGraphs = 32;

struct GraphCache {
  std::mutex mu;
  std::set<std::string> seen;
  std::list<std::pair<std::string, hipGraphExec_t>> lru;   // most recent first
};

GraphCache& graph_cache() {
  static GraphCache* c = new GraphCache();   // kept until exit (executables are per process)
  return *c;
}

bool graphs_on() {
  static const bool on = [] {
    const char* v = std::getenv("GEV2_RNN_GRAPH");
    return !(v && v[0] == '0');
  }();
  return on;
}

// `graph_ok`: every operator call of the loop runs on the descriptor's own
// scratch (or needs none), so a recorded graph names no per-stream buffer
// that a later call on the stream could reallocate.
template <typename Desc, typename Fn>
int run_cached(const Desc* d, char dir, hipStream_t s, bool graph_ok, Fn&& work) {
  if (!s || !graph_ok || !graphs_on()) return work();
  std::string key(1, dir);
  key.append(reinterpret_cast<const char*>(d), sizeof(Desc));
  key.append(reinterpret_cast<const char*>(&s), sizeof(s));
  GraphCache& c = graph_cache();
  bool first = false;
  {
    std::lock_guard<std::mutex> lk(c.mu);
    for (auto it = c.lru.begin(); it != c.lru.end(); ++it) {
      if (it->first == key) {
        c.lru.splice(c.lru.begin(), c.lru, it);
        return hip_status(hipGraphLaunch(it->second, s), "rnn graph launch");
      }
    }
    first = c.seen.insert(key).second;
    if (first && c.seen.size() > 4 * kMaxGraphs) {
      c.seen.clear();
      c.seen.insert(key);
    }
  }
  if (first) return work();                  // first sighting: eager
  {
    int st = hip_status(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "rnn graph capture");
    if (st != GEV2_OK) return st;
    st = work();
    hipGraph_t g = nullptr;
    const hipError_t ee = hipStreamEndCapture(s, &g);
    if (st != GEV2_OK || ee != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      return st != GEV2_OK ? st : hip_status(ee, "rnn graph capture");
    }
    hipGraphExec_t ex = nullptr;
    const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) return hip_status(ie, "rnn graph instantiate");
    std::lock_guard<std::mutex> lk(c.mu);
    c.lru.emplace_front(key, ex);
    if (c.lru.size() > kMaxGraphs) {
      (void)hipGraphExecDestroy(c.lru.back().second);
      c.lru.pop_back();
    }
    return hip_status(hipGraphLaunch(ex, s), "rnn graph launch");
  }
}

}  // namespace

extern "C" {

const char* gev2_rnn_last_error(void) { return t_rnn_error.c_str(); }

int gev2_rnn_fwd(const gev2_rnn_desc* d, void* stream) {
  t_rnn_error.clear();
  int st = rnn_check(d);
  if (st != GEV2_OK) return st;
  if (!d->X || !d->Wx || !d->Wh || !d->h0) return rnn_fail(GEV2_MISSING_INPUT, "X / Wx / Wh / h0 is null");
  if (!d->Y) return rnn_fail(GEV2_MISSING_OUTPUT, "Y is null");
  if (d->save_z && !d->Z) return rnn_fail(GEV2_MISSING_OUTPUT, "save_z requires Z");
  if (d->save_z && d->Z == d->Y) return rnn_fail(GEV2_INVALID, "Z must not alias Y");
  if (!d->xh || !d->wcat) return rnn_fail(GEV2_MISSING_INPUT, "xh and wcat workspaces are required");
  const gev2::RnnDims dm{d->N, d->T, d->I, d->H};
  const int64_t es = esize(d->dtype), IH = d->I + d->H;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  bool graph_ok;
  {
    gev2_gemm_fwd_desc f{};
    f.dtype = d->dtype; f.act = d->act; f.alpha = 1.f; f.bias_kind = d->bias ? GEV2_BIAS_PER_N : GEV2_BIAS_NONE;
    f.M = d->N; f.N = d->H; f.K = IH; f.batch = 1;
    f.A = d->xh; f.lda = IH; f.B = d->wcat; f.ldb = d->H; f.bias = d->bias;
    f.Y = d->Y; f.ldy = (int64_t)d->T * d->H;
    const int64_t need = gev2_gemm_fwd_workspace_size(&f);
    // the operator takes the caller's workspace only when it is 256-byte aligned
    graph_ok = need == 0 || (need > 0 && d->ws && d->ws_bytes >= need &&
                             (reinterpret_cast<uintptr_t>(d->ws) & 255) == 0);
  }
  return run_cached(d, 'f', s, graph_ok, [&]() -> int {
  int st = GEV2_OK;
  // wcat = [Wx ; Wh]  ([I+H, H])
  st = hip_status(hipMemcpyAsync(d->wcat, d->Wx, (size_t)d->I * d->H * es, hipMemcpyDeviceToDevice, s), "pack Wx");
  if (st != GEV2_OK) return st;
  st = hip_status(hipMemcpyAsync(static_cast<char*>(d->wcat) + (size_t)d->I * d->H * es, d->Wh,
                                 (size_t)d->H * d->H * es, hipMemcpyDeviceToDevice, s), "pack Wh");
  if (st != GEV2_OK) return st;
  const int64_t ldy = (int64_t)d->T * d->H;
  const bool two_part = rnn_fwd_two_part(d);
  const bool small_two_part = rnn_fwd_small_two_part(d);
  for (int t = 0; t < d->T; ++t) {
    const void* hprev = t == 0 ? d->h0 : static_cast<const char*>(d->Y) + (size_t)(t - 1) * d->H * es;
    if (small_two_part) {
      gev2::SmallArgs a{};
      gev2::SmallJob& J = a.job[0];
      const float* xt = static_cast<const float*>(d->X) + (size_t)t * d->I;
      const float* hp = static_cast<const float*>(hprev);
      const int64_t ldh = t == 0 ? d->H : ldy;
      J.a.p = xt; J.a.rs = (int64_t)d->T * d->I; J.a.ks = 1;
      J.a.p2 = hp; J.a.rs2 = ldh; J.a.k1 = d->I;
      J.a.vec = J.a.rs % 4 == 0 && ldh % 4 == 0 && (reinterpret_cast<uintptr_t>(xt) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(hp) & 15) == 0;
      J.b.p = static_cast<const float*>(d->wcat); J.b.rs = 1; J.b.ks = d->H;
      J.kind = 0;
      J.rows = d->N; J.cols = d->H; J.red = static_cast<int>(IH);
      J.tiles_c = (d->H + 15) / 16;
      J.tiles = ((d->N + 15) / 16) * J.tiles_c;
      J.wgs = J.tiles;
      J.scale = 1.f;
      J.out = static_cast<float*>(d->Y) + (size_t)t * d->H; J.ldo = ldy;
      a.njobs = 1; a.fwd = 1;
      a.act = d->act; a.slope = d->leaky_slope;
      a.bias = d->bias; a.bias_kind = d->bias ? GEV2_BIAS_PER_N : GEV2_BIAS_NONE;
      a.Z = d->save_z ? static_cast<float*>(d->Z) + (size_t)t * d->H : nullptr; a.ldz = ldy;
      st = hip_status(gev2::launch_small(a, gev2::small_waves_for(IH), s), "small step");
      if (st != GEV2_OK) return st;
      continue;
    }
    if (two_part) {
      gev2::SkinnyArgs a{};
      a.A = static_cast<const char*>(d->X) + (size_t)t * d->I * es; a.lda = (int64_t)d->T * d->I;
      a.A2 = hprev; a.lda2 = t == 0 ? d->H : ldy; a.K1 = d->I;
      a.B = d->wcat; a.ldb = d->H;
      a.D = static_cast<char*>(d->Y) + (size_t)t * d->H * es; a.ldd = ldy;
      a.Zo = d->save_z ? static_cast<char*>(d->Z) + (size_t)t * d->H * es : nullptr; a.ldzo = ldy;
      a.bias = d->bias; a.bias_kind = d->bias ? GEV2_BIAS_PER_N : GEV2_BIAS_NONE;
      a.M = d->N; a.N = d->H; a.K = static_cast<int>(IH);
      a.act = d->act; a.slope = d->leaky_slope; a.alpha = 1.f;
      a.x_vec = 2;
      st = hip_status(gev2::launch_skinny(d->dtype, a, static_cast<float*>(d->ws), s), "skinny step");
      if (st != GEV2_OK) return st;
      continue;
    }
    st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_fwd_gather, d->X, hprev, t == 0 ? d->H : ldy, d->xh,
                                      dm, t, s), "gather");
    if (st != GEV2_OK) return st;
    gev2_gemm_fwd_desc f{};
    f.dtype = d->dtype; f.act = d->act; f.leaky_slope = d->leaky_slope; f.alpha = 1.f;
    f.bias_kind = d->bias ? GEV2_BIAS_PER_N : GEV2_BIAS_NONE;
    f.M = d->N; f.N = d->H; f.K = IH; f.batch = 1;
    f.A = d->xh; f.lda = IH;
    f.B = d->wcat; f.ldb = d->H;
    f.bias = d->bias;
    f.Y = static_cast<char*>(d->Y) + (size_t)t * d->H * es; f.ldy = ldy;
    if (d->save_z) { f.Z = static_cast<char*>(d->Z) + (size_t)t * d->H * es; f.ldz = ldy; }
    f.workspace = d->ws; f.workspace_bytes = d->ws_bytes;
    st = gemm_status(gev2_gemm_fwd(&f, stream));
    if (st != GEV2_OK) return st;
  }
  return GEV2_OK;
  });
}

int gev2_rnn_bwd(const gev2_rnn_bwd_desc* d, void* stream) {
  t_rnn_error.clear();
  int st = rnn_check(d);
  if (st != GEV2_OK) return st;
  if (!d->X || !d->Wx || !d->Wh || !d->h0 || !d->dY || !d->Z)
    return rnn_fail(GEV2_MISSING_INPUT, "X / Wx / Wh / h0 / dY / Z is null");
  if (!d->xh || !d->g || !d->wcat || !d->dxh || !d->dwcat || !d->tmpw || !d->gb)
    return rnn_fail(GEV2_MISSING_INPUT, "workspaces xh, g, wcat, dxh, dwcat, tmpw and gb are required");
  const gev2::RnnDims dm{d->N, d->T, d->I, d->H};
  const int64_t es = esize(d->dtype), IH = d->I + d->H;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (d->T == 0) {
    // no steps: every gradient is zero
    st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_zero, d->dWx, (int64_t)d->I * d->H, s), "zero");
    if (st == GEV2_OK) st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_zero, d->dWh, (int64_t)d->H * d->H, s), "zero");
    if (st == GEV2_OK) st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_zero, d->dh0, (int64_t)d->N * d->H, s), "zero");
    if (st == GEV2_OK) st = hip_status(gev2::launch_zero<float>(d->dB, d->H, s), "zero");
    return st;
  }
  bool graph_ok;
  if (rnn_bwd_gathered(d)) {
    // the weight-gradient GEMMs must run with the descriptor's scratch (or none)
    // when recorded, as they do eagerly
    auto fits = [&](const gev2_gemm_fwd_desc& f) {
      if (!f.Y) return true;                     // that gradient is not requested
      const int64_t need = gev2_gemm_fwd_workspace_size(&f);
      return need == 0 || (need > 0 && d->ws && d->ws_bytes >= need && (reinterpret_cast<uintptr_t>(d->ws) & 255) == 0);
    };
    graph_ok = fits(rnn_wgrad_desc(d, d->X, d->I, d->I, d->dWx)) && fits(rnn_wgrad_desc(d, d->dwcat, d->H, d->H, d->dWh));
  } else {
    gev2_gemm_bwd_desc b{};
    b.dtype = d->dtype; b.act = d->act; b.alpha = 1.f; b.bias_kind = d->dB ? GEV2_BIAS_PER_N : GEV2_BIAS_NONE;
    b.M = d->N; b.N = d->H; b.K = IH; b.batch = 1;
    b.A = d->xh; b.lda = IH; b.B = d->wcat; b.ldb = d->H; b.gY = d->g; b.ldgy = d->H;
    b.Z = d->Z; b.ldz = (int64_t)d->T * d->H;
    b.gA = d->dxh; b.ldga = IH; b.gB = (d->dWx || d->dWh) ? d->tmpw : nullptr; b.ldgb = d->H;
    b.gBias = d->dB ? d->gb : nullptr;
    const int64_t need = gev2_gemm_bwd_workspace_size(&b);
    // every step's Z slice (Z + t*H) must share the alignment the size was computed for
    graph_ok = (d->H * es) % 16 == 0 &&
               (need == 0 || (need > 0 && d->ws && d->ws_bytes >= need &&
                              (reinterpret_cast<uintptr_t>(d->ws) & 255) == 0));
  }
  return run_cached(d, 'b', s, graph_ok, [&]() -> int {
  int st = GEV2_OK;
  st = hip_status(hipMemcpyAsync(d->wcat, d->Wx, (size_t)d->I * d->H * es, hipMemcpyDeviceToDevice, s), "pack Wx");
  if (st != GEV2_OK) return st;
  st = hip_status(hipMemcpyAsync(static_cast<char*>(d->wcat) + (size_t)d->I * d->H * es, d->Wh,
                                 (size_t)d->H * d->H * es, hipMemcpyDeviceToDevice, s), "pack Wh");
  if (st != GEV2_OK) return st;
  const int64_t ldz = (int64_t)d->T * d->H;
  const bool want_w = d->dWx || d->dWh;
  if (rnn_bwd_gathered(d)) {
    // G'_{T-1} from dY alone; then one kernel per step t >= 1 (dX_t and
    // G'_{t-1} from dXH_t); step 0's dXH goes to dxh for dX_0 and dh0
    st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_bwd_gather_g, d->Z, d->dY, d->dxh, d->tmpw, d->dX, dm,
                                      d->T - 1, d->act, d->leaky_slope, s), "gather G'");
    if (st != GEV2_OK) return st;
    for (int t = d->T - 1; t >= 0; --t) {
      gev2::SkinnyNtArgs a{};
      a.G = static_cast<const char*>(d->tmpw) + (size_t)t * d->H * es; a.ldg = ldz;
      a.Z = nullptr; a.ldz = 0;
      a.B = d->wcat; a.ldb = d->H;
      a.D = d->dxh; a.ldd = IH;
      a.M = d->N; a.N = d->H; a.K = static_cast<int>(IH);
      a.act = GEV2_ACT_NONE; a.slope = 0.f; a.alpha = 1.f;
      if (t > 0)
        st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_step_nt, a, d->dY, d->Z, d->tmpw, d->dX, dm, t,
                                          d->act, d->leaky_slope, s), "step");
      else
        st = hip_status(gev2::launch_skinny_nt(d->dtype, a, s), "dXH");
      if (st != GEV2_OK) return st;
    }
    const int64_t rows = (int64_t)d->N * d->T;
    auto wgrad = [&](const void* A, int64_t lda, int M, void* out) -> int {
      const gev2_gemm_fwd_desc f = rnn_wgrad_desc(d, A, lda, M, out);
      return gemm_status(gev2_gemm_fwd(&f, stream));
    };
    if (d->dWx) {
      st = wgrad(d->X, d->I, d->I, d->dWx);
      if (st != GEV2_OK) return st;
    }
    if (d->dWh) {
      st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_hprev, d->Z, d->h0, d->dwcat, dm, d->act,
                                        d->leaky_slope, s), "hprev");
      if (st == GEV2_OK) st = wgrad(d->dwcat, d->H, d->H, d->dWh);
      if (st != GEV2_OK) return st;
    }
    if (d->dB) {
      st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_colsum, d->tmpw, rows, d->H, d->dB, s), "dB");
      if (st != GEV2_OK) return st;
    }
    return hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_bwd_finish, d->dxh, d->dwcat, d->dX, d->dh0,
                                        nullptr, nullptr, dm, s), "finish");
  }
  for (int t = d->T - 1; t >= 0; --t) {
    st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_bwd_gather, d->X, d->Z, d->h0, d->dY, d->dxh, d->xh,
                                      d->g, d->dX, dm, t, d->act, d->leaky_slope, s), "gather");
    if (st != GEV2_OK) return st;
    gev2_gemm_bwd_desc b{};
    b.dtype = d->dtype; b.act = d->act; b.leaky_slope = d->leaky_slope; b.alpha = 1.f; b.beta = 0.f;
    b.bias_kind = d->dB ? GEV2_BIAS_PER_N : GEV2_BIAS_NONE;
    b.M = d->N; b.N = d->H; b.K = IH; b.batch = 1;
    b.A = d->xh; b.lda = IH;
    b.B = d->wcat; b.ldb = d->H;
    b.gY = d->g; b.ldgy = d->H;
    b.Z = static_cast<const char*>(d->Z) + (size_t)t * d->H * es; b.ldz = ldz;
    b.gA = d->dxh; b.ldga = IH;
    if (want_w) { b.gB = d->tmpw; b.ldgb = d->H; }
    b.gBias = d->dB ? d->gb : nullptr;
    b.workspace = d->ws; b.workspace_bytes = d->ws_bytes;
    st = gemm_status(gev2_gemm_bwd(&b, stream));
    if (st != GEV2_OK) return st;
    if (want_w || d->dB) {
      st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_acc, d->dwcat, d->tmpw, want_w ? IH * d->H : 0, d->dB,
                                        d->gb, d->H, t == d->T - 1, s), "accumulate");
      if (st != GEV2_OK) return st;
    }
  }
  st = hip_status(GEV2_RNN_DISPATCH(d->dtype, gev2::launch_bwd_finish, d->dxh, d->dwcat, d->dX, d->dh0, d->dWx,
                                    d->dWh, dm, s), "finish");
  return st;
  });
}

}  // extern "C"
