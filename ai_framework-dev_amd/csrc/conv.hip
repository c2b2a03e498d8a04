// 2-D convolution (NCHW, groups = 1) on the batched GEMM: the conv2d launcher
// of graph_executor_v2 (backends/cuda/ops/conv2d/launcher.cu:106-459,
// kernels.cu:12-175) rebuilt around the operator.
//
// Forward, per chunk of images:
//   im2col into Col^T [K, Ho*Wo] per image, K = Cin*Kh*Kw ordered
//   (c*Kh + kh)*Kw + kw (kernels.cu:12-45), then ONE batched GEMM
//     Y_n [Cout, Ho*Wo] = W [Cout, K] . Col^T_n  (+ bias per row, act, Z)
//   whose output rows are already the NCHW planes: the OIHW weight tensor is
//   the [Cout, K] operand as it lies in memory, so there is no weight packing
//   and no output transpose (the reference packs W, runs one GEMM per image
//   into [HWo, Cout] rows and transposes each result).
// Backward, per chunk of images (as many as the workspaces hold): im2col,
//   then ONE batched operator backward with A = W (slice stride 0),
//   B = Col^T_n, gY = dY_n, Z = Z_n, giving per image dW_n = dY'_n Col_n (gA),
//   the input-gradient columns W^T dY'_n (gB, [K, HWo]) and dB_n (PerM gBias).
//   dW and dB are summed over images in fp32 in image order, and col2im
//   gathers each input element's columns in a fixed (kh, kw) order, so the
//   results do not depend on the chunk size.  (The reference runs one GEMM
//   backward per image and zero-fills the bias gradient inside each, so its dB
//   holds the last image only.)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <type_traits>

#include "../../include/gev2_gemm.h"
#include "gev2_device.hpp"

namespace gev2 {

struct ConvGeom {
  int Cin, H, W, Kh, Kw, sh, sw, ph, pw, dh, dw, Ho, Wo;
};

// Raw storage word of T: im2col and col2im's scatter-free gather move bits.
template <typename T> struct Word { using type = uint16_t; };
template <> struct Word<float> { using type = uint32_t; };

constexpr int kRun = 8;   // consecutive outputs per thread (one 16-byte store of a 16-bit type)

// Store a thread's run of kRun words at dst: as 16-byte pieces when `vec`
// (the run is whole and 16-byte aligned), else element by element up to n.
template <typename U>
__device__ __forceinline__ void store_run(U* dst, const U (&v)[kRun], int n, bool vec) {
  if (vec && n >= kRun) {
    constexpr int kWords = 16 / sizeof(U);
#pragma unroll
    for (int q = 0; q < kRun / kWords; ++q) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(U) == 2) w[i] = static_cast<uint32_t>(v[q * kWords + 2 * i]) |
                                             (static_cast<uint32_t>(v[q * kWords + 2 * i + 1]) << 16);
        else w[i] = v[q * kWords + i];
      }
      *reinterpret_cast<u32x4*>(dst + q * kWords) = w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kRun; ++j)
      if (j < n) dst[j] = v[j];
  }
}

// col[(img*K + k) * HWo + hw] = X[img][c][ho*sh - ph + kh*dh][wo*sw - pw + kw*dw] (0 outside),
// k = (c*Kh + kh)*Kw + kw, hw = ho*Wo + wo (kernels.cu:12-45).  A thread writes
// kRun consecutive hw of one (img, k) row; its row and window offsets are
// derived once, then ho / wo advance incrementally.
template <typename T>
__global__ void __launch_bounds__(256) im2col_t_kernel(const T* __restrict__ Xt, T* __restrict__ colt, ConvGeom g,
                                                       int runs_per_row, int64_t threads, int vec) {
  using U = typename Word<T>::type;
  const U* __restrict__ X = reinterpret_cast<const U*>(Xt);
  U* __restrict__ col = reinterpret_cast<U*>(colt);
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= threads) return;
  const int HWo = g.Ho * g.Wo;
  const int K = g.Cin * g.Kh * g.Kw;
  const int64_t row = t / runs_per_row;             // img*K + k
  const int hw0 = static_cast<int>(t - row * runs_per_row) * kRun;
  const int img = static_cast<int>(row / K), k = static_cast<int>(row - (int64_t)img * K);
  const int kw = k % g.Kw, kh = (k / g.Kw) % g.Kh, c = k / (g.Kw * g.Kh);
  int ho = hw0 / g.Wo, wo = hw0 - ho * g.Wo;
  const U* __restrict__ xp = X + ((int64_t)img * g.Cin + c) * g.H * g.W;
  const int hoff = kh * g.dh - g.ph, woff = kw * g.dw - g.pw;
  U v[kRun];
#pragma unroll
  for (int j = 0; j < kRun; ++j) {
    const int hi = ho * g.sh + hoff, wi = wo * g.sw + woff;
    const bool in = hw0 + j < HWo && static_cast<unsigned>(hi) < static_cast<unsigned>(g.H) &&
                    static_cast<unsigned>(wi) < static_cast<unsigned>(g.W);
    v[j] = in ? xp[hi * g.W + wi] : U(0);
    if (++wo == g.Wo) { wo = 0; ++ho; }
  }
  store_run(col + row * HWo + hw0, v, HWo - hw0, vec != 0);
}

// The same col through LDS: a workgroup owns one (img, c) input plane and a
// band of TH output rows.  It reads the R = (TH-1)*sh + (Kh-1)*dh + 1 input
// rows the band needs into LDS once (rows outside the image as zeros), then
// writes the Kh*Kw col rows of the band as runs of kRun consecutive hw, so X
// is read from HBM once instead of Kh*Kw times through the caches.
template <typename T, bool WIN>
__global__ void __launch_bounds__(256) im2col_lds_kernel(const T* __restrict__ Xt, T* __restrict__ colt, ConvGeom g,
                                                         int TH, int bands, int vec, int xvec) {
  using U = typename Word<T>::type;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  U* lds = reinterpret_cast<U*>(lds_raw);
  const int band = static_cast<int>(blockIdx.x % bands);
  const int64_t ic = blockIdx.x / bands;            // img*Cin + c
  const int img = static_cast<int>(ic / g.Cin), c = static_cast<int>(ic - (int64_t)img * g.Cin);
  const int ho0 = band * TH;
  const int rows = min(TH, g.Ho - ho0);
  const int R = (rows - 1) * g.sh + (g.Kh - 1) * g.dh + 1;
  const int hbase = ho0 * g.sh - g.ph;
  const U* __restrict__ xp = reinterpret_cast<const U*>(Xt) + ic * g.H * g.W;
  if (xvec) {
    // rows are whole 16-byte chunks (and the plane starts on one): copy chunks
    constexpr int kWords = 16 / sizeof(U);
    const int cpr = g.W / kWords, chunks = R * cpr;
#pragma unroll 4
    for (int i = threadIdx.x; i < chunks; i += 256) {
      const int r = i / cpr;
      const int hi = hbase + r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (static_cast<unsigned>(hi) < static_cast<unsigned>(g.H))
        v = *reinterpret_cast<const u32x4*>(xp + (int64_t)hi * g.W + (i - r * cpr) * kWords);
      *reinterpret_cast<u32x4*>(lds + i * kWords) = v;
    }
  } else {
#pragma unroll 8
    for (int i = threadIdx.x; i < R * g.W; i += 256) {
      const int r = i / g.W;
      const int hi = hbase + r;
      lds[i] = static_cast<unsigned>(hi) < static_cast<unsigned>(g.H) ? xp[hi * g.W + (i - r * g.W)] : U(0);
    }
  }
  __syncthreads();
  const int KK = g.Kh * g.Kw, HWo = g.Ho * g.Wo, K = g.Cin * KK;
  const int n_out = rows * g.Wo;
  const int runs = (n_out + kRun - 1) / kRun;
  U* __restrict__ col = reinterpret_cast<U*>(colt) + ((int64_t)img * K + (int64_t)c * KK) * HWo + ho0 * g.Wo;
  if constexpr (WIN) {
    // unit horizontal stride, Wo a multiple of kRun, 16-byte LDS rows: a run's
    // kRun inputs are consecutive in one LDS row, read as the aligned chunks
    // that cover them and shifted into place (chunks past either end of the
    // band are clamped into it; they only feed masked positions)
    constexpr int EPC = 16 / sizeof(U), EW = 4 / sizeof(U);
    constexpr int NCH = kRun / EPC + 1, NWD = 4 * NCH, OUTW = kRun / EW;
    const int lds_chunks = R * g.W / EPC;
    const int rpr = g.Wo / kRun;                   // runs per output row
    for (int run = threadIdx.x; run < KK * runs; run += 256) {
      const int kidx = run / runs;
      const int r0 = run - kidx * runs;
      const int kh = kidx / g.Kw, kw = kidx - kh * g.Kw;
      const int hl = r0 / rpr, wo0 = (r0 - hl * rpr) * kRun;
      const int wi0 = wo0 + kw * g.dw - g.pw;
      const int a = (hl * g.sh + kh * g.dh) * g.W + wi0;
      const int c0 = (a >= 0 ? a : a - (EPC - 1)) / EPC;
      const int sh = a - c0 * EPC;
      uint32_t wd[NWD];
#pragma unroll
      for (int q = 0; q < NCH; ++q) {
        const int ci = min(max(c0 + q, 0), lds_chunks - 1);
        const u32x4 v = *reinterpret_cast<const u32x4*>(lds + ci * EPC);
#pragma unroll
        for (int i = 0; i < 4; ++i) wd[4 * q + i] = v[i];
      }
      const int bw = sh / EW;
      if (bw & 1) {
#pragma unroll
        for (int i = 0; i + 1 < NWD; ++i) wd[i] = wd[i + 1];
      }
      if (bw & 2) {
#pragma unroll
        for (int i = 0; i + 2 < NWD; ++i) wd[i] = wd[i + 2];
      }
      U v[kRun];
#pragma unroll
      for (int q = 0; q < OUTW; ++q) {
        uint32_t w;
        if constexpr (EW == 2) w = (sh & 1) ? __builtin_amdgcn_alignbit(wd[q + 1], wd[q], 16) : wd[q];
        else w = wd[q];
#pragma unroll
        for (int e = 0; e < EW; ++e) {
          const int j = q * EW + e;
          const bool in = static_cast<unsigned>(wi0 + j) < static_cast<unsigned>(g.W);
          v[j] = in ? static_cast<U>(EW == 2 ? (w >> (16 * e)) & 0xffffu : w) : U(0);
        }
      }
      store_run(col + (int64_t)kidx * HWo + hl * g.Wo + wo0, v, kRun, vec != 0);
    }
    return;
  }
  for (int run = threadIdx.x; run < KK * runs; run += 256) {
    const int kidx = run / runs;
    const int o0 = (run - kidx * runs) * kRun;
    const int kh = kidx / g.Kw, kw = kidx - kh * g.Kw;
    int hl = o0 / g.Wo, wo = o0 - hl * g.Wo;
    const int woff = kw * g.dw - g.pw;
    U v[kRun];
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const int wi = wo * g.sw + woff;
      const bool in = o0 + j < n_out && static_cast<unsigned>(wi) < static_cast<unsigned>(g.W);
      v[j] = in ? lds[(hl * g.sh + kh * g.dh) * g.W + wi] : U(0);
      if (++wo == g.Wo) { wo = 0; ++hl; }
    }
    store_run(col + (int64_t)kidx * HWo + o0, v, n_out - o0, vec != 0);
  }
}

// dX[img][c][h][w] = sum over (kh, kw), in that order, of dcol[k][ho*Wo + wo]
// for the output positions whose window covers (h, w) (kernels.cu:50-87, as a
// gather: no atomics, a fixed summation order).  A thread computes kRun
// consecutive w of one (img, c, h) row; the kh terms are shared by the run.
template <typename T>
__global__ void __launch_bounds__(256) col2im_t_kernel(const T* __restrict__ dcol, T* __restrict__ dXt, ConvGeom g,
                                                       int runs_per_row, int64_t threads, int vec) {
  using U = typename Word<T>::type;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= threads) return;
  const int64_t row = t / runs_per_row;             // (img*Cin + c)*H + h
  const int w0 = static_cast<int>(t - row * runs_per_row) * kRun;
  const int h = static_cast<int>(row % g.H);
  const int64_t ic = row / g.H;                     // img*Cin + c
  const int img = static_cast<int>(ic / g.Cin), c = static_cast<int>(ic - (int64_t)img * g.Cin);
  const int HWo = g.Ho * g.Wo;
  const int K = g.Cin * g.Kh * g.Kw;
  const T* __restrict__ base = dcol + ((int64_t)img * K + (int64_t)c * g.Kh * g.Kw) * HWo;
  float acc[kRun];
#pragma unroll
  for (int j = 0; j < kRun; ++j) acc[j] = 0.f;
  for (int kh = 0; kh < g.Kh; ++kh) {
    const int hn = h + g.ph - kh * g.dh;
    if (hn < 0) break;                              // hn only falls as kh grows
    const int ho = hn / g.sh;
    if (ho * g.sh != hn || ho >= g.Ho) continue;
    const T* __restrict__ rowp = base + (int64_t)kh * g.Kw * HWo + ho * g.Wo;
    for (int kw = 0; kw < g.Kw; ++kw) {
      const T* __restrict__ p = rowp + (int64_t)kw * HWo;
#pragma unroll
      for (int j = 0; j < kRun; ++j) {
        const int wn = w0 + j + g.pw - kw * g.dw;
        const int wo = wn / g.sw;
        if (w0 + j < g.W && wn >= 0 && wo * g.sw == wn && wo < g.Wo) acc[j] += Elem<T>::load1(p + wo);
      }
    }
  }
  U v[kRun];
#pragma unroll
  for (int j = 0; j < kRun; ++j) v[j] = static_cast<U>(Elem<T>::bits(acc[j]));
  store_run(reinterpret_cast<U*>(dXt) + row * g.W + w0, v, g.W - w0, vec != 0);
}

// col2im_t for unit horizontal stride with 16-byte aligned dcol rows (HWo a
// multiple of the chunk): a thread's kRun outputs read kRun consecutive
// elements of each contributing dcol row, at an offset that is not chunk
// aligned.  The thread loads the aligned 16-byte chunks that cover that window
// and shifts it into place in registers, instead of kRun element loads.
// Chunks that would lie outside the dcol row are clamped into it: they can
// only hold elements whose output position is masked.  Sums are formed in the
// same (kh, kw) order as col2im_t_kernel, so the two give identical results.
template <typename T>
__global__ void __launch_bounds__(256) col2im_vec_kernel(const T* __restrict__ dcol, T* __restrict__ dXt, ConvGeom g,
                                                         int runs_per_row, int64_t threads, int vec) {
  using U = typename Word<T>::type;
  constexpr int EPC = Elem<T>::kPerChunk;        // elements per chunk
  constexpr int EW = 4 / sizeof(T);              // elements per 32-bit word
  constexpr int NCH = kRun / EPC + 1;            // chunks covering a window
  constexpr int NWD = 4 * NCH;                   // their words
  constexpr int OUTW = kRun / EW;                // words of the window
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= threads) return;
  const int64_t row = t / runs_per_row;             // (img*Cin + c)*H + h
  const int w0 = static_cast<int>(t - row * runs_per_row) * kRun;
  const int h = static_cast<int>(row % g.H);
  const int64_t ic = row / g.H;                     // img*Cin + c
  const int img = static_cast<int>(ic / g.Cin), c = static_cast<int>(ic - (int64_t)img * g.Cin);
  const int HWo = g.Ho * g.Wo;
  const int K = g.Cin * g.Kh * g.Kw;
  const int row_chunks = HWo / EPC;
  const T* __restrict__ base = dcol + ((int64_t)img * K + (int64_t)c * g.Kh * g.Kw) * HWo;
  float acc[kRun];
#pragma unroll
  for (int j = 0; j < kRun; ++j) acc[j] = 0.f;
  for (int kh = 0; kh < g.Kh; ++kh) {
    const int hn = h + g.ph - kh * g.dh;
    if (hn < 0) break;                              // hn only falls as kh grows
    const int ho = hn / g.sh;
    if (ho * g.sh != hn || ho >= g.Ho) continue;
    const T* __restrict__ krow = base + (int64_t)kh * g.Kw * HWo;
    for (int kw = 0; kw < g.Kw; ++kw) {
      const int wn0 = w0 + g.pw - kw * g.dw;        // output column of the first output
      const int a = ho * g.Wo + wn0;                // window start in the dcol row (may be < 0)
      const int c0 = (a >= 0 ? a : a - (EPC - 1)) / EPC;
      const int sh = a - c0 * EPC;                  // 0 .. EPC-1
      const T* __restrict__ p = krow + (int64_t)kw * HWo;
      uint32_t wd[NWD];
#pragma unroll
      for (int q = 0; q < NCH; ++q) {
        const int ci = min(max(c0 + q, 0), row_chunks - 1);
        const u32x4 v = *reinterpret_cast<const u32x4*>(p + (int64_t)ci * EPC);
#pragma unroll
        for (int i = 0; i < 4; ++i) wd[4 * q + i] = v[i];
      }
      // shift left by sh / EW words (two select stages), then by the odd
      // element of a 16-bit pair
      const int bw = sh / EW;
      if (bw & 1) {
#pragma unroll
        for (int i = 0; i + 1 < NWD; ++i) wd[i] = wd[i + 1];
      }
      if (bw & 2) {
#pragma unroll
        for (int i = 0; i + 2 < NWD; ++i) wd[i] = wd[i + 2];
      }
      uint32_t ow[OUTW];
#pragma unroll
      for (int q = 0; q < OUTW; ++q) {
        if constexpr (EW == 2) ow[q] = (sh & 1) ? __builtin_amdgcn_alignbit(wd[q + 1], wd[q], 16) : wd[q];
        else ow[q] = wd[q];
      }
#pragma unroll
      for (int j = 0; j < kRun; ++j) {
        const int wn = wn0 + j;
        if (w0 + j < g.W && wn >= 0 && wn < g.Wo) {
          if constexpr (EW == 2) acc[j] += Elem<T>::from_bits((ow[j >> 1] >> (16 * (j & 1))) & 0xffffu);
          else acc[j] += __uint_as_float(ow[j]);
        }
      }
    }
  }
  U v[kRun];
#pragma unroll
  for (int j = 0; j < kRun; ++j) v[j] = static_cast<U>(Elem<T>::bits(acc[j]));
  store_run(reinterpret_cast<U*>(dXt) + row * g.W + w0, v, g.W - w0, vec != 0);
}

// Running sums over images, in fp32: acc[i] = (first ? 0 : acc[i]) + src[0*n + i]
// + src[1*n + i] + ... with the slices added in order, so the sum does not depend
// on how many images one call holds.  One launch serves two jobs, dW (slices of
// T) and dB (fp32 slices).  A thread owns kAccV consecutive elements; with `vec`
// (n a multiple of kAccV, both arrays 16-byte aligned) a slice is one 8- or
// 16-byte load, and the loads of up to kAccSlices slices are issued before
// their adds.
constexpr int kAccV = 4;
constexpr int kAccSlices = 16;

struct AccJob {
  float* acc; const void* src; int64_t n; int64_t threads; int vec;
};

template <typename T>
__device__ __forceinline__ void acc_job(const AccJob& j, int64_t t, int slices, int first) {
  using Raw = typename std::conditional<sizeof(T) == 2, u32x2, u32x4>::type;
  const int64_t i0 = t * kAccV;
  const T* __restrict__ src = static_cast<const T*>(j.src);
  float v[kAccV];
  if (j.vec) {
    if (first) {
#pragma unroll
      for (int e = 0; e < kAccV; ++e) v[e] = 0.f;
    } else {
      const f32x4_t a = *reinterpret_cast<const f32x4_t*>(j.acc + i0);
#pragma unroll
      for (int e = 0; e < kAccV; ++e) v[e] = a[e];
    }
    for (int s0 = 0; s0 < slices; s0 += kAccSlices) {
      Raw r[kAccSlices];
#pragma unroll
      for (int u = 0; u < kAccSlices; ++u)
        if (s0 + u < slices) r[u] = *reinterpret_cast<const Raw*>(src + (int64_t)(s0 + u) * j.n + i0);
#pragma unroll
      for (int u = 0; u < kAccSlices; ++u) {
        if (s0 + u >= slices) continue;
#pragma unroll
        for (int e = 0; e < kAccV; ++e) {
          if constexpr (sizeof(T) == 2) v[e] += Elem<T>::from_bits((r[u][e >> 1] >> (16 * (e & 1))) & 0xffffu);
          else v[e] += __uint_as_float(r[u][e]);
        }
      }
    }
    f32x4_t a;
#pragma unroll
    for (int e = 0; e < kAccV; ++e) a[e] = v[e];
    *reinterpret_cast<f32x4_t*>(j.acc + i0) = a;
    return;
  }
  for (int e = 0; e < kAccV; ++e) {
    const int64_t i = i0 + e;
    if (i >= j.n) break;
    float x = first ? 0.f : j.acc[i];
    for (int q = 0; q < slices; ++q) x += Elem<T>::load1(src + (int64_t)q * j.n + i);
    j.acc[i] = x;
  }
}

template <typename T>
__global__ void __launch_bounds__(64) acc_add_kernel(AccJob w, AccJob b, int slices, int first) {
  const int64_t t = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (t < w.threads) acc_job<T>(w, t, slices, first);
  else if (t - w.threads < b.threads) acc_job<float>(b, t - w.threads, slices, first);
}

// The results: dW (rounded to T) from its sum and dB (fp32) from its sum, in
// one launch.
template <typename T>
__global__ void __launch_bounds__(256) acc_store_kernel(T* __restrict__ dW, const float* __restrict__ accW, int64_t nW,
                                                        float* __restrict__ dB, const float* __restrict__ accB,
                                                        int64_t nB) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nW) Elem<T>::store1(dW + i, accW[i]);
  else if (i - nW < nB) dB[i - nW] = accB[i - nW];
}

constexpr int kIm2colLdsBytes = 32 * 1024;

template <typename T>
static hipError_t launch_im2col(const void* X, void* col, const ConvGeom& g, int imgs, hipStream_t s) {
  const int64_t HWo = (int64_t)g.Ho * g.Wo;
  // LDS band: the most output rows whose input rows fit in kIm2colLdsBytes
  int TH = g.Ho;
  auto band_bytes = [&g](int th) { return ((int64_t)(th - 1) * g.sh + (int64_t)(g.Kh - 1) * g.dh + 1) * g.W * sizeof(T); };
  while (TH > 1 && band_bytes(TH) > kIm2colLdsBytes) TH = (TH + 1) / 2;
  if (band_bytes(TH) <= kIm2colLdsBytes) {
    const int bands = (g.Ho + TH - 1) / TH;
    const int64_t blocks = (int64_t)imgs * g.Cin * bands;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    // 16-byte stores: every band starts on a 16-byte boundary of its col row
    const int vec = (HWo * (int64_t)sizeof(T)) % 16 == 0 && ((int64_t)TH * g.Wo * sizeof(T)) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(col) % 16 == 0;
    const int xvec = ((int64_t)g.W * sizeof(T)) % 16 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0;
    // chunked LDS reads: unit horizontal stride, whole runs per output row,
    // 16-byte LDS rows
    if (g.sw == 1 && g.Wo % kRun == 0 && xvec)
      hipLaunchKernelGGL((im2col_lds_kernel<T, true>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                         static_cast<unsigned>(band_bytes(TH)), s, static_cast<const T*>(X), static_cast<T*>(col), g,
                         TH, bands, vec, xvec);
    else
      hipLaunchKernelGGL((im2col_lds_kernel<T, false>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                         static_cast<unsigned>(band_bytes(TH)), s, static_cast<const T*>(X), static_cast<T*>(col), g,
                         TH, bands, vec, xvec);
    return hipGetLastError();
  }
  const int runs = static_cast<int>((HWo + kRun - 1) / kRun);
  const int64_t threads = (int64_t)imgs * g.Cin * g.Kh * g.Kw * runs;
  if ((threads + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
  // 16-byte stores: every row starts on a 16-byte boundary
  const int vec = (HWo * (int64_t)sizeof(T)) % 16 == 0 && reinterpret_cast<uintptr_t>(col) % 16 == 0;
  hipLaunchKernelGGL((im2col_t_kernel<T>), dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s,
                     static_cast<const T*>(X), static_cast<T*>(col), g, runs, threads, vec);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_col2im(const void* dcol, void* dX, const ConvGeom& g, int imgs, hipStream_t s) {
  const int runs = (g.W + kRun - 1) / kRun;
  const int64_t threads = (int64_t)imgs * g.Cin * g.H * runs;
  if ((threads + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
  const int vec = ((int64_t)g.W * sizeof(T)) % 16 == 0 && reinterpret_cast<uintptr_t>(dX) % 16 == 0;
  const bool rows16 = ((int64_t)g.Ho * g.Wo * sizeof(T)) % 16 == 0 && reinterpret_cast<uintptr_t>(dcol) % 16 == 0;
  if (g.sw == 1 && rows16)
    hipLaunchKernelGGL((col2im_vec_kernel<T>), dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s,
                       static_cast<const T*>(dcol), static_cast<T*>(dX), g, runs, threads, vec);
  else
    hipLaunchKernelGGL((col2im_t_kernel<T>), dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s,
                       static_cast<const T*>(dcol), static_cast<T*>(dX), g, runs, threads, vec);
  return hipGetLastError();
}

inline AccJob acc_job_of(float* acc, const void* src, int64_t n, size_t es) {
  AccJob j{acc, src, acc ? n : 0, 0, 0};
  if (!acc) return j;
  j.threads = (n + kAccV - 1) / kAccV;
  j.vec = n % kAccV == 0 && reinterpret_cast<uintptr_t>(acc) % 16 == 0 &&
          reinterpret_cast<uintptr_t>(src) % (kAccV * es) == 0;
  return j;
}

// accW += the `slices` dW slices of T at gw (when accW is set), accB += the dB
// slices at gb (when accB is set), in one launch.
template <typename T>
static hipError_t launch_acc_add(float* accW, const void* gw, int64_t nW, float* accB, const float* gb, int64_t nB,
                                 int slices, bool first, hipStream_t s) {
  const AccJob w = acc_job_of(accW, gw, nW, sizeof(T)), b = acc_job_of(accB, gb, nB, sizeof(float));
  const int64_t threads = w.threads + b.threads;
  if (threads == 0) return hipSuccess;
  if ((threads + 63) / 64 > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((acc_add_kernel<T>), dim3(static_cast<unsigned>((threads + 63) / 64)), dim3(64), 0, s, w, b,
                     slices, first ? 1 : 0);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_acc_store(void* dW, const float* accW, int64_t nW, float* dB, const float* accB, int64_t nB,
                                   hipStream_t s) {
  if (!dW) nW = 0;
  if (!dB) nB = 0;
  const int64_t n = nW + nB;
  if (n == 0) return hipSuccess;
  if ((n + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((acc_store_kernel<T>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                     static_cast<T*>(dW), accW, nW, dB, accB, nB);
  return hipGetLastError();
}

#define GEV2_DISPATCH_T(dtype, F, ...)                            \
  ((dtype) == GEV2_F32 ? F<float>(__VA_ARGS__)                    \
   : (dtype) == GEV2_BF16 ? F<__bf16>(__VA_ARGS__)                \
                          : F<_Float16>(__VA_ARGS__))

}  // namespace gev2

namespace {

thread_local std::string t_conv_error;

int conv_fail(int st, const char* msg) {
  t_conv_error = msg;
  return st;
}

size_t esize(int dtype) { return dtype == GEV2_F32 ? 4 : 2; }

// Shape validation shared by forward and backward (launcher.cu:110-144, 241-276).
template <typename D>
int conv_check(const D* d, gev2::ConvGeom* g) {
  if (!d) return conv_fail(GEV2_INVALID_ARGUMENT, "null descriptor");
  if (d->dtype != GEV2_F32 && d->dtype != GEV2_F16 && d->dtype != GEV2_BF16)
    return conv_fail(GEV2_DTYPE_MISMATCH, "dtype must be F32, F16 or BF16");
  if (d->act < GEV2_ACT_NONE || d->act > GEV2_ACT_TANH) return conv_fail(GEV2_INVALID_ARGUMENT, "bad act kind");
  if (d->groups != 1) return conv_fail(GEV2_UNIMPLEMENTED, "groups != 1");
  if (d->N <= 0 || d->Cin <= 0 || d->H <= 0 || d->W <= 0 || d->Cout <= 0 || d->Kh <= 0 || d->Kw <= 0 ||
      d->stride_h <= 0 || d->stride_w <= 0 || d->dil_h <= 0 || d->dil_w <= 0 || d->pad_h < 0 || d->pad_w < 0)
    return conv_fail(GEV2_INVALID, "non-positive dimension, stride or dilation, or negative padding");
  g->Cin = d->Cin; g->H = d->H; g->W = d->W; g->Kh = d->Kh; g->Kw = d->Kw;
  g->sh = d->stride_h; g->sw = d->stride_w; g->ph = d->pad_h; g->pw = d->pad_w; g->dh = d->dil_h; g->dw = d->dil_w;
  g->Ho = (d->H + 2 * d->pad_h - d->dil_h * (d->Kh - 1) - 1) / d->stride_h + 1;
  g->Wo = (d->W + 2 * d->pad_w - d->dil_w * (d->Kw - 1) - 1) / d->stride_w + 1;
  if (g->Ho <= 0 || g->Wo <= 0) return conv_fail(GEV2_INVALID, "empty output");
  const int64_t K = (int64_t)d->Cin * d->Kh * d->Kw, HWo = (int64_t)g->Ho * g->Wo;
  if (K * HWo > 0x7fffffffLL || (int64_t)d->Cout * HWo > 0x7fffffffLL || (int64_t)d->Cin * d->H * d->W > 0x7fffffffLL)
    return conv_fail(GEV2_INVALID, "per-image sizes must fit int32");
  return GEV2_OK;
}

int gemm_status(int st) {
  if (st != GEV2_OK) t_conv_error = std::string("gemm: ") + gev2_last_error();
  return st;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return GEV2_OK;
  t_conv_error = std::string(where) + ": " + hipGetErrorString(e);
  return GEV2_HIP_ERROR;
}

}  // namespace

extern "C" {

const char* gev2_conv2d_last_error(void) { return t_conv_error.c_str(); }

int gev2_conv2d_fwd(const gev2_conv2d_desc* d, void* stream) {
  t_conv_error.clear();
  gev2::ConvGeom g{};
  int st = conv_check(d, &g);
  if (st != GEV2_OK) return st;
  if (!d->X || !d->Wt) return conv_fail(GEV2_MISSING_INPUT, "X / W is null");
  if (!d->Y) return conv_fail(GEV2_MISSING_OUTPUT, "Y is null");
  if (d->save_z && !d->Z) return conv_fail(GEV2_MISSING_OUTPUT, "save_z requires Z");
  const int64_t K = (int64_t)d->Cin * d->Kh * d->Kw, HWo = (int64_t)g.Ho * g.Wo;
  const int64_t per_img = K * HWo * static_cast<int64_t>(esize(d->dtype));
  if (!d->col || d->col_bytes < per_img) return conv_fail(GEV2_MISSING_INPUT, "col workspace smaller than one image");
  const int chunk = static_cast<int>(std::min<int64_t>(d->N, d->col_bytes / per_img));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const size_t es = esize(d->dtype);
  for (int n0 = 0; n0 < d->N; n0 += chunk) {
    const int c = std::min(chunk, d->N - n0);
    const char* x = static_cast<const char*>(d->X) + (size_t)n0 * d->Cin * d->H * d->W * es;
    st = hip_status(GEV2_DISPATCH_T(d->dtype, gev2::launch_im2col, x, d->col, g, c, s), "im2col");
    if (st != GEV2_OK) return st;
    gev2_gemm_fwd_desc f{};
    f.dtype = d->dtype; f.act = d->act; f.leaky_slope = d->leaky_slope; f.alpha = 1.f;
    f.bias_kind = d->bias ? GEV2_BIAS_PER_M : GEV2_BIAS_NONE;
    f.M = d->Cout; f.N = HWo; f.K = K; f.batch = c;
    f.A = d->Wt; f.lda = K; f.stride_a = 0;
    f.B = d->col; f.ldb = HWo; f.stride_b = K * HWo;
    f.bias = d->bias; f.stride_bias = 0;
    f.Y = static_cast<char*>(d->Y) + (size_t)n0 * d->Cout * HWo * es; f.ldy = HWo; f.stride_y = d->Cout * HWo;
    if (d->save_z) {
      f.Z = static_cast<char*>(d->Z) + (size_t)n0 * d->Cout * HWo * es; f.ldz = HWo; f.stride_z = d->Cout * HWo;
    }
    st = gemm_status(gev2_gemm_fwd(&f, stream));
    if (st != GEV2_OK) return st;
  }
  return GEV2_OK;
}

int gev2_conv2d_bwd(const gev2_conv2d_bwd_desc* d, void* stream) {
  t_conv_error.clear();
  gev2::ConvGeom g{};
  int st = conv_check(d, &g);
  if (st != GEV2_OK) return st;
  if (!d->X || !d->Wt || !d->dY || !d->Z) return conv_fail(GEV2_MISSING_INPUT, "X / W / dY / Z is null");
  if (!d->dW && !d->dB && !d->dX) return GEV2_OK;
  const int64_t K = (int64_t)d->Cin * d->Kh * d->Kw, HWo = (int64_t)g.Ho * g.Wo, CK = (int64_t)d->Cout * K;
  const int64_t es = static_cast<int64_t>(esize(d->dtype));
  // images per batched call: what every workspace in use holds
  int64_t chunk = d->N;
  auto fit = [&chunk](int64_t bytes, int64_t per_img) { chunk = std::min(chunk, bytes / per_img); };
  if (!d->col) return conv_fail(GEV2_MISSING_INPUT, "col workspace is required");
  fit(d->col_bytes, K * HWo * es);
  if (d->dX) {
    if (!d->dcol) return conv_fail(GEV2_MISSING_INPUT, "dX needs the dcol workspace");
    fit(d->dcol_bytes, K * HWo * es);
  }
  if (d->dW) {
    if (!d->gw || !d->acc_w) return conv_fail(GEV2_MISSING_INPUT, "dW needs the gw and acc_w workspaces");
    fit(d->gw_bytes, CK * es);
  }
  // dB: acc_b holds the running sum [Cout] and, when it has room, the chunk's
  // per-image slices [chunk][Cout].  With room for the sum only (the
  // reference's gy_rows is Cout*Ho*Wo floats, so Cout floats at a 1x1 output),
  // each image's slice goes to dB itself, one image per call: dB is written
  // from the sum only after the last image.
  bool db_slices_in_acc = true;
  if (d->dB) {
    if (!d->acc_b || d->acc_b_bytes < 4 * (int64_t)d->Cout)
      return conv_fail(GEV2_MISSING_INPUT, "dB needs the acc_b workspace (at least Cout floats)");
    if (d->acc_b_bytes >= 8 * (int64_t)d->Cout) {
      fit(d->acc_b_bytes - 4 * (int64_t)d->Cout, 4 * (int64_t)d->Cout);
    } else {
      db_slices_in_acc = false;
      chunk = std::min<int64_t>(chunk, 1);
    }
  }
  if (chunk < 1) return conv_fail(GEV2_MISSING_INPUT, "a workspace is smaller than one image needs");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float* accW = d->acc_w;               // [Cout*K] sum of dW_n
  float* accB = d->acc_b;               // [Cout]   sum of dB_n
  float* gb = db_slices_in_acc ? d->acc_b + d->Cout : d->dB;   // [chunk][Cout] dB_n
  for (int64_t n0 = 0; n0 < d->N; n0 += chunk) {
    const int c = static_cast<int>(std::min<int64_t>(chunk, d->N - n0));
    const char* x = static_cast<const char*>(d->X) + n0 * d->Cin * d->H * d->W * es;
    st = hip_status(GEV2_DISPATCH_T(d->dtype, gev2::launch_im2col, x, d->col, g, c, s), "im2col");
    if (st != GEV2_OK) return st;
    gev2_gemm_bwd_desc b{};
    b.dtype = d->dtype; b.act = d->act; b.leaky_slope = d->leaky_slope; b.alpha = 1.f; b.beta = 0.f;
    b.bias_kind = d->dB ? GEV2_BIAS_PER_M : GEV2_BIAS_NONE;
    b.M = d->Cout; b.N = HWo; b.K = K; b.batch = c;
    b.A = d->Wt; b.lda = K; b.stride_a = 0;
    b.B = d->col; b.ldb = HWo; b.stride_b = K * HWo;
    b.gY = static_cast<const char*>(d->dY) + n0 * d->Cout * HWo * es; b.ldgy = HWo; b.stride_gy = d->Cout * HWo;
    b.Z = static_cast<const char*>(d->Z) + n0 * d->Cout * HWo * es; b.ldz = HWo; b.stride_z = d->Cout * HWo;
    if (d->dW) { b.gA = d->gw; b.ldga = K; b.stride_ga = CK; }
    if (d->dX) { b.gB = d->dcol; b.ldgb = HWo; b.stride_gb = K * HWo; }
    if (d->dB) { b.gBias = gb; b.stride_gbias = d->Cout; }
    b.workspace = d->dz; b.workspace_bytes = d->dz_bytes;
    st = gemm_status(gev2_gemm_bwd(&b, stream));
    if (st != GEV2_OK) return st;
    if (d->dW || d->dB) {
      st = hip_status(GEV2_DISPATCH_T(d->dtype, gev2::launch_acc_add, d->dW ? accW : nullptr, d->gw, CK,
                                      d->dB ? accB : nullptr, gb, d->Cout, c, n0 == 0, s),
                      "acc dW / dB");
      if (st != GEV2_OK) return st;
    }
    if (d->dX) {
      char* dx = static_cast<char*>(d->dX) + n0 * d->Cin * d->H * d->W * es;
      st = hip_status(GEV2_DISPATCH_T(d->dtype, gev2::launch_col2im, d->dcol, dx, g, c, s), "col2im");
      if (st != GEV2_OK) return st;
    }
  }
  return hip_status(GEV2_DISPATCH_T(d->dtype, gev2::launch_acc_store, d->dW, accW, CK, d->dB, accB, d->Cout, s),
                    "store dW / dB");
}

}  // extern "C"
