// Scaled dot-product attention: the sdpa op of graph_executor_v2
// (backends/cuda/ops/sdpa/api.hpp:8-33, launcher.cu:129-747) rebuilt for
// gfx950.
//
//   S = scale * Q K^T (+ mask) ,  P = softmax_rows(S) ,  Y = P V
//   Q [B,H,M,D], K / V [B,H,N,D], Y [B,H,M,D]; scale = attrs.scale or 1/sqrt(D);
//   causal adds -1e9 where key > query; an external mask [B,1,M,N] adds -1e9
//   where an I8 / I32 entry is non-zero, or adds an F32 entry
//   (launcher.cu:44-105, 179-215, 251-257).
//
// 16-bit tensors: one fused kernel (flash style) per launch.  A workgroup
// owns 128 queries of one (b, h) and streams K / V in blocks of 64 keys
// through LDS (direct-to-LDS loads, two stages).  Each wave computes
// S^T = K Q^T for its 32 queries with v_mfma_f32_16x16x32 (K rows as the
// A operand, Q rows held in registers as the B operand), so every lane owns
// one query column: the online softmax (running max and sum, fp32) needs only
// two cross-lane steps, and P^T goes from the accumulators straight into the
// B operand of O^T += V^T P^T (V read with LDS transpose reads, keys in the
// matching permuted order).  S and P never reach memory; the row
// log-sum-exp is written for the backward.
// fp32 tensors (the reference's type): the reference's algorithm, batched --
// one strided GEMM launch for all (b, h) slices per product, with the scale
// as the GEMM's alpha and K read transposed in place, a row-softmax kernel
// that applies the masks, S / P in a caller workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>

#include "../../include/gev2_gemm.h"
#include "gev2_device.hpp"

namespace gev2 {

constexpr float kMaskNeg = -1e9f;          // launcher.cu:152
// queries per wave: 16 * QT (QT = 1 or 2); a workgroup has 4 waves
__host__ __device__ constexpr int attn_wg_queries(int qt) { return 64 * qt; }
// keys per block: 16 * KT (KT = 4 or 8)

struct AttnArgs {
  const void* Q;
  const void* K;
  const void* V;
  void* Y;
  float* lse;            // [BH, M] natural-log sum of exp, optional
  const void* mask;      // [B, M, N] (broadcast over H), optional
  int mask_kind;         // GEV2_MASK_*
  int BH, H, M, N;
  float scale;
  int causal;
  int qblocks;           // ceil(M / attn_wg_queries(QT))
};

// Mask term added to a scaled score (the reference adds the external mask,
// then the causal term).
__device__ __forceinline__ float mask_add(float x, const AttnArgs& a, int b, int q, int key) {
  if (a.mask_kind != GEV2_MASK_NONE) {
    const int64_t i = ((int64_t)b * a.M + q) * a.N + key;
    if (a.mask_kind == GEV2_MASK_I8) {
      if (static_cast<const int8_t*>(a.mask)[i]) x += kMaskNeg;
    } else if (a.mask_kind == GEV2_MASK_I32) {
      if (static_cast<const int32_t*>(a.mask)[i]) x += kMaskNeg;
    } else {
      x += static_cast<const float*>(a.mask)[i];
    }
  }
  if (a.causal && key > q) x += kMaskNeg;
  return x;
}

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m)); }
__device__ __forceinline__ float xor_sum(float v, int m) { return v + __shfl_xor(v, m); }

template <typename T>
__device__ __forceinline__ f32x4_t mfma_16x16x32(const u32x4& a, const u32x4& b, const f32x4_t& c) {
  if constexpr (__is_same(T, __bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

// LDS image of one key block: K rows with 16-byte chunks XOR-swizzled by
// (row & 7) (rows read whole for the A operand), V rows with 32-byte blocks
// XOR-swizzled by (row & 3) (read with transpose reads).
template <int D, int KT>
struct KvBlock {
  static constexpr int kKeys = 16 * KT;
  static constexpr int kRowBytes = D * 2;
  static constexpr int kBytes = kKeys * kRowBytes;            // one of K or V
  static constexpr int kLoadsPerWave = kBytes / 1024 / 4;     // 1 KB loads, 4 waves
  static constexpr int kChunks = D / 8;                       // 16-byte chunks per row
};

// Issue this wave's direct-to-LDS loads of K and V rows [key0, key0 + 16 KT).
template <int D, int KT>
__device__ __forceinline__ void load_kv(const i32x4_t& rK, const i32x4_t& rV, int64_t head_off, int key0, int N,
                                        int wave, int lane, uint32_t k_lds, uint32_t v_lds) {
  using B = KvBlock<D, KT>;
  constexpr int rows_per_load = 1024 / B::kRowBytes;
#pragma unroll
  for (int j = 0; j < B::kLoadsPerWave; ++j) {
    const int ld = wave * B::kLoadsPerWave + j;               // 1 KB piece of the block
    const int row = ld * rows_per_load + lane / B::kChunks;
    const int pc = lane % B::kChunks;                         // physical 16-byte chunk
    const int key = key0 + row;
    const int ck = pc ^ (row & 7);                            // K: logical chunk
    const int cv = (((pc >> 1) ^ (row & 3)) << 1) | (pc & 1); // V: logical chunk
    const bool in = key < N;
    const int offk = in ? static_cast<int>(((head_off + key) * D + ck * 8) * 2) : kOobOffset;
    const int offv = in ? static_cast<int>(((head_off + key) * D + cv * 8) * 2) : kOobOffset;
    dma16(rK, offk, 0, k_lds + ld * 1024);
    dma16(rV, offv, 0, v_lds + ld * 1024);
  }
}

// MASKED: causal and / or an external mask, or a scale <= 0 (scores formed as
// the reference forms them: scale, then the fp32 mask additions).  Otherwise
// the row maximum is taken over the raw dot products and scale * log2(e)
// enters through the exponent's FMA.  Maxima are kept in base-2 units.
// CAUSAL (without MASKED): a key past the query is excluded outright.  With
// causal masking alone no row is fully masked (key 0 is never past a query),
// so exp(score - 1e9 - max) underflows to exactly 0 and the exclusion is the
// same as the reference's -1e9 addition.
template <typename T, int D, bool MASKED, bool CAUSAL, int QT, int KT>
__global__ void __launch_bounds__(256) attn_fwd_kernel(AttnArgs a) {
  constexpr int kWgQ = attn_wg_queries(QT);
  using B = KvBlock<D, KT>;
  constexpr int kAttnKeys = B::kKeys;
  constexpr int KS = D / 32;                 // k-steps of the S^T product
  constexpr int DT = D / 16;                 // 16-row tiles of O^T
  constexpr int NL = 2 * B::kLoadsPerWave;   // loads per wave per block
  __shared__ __attribute__((aligned(1024))) char lds[2][2][B::kBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, col = lane & 15;

  // workgroup -> (head, query block); the 8 XCDs each take a contiguous
  // range of heads so that a head's K / V stay in one L2
  const int total = a.BH * a.qblocks;
  int lin = blockIdx.x;
  if ((total & 7) == 0) lin = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int bh = lin / a.qblocks;
  int qb = lin - bh * a.qblocks;
  if (CAUSAL) qb = a.qblocks - 1 - qb;       // the longest query blocks start first
  const int b = bh / a.H;
  const int64_t qhead = (int64_t)bh * a.M, khead = (int64_t)bh * a.N;

  // this lane's query columns; Q rows as B operands (k = d 32s + 8g ..)
  int q[QT];
  u32x4 qf[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    q[qt] = qb * kWgQ + wave * 16 * QT + qt * 16 + col;
    const T* qrow = static_cast<const T*>(a.Q) + (qhead + q[qt]) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[qt][s] = q[qt] < a.M ? *reinterpret_cast<const u32x4*>(qrow + 32 * s + 8 * g) : u32x4{0u, 0u, 0u, 0u};
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);        // vmcnt(0): Q in registers before the loads below
  asm volatile("" ::: "memory");

  const int qmin = qb * kWgQ + wave * 16 * QT;    // this wave's first query
  int nkb = (a.N + kAttnKeys - 1) / kAttnKeys;
  if (a.causal && a.mask_kind == GEV2_MASK_NONE) {
    // blocks whose every key is past every query here add exp(-1e9 + ...) = 0
    nkb = min(nkb, (qb * kWgQ + kWgQ - 1) / kAttnKeys + 1);
  }
  const i32x4_t rK = rsrc_words(a.K), rV = rsrc_words(a.V);
  const uint32_t base = lds_addr(&lds[0][0][0]);
  auto k_lds = [&](int st) { return base + st * 2 * B::kBytes; };
  auto v_lds = [&](int st) { return base + st * 2 * B::kBytes + B::kBytes; };

  float m_run[QT], l_run[QT];
  f32x4_t o[QT][DT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const float kLog2e = 1.4426950408889634f;
  // base-2 units throughout: x2 = score * log2(e), m in the same units
  const float xscale = a.scale * kLog2e;

  load_kv<D, KT>(rK, rV, khead, 0, a.N, wave, lane, k_lds(0), v_lds(0));
  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    if (kb + 1 < nkb) {
      load_kv<D, KT>(rK, rV, khead, (kb + 1) * kAttnKeys, a.N, wave, lane, k_lds(st ^ 1), v_lds(st ^ 1));
      __builtin_amdgcn_s_waitcnt(0x3f70 | (NL & 0xf) | ((NL >> 4) << 14));   // this block's loads done
    } else {
      __builtin_amdgcn_s_waitcnt(0x3f70);
    }
    __syncthreads();
    asm volatile("" ::: "memory");
    const char* kl = &lds[st][0][0];
    const char* vl = &lds[st][1][0];
    const bool tail = (kb + 1) * kAttnKeys > a.N;

    // S^T tiles: s[qt][kt] rows = keys 16 kt + 4 g + r, column = query q[qt]
    f32x4_t s[QT][KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int row = 16 * kt + col;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[qt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c = (4 * ks + g) ^ (row & 7);
        const u32x4 kf = *reinterpret_cast<const u32x4*>(kl + row * B::kRowBytes + c * 16);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) s[qt][kt] = mfma_16x16x32<T>(kf, qf[qt][ks], s[qt][kt]);
      }
    }

    // online softmax; P^T packed as the B operand of O^T += V^T P^T
    u32x4 pf[QT][KT / 2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      // x = the score in base-2 units: MASKED forms it as the reference does
      // (scale, then the fp32 mask additions); otherwise the scale (> 0) is
      // applied inside the exponent's FMA and the maximum taken over raw dots
      float x[KT][4];
      float mloc = -INFINITY;
      const int key0 = kb * kAttnKeys + 4 * g;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = s[qt][kt][r];
          if constexpr (MASKED) {
            const int key = key0 + 16 * kt + r;
            v = key < a.N ? mask_add(v * a.scale, a, b, min(q[qt], a.M - 1), key) * kLog2e : -INFINITY;
          }
          x[kt][r] = v;
        }
      }
      if (!MASKED && (tail || (CAUSAL && kb * kAttnKeys + kAttnKeys - 1 > qmin))) {
        // past the last key (zero-filled rows), or past the query: out of the softmax
        const int lim = CAUSAL ? min(a.N - 1, q[qt]) : a.N - 1;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) x[kt][r] = key0 + 16 * kt + r <= lim ? x[kt][r] : -INFINITY;
        }
      }
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) mloc = fmaxf(mloc, fmaxf(fmaxf(x[kt][0], x[kt][1]), fmaxf(x[kt][2], x[kt][3])));
      mloc = xor_max(xor_max(mloc, 16), 32);
      if constexpr (!MASKED) mloc *= xscale;
      const float m_new = fmaxf(m_run[qt], mloc);
      // raw v_exp_f32: every argument here is <= 0, so no range fix-up is needed
      const float corr = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
      const bool grew = m_new > m_run[qt];
      m_run[qt] = m_new;
      float lsum = 0.f;
      uint32_t pb[KT][4];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float arg = MASKED ? x[kt][r] - m_new : fmaf(x[kt][r], xscale, -m_new);
          const float p = __builtin_amdgcn_exp2f(arg);
          lsum += p;
          pb[kt][r] = Elem<T>::bits(p);
        }
      }
      l_run[qt] = l_run[qt] * corr + lsum;
      if (__any(grew)) {                      // rescale only when some row's maximum moved
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) o[qt][dt][r] *= corr;
        }
      }
#pragma unroll
      for (int j = 0; j < KT / 2; ++j) {
        pf[qt][j][0] = pack2(pb[2 * j][0], pb[2 * j][1]);
        pf[qt][j][1] = pack2(pb[2 * j][2], pb[2 * j][3]);
        pf[qt][j][2] = pack2(pb[2 * j + 1][0], pb[2 * j + 1][1]);
        pf[qt][j][3] = pack2(pb[2 * j + 1][2], pb[2 * j + 1][3]);
      }
    }

    // O^T[d][q] += V^T[d][key] P^T[key][q]; transpose reads: lane 16g + 4e + cq
    // addresses key 32j + 16h + 4g + e, columns 16 dt + 4 cq ..
    const int e = (lane >> 2) & 3, cq = lane & 3;
#pragma unroll
    for (int j = 0; j < KT / 2; ++j) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        u32x4 vf;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int row = 32 * j + 16 * h + 4 * g + e;
          const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4_t*)(vl + row * B::kRowBytes + ((dt ^ (row & 3)) << 5) +
                                                           cq * 8));
          const u32x2 w2 = __builtin_bit_cast(u32x2, v);
          vf[2 * h] = w2[0];
          vf[2 * h + 1] = w2[1];
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][dt] = mfma_16x16x32<T>(vf, pf[qt][j], o[qt][dt]);
      }
    }
    __syncthreads();                          // stage st is free for block kb + 2
  }

  // Y[q][16 dt + 4 g + r] = O^T / l; 8-byte stores
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l = xor_sum(xor_sum(l_run[qt], 16), 32);
    if (q[qt] >= a.M) continue;
    const float inv = 1.f / l;
    T* yrow = static_cast<T*>(a.Y) + (qhead + q[qt]) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      u32x2 w;
      w[0] = pack2(Elem<T>::bits(o[qt][dt][0] * inv), Elem<T>::bits(o[qt][dt][1] * inv));
      w[1] = pack2(Elem<T>::bits(o[qt][dt][2] * inv), Elem<T>::bits(o[qt][dt][3] * inv));
      *reinterpret_cast<u32x2*>(yrow + 16 * dt + 4 * g) = w;
    }
    if (a.lse && g == 0) a.lse[qhead + q[qt]] = (m_run[qt] + log2f(l)) * 0.69314718055994531f;
  }
}

template <typename T, int D, int QT>
hipError_t launch_attn_fwd_qt(AttnArgs a, hipStream_t s) {
  constexpr int KT = D == 64 ? 8 : 4;       // 128 keys per block at D = 64 (two workgroups per CU fit in LDS)
  a.qblocks = (a.M + attn_wg_queries(QT) - 1) / attn_wg_queries(QT);
  const int64_t blocks = (int64_t)a.BH * a.qblocks;
  if (a.mask_kind != GEV2_MASK_NONE || !(a.scale > 0.f))
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, true, false, QT, KT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       s, a);
  else if (a.causal)
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, false, true, QT, KT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       s, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, false, false, QT, KT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       s, a);
  return hipGetLastError();
}

// 32 queries per wave reuse each K / V fragment read twice; 16 per wave give
// twice the waves.  The second is taken when the first would leave CUs with
// fewer than two workgroups (one wave per SIMD cannot overlap the MFMA and
// softmax phases of a block).
template <typename T, int D>
hipError_t launch_attn_fwd(const AttnArgs& a, hipStream_t s) {
  const int64_t wg2 = (int64_t)a.BH * ((a.M + attn_wg_queries(2) - 1) / attn_wg_queries(2));
  const char* env = std::getenv("GEV2_ATTN_QT");        // 1 or 2 forces a variant (tuning runs)
  const int forced = env ? std::atoi(env) : 0;
  if (forced == 2 || (forced != 1 && wg2 >= 512)) return launch_attn_fwd_qt<T, D, 2>(a, s);
  return launch_attn_fwd_qt<T, D, 1>(a, s);
}

// ---------------------------------------------------------------------------
// fp32: row softmax of the scaled scores with the masks (softmax_run with
// scale 1 after scale_kernel and the mask kernels), in place on S.
// One wave per row.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) attn_softmax_rows_kernel(float* __restrict__ S, AttnArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (int64_t)a.BH * a.M) return;
  const int q = static_cast<int>(row % a.M);
  const int b = static_cast<int>(row / a.M) / a.H;
  float* srow = S + row * a.N;
  float mx = -INFINITY;
  for (int k = lane; k < a.N; k += 64) {
    const float v = mask_add(srow[k], a, b, q, k);
    srow[k] = v;
    mx = fmaxf(mx, v);
  }
  for (int o = 32; o > 0; o >>= 1) mx = xor_max(mx, o);
  float sum = 0.f;
  for (int k = lane; k < a.N; k += 64) {
    const float p = expf(srow[k] - mx);
    srow[k] = p;
    sum += p;
  }
  for (int o = 32; o > 0; o >>= 1) sum = xor_sum(sum, o);
  const float inv = 1.f / sum;
  for (int k = lane; k < a.N; k += 64) srow[k] *= inv;
}

// dS = P * (dP - sum_k dP P) on unmasked positions, 0 where masked
// (softmax_backward_run, then the mask / causal zeroing, launcher.cu:640-690).
__global__ void __launch_bounds__(256) attn_softmax_bwd_rows_kernel(const float* __restrict__ P, float* __restrict__ dP,
                                                                    AttnArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (int64_t)a.BH * a.M) return;
  const int q = static_cast<int>(row % a.M);
  const int b = static_cast<int>(row / a.M) / a.H;
  const float* prow = P + row * a.N;
  float* grow = dP + row * a.N;
  float dot = 0.f;
  for (int k = lane; k < a.N; k += 64) dot += grow[k] * prow[k];
  for (int o = 32; o > 0; o >>= 1) dot = xor_sum(dot, o);
  for (int k = lane; k < a.N; k += 64) {
    bool masked = a.causal && k > q;
    if (a.mask_kind != GEV2_MASK_NONE) {
      const int64_t i = ((int64_t)b * a.M + q) * a.N + k;
      if (a.mask_kind == GEV2_MASK_I8) masked |= static_cast<const int8_t*>(a.mask)[i] != 0;
      else if (a.mask_kind == GEV2_MASK_I32) masked |= static_cast<const int32_t*>(a.mask)[i] != 0;
      else masked |= static_cast<const float*>(a.mask)[i] != 0.f;
    }
    grow[k] = masked ? 0.f : prow[k] * (grow[k] - dot);
  }
}

// 16-bit <-> fp32 copies for the backward of 16-bit tensors
template <typename T>
__global__ void __launch_bounds__(256) attn_widen_kernel(const T* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = Elem<T>::load1(src + i);
}

template <typename T>
__global__ void __launch_bounds__(256) attn_narrow_kernel(const float* __restrict__ src, T* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) Elem<T>::store1(dst + i, src[i]);
}

inline hipError_t convert(int dtype, bool widen, const void* src, void* dst, int64_t n, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  if (dtype == GEV2_BF16) {
    if (widen) hipLaunchKernelGGL(attn_widen_kernel<__bf16>, grid, dim3(256), 0, s, static_cast<const __bf16*>(src),
                                  static_cast<float*>(dst), n);
    else hipLaunchKernelGGL(attn_narrow_kernel<__bf16>, grid, dim3(256), 0, s, static_cast<const float*>(src),
                            static_cast<__bf16*>(dst), n);
  } else {
    if (widen) hipLaunchKernelGGL(attn_widen_kernel<_Float16>, grid, dim3(256), 0, s,
                                  static_cast<const _Float16*>(src), static_cast<float*>(dst), n);
    else hipLaunchKernelGGL(attn_narrow_kernel<_Float16>, grid, dim3(256), 0, s, static_cast<const float*>(src),
                            static_cast<_Float16*>(dst), n);
  }
  return hipGetLastError();
}

}  // namespace gev2

namespace {

thread_local std::string t_attn_error;

int attn_fail(int st, const char* msg) {
  t_attn_error = msg;
  return st;
}

int gemm_status(int st) {
  if (st != GEV2_OK) t_attn_error = std::string("gemm: ") + gev2_last_error();
  return st;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return GEV2_OK;
  t_attn_error = std::string(where) + ": " + hipGetErrorString(e);
  return GEV2_HIP_ERROR;
}

template <typename Desc>
int attn_check(const Desc* d, gev2::AttnArgs* a) {
  if (!d) return attn_fail(GEV2_INVALID_ARGUMENT, "null descriptor");
  if (d->dtype != GEV2_F32 && d->dtype != GEV2_F16 && d->dtype != GEV2_BF16)
    return attn_fail(GEV2_DTYPE_MISMATCH, "dtype must be F32, F16 or BF16");
  if (d->B <= 0 || d->H <= 0 || d->M <= 0 || d->N <= 0 || d->D <= 0)
    return attn_fail(GEV2_INVALID, "B, H, M, N, D must be positive");
  if (d->mask_kind < GEV2_MASK_NONE || d->mask_kind > GEV2_MASK_F32)
    return attn_fail(GEV2_INVALID_ARGUMENT, "bad mask kind");
  if (d->mask_kind != GEV2_MASK_NONE && !d->mask) return attn_fail(GEV2_MISSING_INPUT, "mask kind set, mask null");
  if (d->dropout_p != 0.f) return attn_fail(GEV2_UNIMPLEMENTED, "dropout_p != 0 is not implemented");
  const int64_t BH = (int64_t)d->B * d->H;
  if (BH * d->M * d->D > 0x7fffffffLL || BH * d->N * d->D > 0x7fffffffLL || (int64_t)d->M * d->N > 0x7fffffffLL ||
      BH > 65535)
    return attn_fail(GEV2_INVALID, "sizes must fit int32 (and B*H <= 65535)");
  a->BH = static_cast<int>(BH);
  a->H = d->H; a->M = d->M; a->N = d->N;
  a->scale = d->scale != 0.f ? d->scale : 1.f / std::sqrt(static_cast<float>(d->D));
  a->causal = d->causal ? 1 : 0;
  a->mask = d->mask;
  a->mask_kind = d->mask_kind;
  return GEV2_OK;
}

bool fused_ok(int dtype, int D) { return dtype != GEV2_F32 && (D == 64 || D == 128); }

// scores workspace of the fp32 path: S / P [BH, M, N] (+ dP for the backward)
int64_t scores_bytes(int64_t BH, int64_t M, int64_t N) { return ((BH * M * N * 4 + 255) / 256) * 256; }

// one strided GEMM over all (b, h) slices
int slice_gemm(int dtype, bool ta, bool tb, float alpha, int64_t BH, int64_t M, int64_t N, int64_t K, const void* A,
               int64_t lda, int64_t sa, const void* Bm, int64_t ldb, int64_t sb, void* C, int64_t ldc, int64_t sc,
               void* stream) {
  gev2_gemm_fwd_desc f{};
  f.dtype = dtype; f.act = GEV2_ACT_NONE; f.bias_kind = GEV2_BIAS_NONE; f.alpha = alpha;
  f.trans_a = ta ? 1 : 0; f.trans_b = tb ? 1 : 0;
  f.M = M; f.N = N; f.K = K; f.batch = BH;
  f.A = A; f.lda = lda; f.stride_a = sa;
  f.B = Bm; f.ldb = ldb; f.stride_b = sb;
  f.Y = C; f.ldy = ldc; f.stride_y = sc;
  return gemm_status(gev2_gemm_fwd(&f, stream));
}

}  // namespace

extern "C" {

const char* gev2_sdpa_last_error(void) { return t_attn_error.c_str(); }

// fp32 copies of Q, K, V, dY and of dQ, dK, dV for a 16-bit backward
int64_t widened_bytes(int64_t BH, int64_t M, int64_t N, int64_t D) {
  return ((BH * (4 * M + 3 * N) * D * 4 + 255) / 256) * 256;
}

int64_t gev2_sdpa_workspace_size(const gev2_sdpa_desc* d, int backward) {
  gev2::AttnArgs a{};
  if (attn_check(d, &a) != GEV2_OK) return -1;
  if (fused_ok(d->dtype, d->D) && !backward) return 0;
  if (!backward) return scores_bytes(a.BH, d->M, d->N);
  const int64_t wide = d->dtype == GEV2_F32 ? 0 : widened_bytes(a.BH, d->M, d->N, d->D);
  return 2 * scores_bytes(a.BH, d->M, d->N) + wide;
}

int gev2_sdpa_fwd(const gev2_sdpa_desc* d, void* stream) {
  t_attn_error.clear();
  gev2::AttnArgs a{};
  int st = attn_check(d, &a);
  if (st != GEV2_OK) return st;
  if (!d->Q || !d->K || !d->V) return attn_fail(GEV2_MISSING_INPUT, "Q / K / V is null");
  if (!d->Y) return attn_fail(GEV2_MISSING_OUTPUT, "Y is null");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  a.Q = d->Q; a.K = d->K; a.V = d->V; a.Y = d->Y; a.lse = d->lse;
  const int64_t M = d->M, N = d->N, D = d->D;
  if (fused_ok(d->dtype, d->D)) {
    if (reinterpret_cast<uintptr_t>(d->Q) % 16 || reinterpret_cast<uintptr_t>(d->Y) % 16 ||
        a.BH * N * D * 2 > 0x7fffff00LL)
      return attn_fail(GEV2_INVALID, "fused path needs 16-byte aligned Q / Y and K / V under 2^31 bytes");
    hipError_t e;
    if (d->dtype == GEV2_BF16) e = d->D == 64 ? gev2::launch_attn_fwd<__bf16, 64>(a, s) : gev2::launch_attn_fwd<__bf16, 128>(a, s);
    else e = d->D == 64 ? gev2::launch_attn_fwd<_Float16, 64>(a, s) : gev2::launch_attn_fwd<_Float16, 128>(a, s);
    return hip_status(e, "attn_fwd");
  }
  if (d->dtype != GEV2_F32) return attn_fail(GEV2_UNIMPLEMENTED, "16-bit attention needs D = 64 or 128");
  if (d->lse) return attn_fail(GEV2_UNIMPLEMENTED, "lse output is produced by the fused 16-bit path only");
  // fp32: S = scale Q K^T (one launch, K read as B^T), row softmax with masks, Y = P V
  if (!d->workspace || d->workspace_bytes < scores_bytes(a.BH, M, N))
    return attn_fail(GEV2_MISSING_INPUT, "fp32 path needs a scores workspace (gev2_sdpa_workspace_size)");
  float* S = static_cast<float*>(d->workspace);
  st = slice_gemm(GEV2_F32, false, true, a.scale, a.BH, M, N, D, d->Q, D, M * D, d->K, D, N * D, S, N, M * N, stream);
  if (st != GEV2_OK) return st;
  hipLaunchKernelGGL(gev2::attn_softmax_rows_kernel, dim3(static_cast<unsigned>((a.BH * M + 3) / 4)), dim3(256), 0, s,
                     S, a);
  st = hip_status(hipGetLastError(), "softmax");
  if (st != GEV2_OK) return st;
  return slice_gemm(GEV2_F32, false, false, 1.f, a.BH, M, D, N, S, N, M * N, d->V, D, N * D, d->Y, D, M * D, stream);
}

int gev2_sdpa_bwd(const gev2_sdpa_bwd_desc* d, void* stream) {
  t_attn_error.clear();
  gev2::AttnArgs a{};
  int st = attn_check(d, &a);
  if (st != GEV2_OK) return st;
  if (!d->Q || !d->K || !d->V || !d->dY) return attn_fail(GEV2_MISSING_INPUT, "Q / K / V / dY is null");
  if (!d->dQ && !d->dK && !d->dV) return attn_fail(GEV2_INVALID, "all outputs null");   // launcher.cu:342
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t M = d->M, N = d->N, D = d->D, BH = a.BH;
  const int64_t sb = scores_bytes(BH, M, N);
  const bool wide = d->dtype != GEV2_F32;
  if (!d->workspace || d->workspace_bytes < 2 * sb + (wide ? widened_bytes(BH, M, N, D) : 0))
    return attn_fail(GEV2_MISSING_INPUT, "backward needs a workspace of gev2_sdpa_workspace_size(desc, 1) bytes");
  float* P = static_cast<float*>(d->workspace);
  float* dP = reinterpret_cast<float*>(static_cast<char*>(d->workspace) + sb);
  if (wide) {
    // 16-bit tensors: the fp32 path below on widened copies, gradients rounded back
    float* w = reinterpret_cast<float*>(static_cast<char*>(d->workspace) + 2 * sb);
    float *q = w, *k = q + BH * M * D, *v = k + BH * N * D, *dy = v + BH * N * D;
    float *dq = dy + BH * M * D, *dk = dq + BH * M * D, *dv = dk + BH * N * D;
    const void* src[4] = {d->Q, d->K, d->V, d->dY};
    float* dst[4] = {q, k, v, dy};
    const int64_t cnt[4] = {BH * M * D, BH * N * D, BH * N * D, BH * M * D};
    for (int i = 0; i < 4; ++i) {
      st = hip_status(gev2::convert(d->dtype, true, src[i], dst[i], cnt[i], s), "widen");
      if (st != GEV2_OK) return st;
    }
    gev2_sdpa_bwd_desc f = *d;
    f.dtype = GEV2_F32;
    f.Q = q; f.K = k; f.V = v; f.dY = dy;
    f.dQ = d->dQ ? dq : nullptr; f.dK = d->dK ? dk : nullptr; f.dV = d->dV ? dv : nullptr;
    f.workspace_bytes = 2 * sb;
    st = gev2_sdpa_bwd(&f, stream);
    if (st != GEV2_OK) return st;
    void* outs[3] = {d->dQ, d->dK, d->dV};
    const float* res[3] = {dq, dk, dv};
    const int64_t on[3] = {BH * M * D, BH * N * D, BH * N * D};
    for (int i = 0; i < 3; ++i) {
      if (!outs[i]) continue;
      st = hip_status(gev2::convert(d->dtype, false, res[i], outs[i], on[i], s), "narrow");
      if (st != GEV2_OK) return st;
    }
    return GEV2_OK;
  }
  // P = softmax(scale Q K^T + masks)
  st = slice_gemm(GEV2_F32, false, true, a.scale, BH, M, N, D, d->Q, D, M * D, d->K, D, N * D, P, N, M * N, stream);
  if (st != GEV2_OK) return st;
  hipLaunchKernelGGL(gev2::attn_softmax_rows_kernel, dim3(static_cast<unsigned>((BH * M + 3) / 4)), dim3(256), 0, s, P,
                     a);
  st = hip_status(hipGetLastError(), "softmax");
  if (st != GEV2_OK) return st;
  // dV = P^T dY
  if (d->dV) {
    st = slice_gemm(GEV2_F32, true, false, 1.f, BH, N, D, M, P, N, M * N, d->dY, D, M * D, d->dV, D, N * D, stream);
    if (st != GEV2_OK) return st;
  }
  if (!d->dQ && !d->dK) return GEV2_OK;
  // dP = dY V^T, then dS = P (dP - rowsum(dP P)) with masked positions zeroed
  st = slice_gemm(GEV2_F32, false, true, 1.f, BH, M, N, D, d->dY, D, M * D, d->V, D, N * D, dP, N, M * N, stream);
  if (st != GEV2_OK) return st;
  hipLaunchKernelGGL(gev2::attn_softmax_bwd_rows_kernel, dim3(static_cast<unsigned>((BH * M + 3) / 4)), dim3(256), 0,
                     s, P, dP, a);
  st = hip_status(hipGetLastError(), "softmax backward");
  if (st != GEV2_OK) return st;
  // dQ = scale dS K ; dK = scale dS^T Q
  if (d->dQ) {
    st = slice_gemm(GEV2_F32, false, false, a.scale, BH, M, D, N, dP, N, M * N, d->K, D, N * D, d->dQ, D, M * D,
                    stream);
    if (st != GEV2_OK) return st;
  }
  if (d->dK) {
    st = slice_gemm(GEV2_F32, true, false, a.scale, BH, N, D, M, dP, N, M * N, d->Q, D, M * D, d->dK, D, N * D,
                    stream);
    if (st != GEV2_OK) return st;
  }
  return GEV2_OK;
}

}  // extern "C"
