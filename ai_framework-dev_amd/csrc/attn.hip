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
  float* lse;            // [BH, lse_ld] natural-log sum of exp, optional
  int lse_ld;            // rows per head in lse (M; the backward pads it to a multiple of 64)
  const void* mask;      // [B, M, N] (broadcast over H), optional
  int mask_kind;         // GEV2_MASK_*
  int BH, H, M, N;
  float scale;
  int causal;
  int qblocks;           // ceil(M / attn_wg_queries(QT))
  int drop;              // dropout on (p > 0)
  float drop_p;          // drop probability
  float drop_scale;      // factor of a kept probability: 1/(1-p) when scale_in_train, else 1
  uint64_t seed;         // dropout stream seed
};

// Dropout of the reference (dropout/kernels.cu:21-41): element (bh, q, key) of
// the [B*H, M, N] probabilities is kept when u, the low 32 bits of
// splitmix64(seed ^ counter) with counter = (bh*M + q)*N + key (the reference's
// counter_base (b*H+h)*M*N plus the index in the slice, sdpa/launcher.cu:249-258),
// gives float(u) * 2^-32 >= p.  splitmix64 is Steele, Lea and Flood's mixing
// function (its standard constants, as in the reference).
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// The factor a probability is multiplied by: drop_scale if kept, else 0.
__device__ __forceinline__ float drop_factor(const AttnArgs& a, int bh, int q, int key) {
  const uint64_t ctr = ((uint64_t)bh * a.M + q) * a.N + key;
  const uint32_t u = static_cast<uint32_t>(splitmix64(a.seed ^ ctr));
  return static_cast<float>(u) * (1.0f / 4294967296.0f) >= a.drop_p ? a.drop_scale : 0.f;
}

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

// Every 64- or 128-element 16-bit row tile in LDS here (K, V, Q, dO) stores
// row r's logical 16-byte chunk c at physical chunk c ^ att_swz<D>(r).  Two
// read patterns use the tiles: 16-byte row reads in which 8 consecutive lanes
// take one chunk of 8 consecutive rows (MFMA operands read whole), and
// transpose reads in which a half-wave takes one 32-byte block (two chunks) of
// 8 consecutive, 8-aligned rows.  Measured with the LDS bank-conflict counter
// on gfx950, the row reads are conflict free when those 8 rows' chunks differ
// in their low three bits, and the transpose reads when the 8 blocks differ in
// chunk bits 1-3 (with 128-byte rows, two rows share a bank period and the
// parity of the row separates them).  row & 7 gives both for D = 64; for
// D = 128, (row & 7) | ((row & 1) << 3) does (row & 7 alone, row & 15, or a
// 32-byte block swizzle each leave one pattern two-way conflicted).
template <int D>
__device__ __forceinline__ int att_swz(int row) {
  if constexpr (D == 128) return (row & 7) | ((row & 1) << 3);
  else return row & 7;
}

// Address of logical 16-byte chunk `chunk` of `row` in a tile of 2D-byte rows.
template <int D>
__device__ __forceinline__ const char* att_chunk(const char* base, int row, int chunk) {
  return base + row * (2 * D) + ((chunk ^ att_swz<D>(row)) << 4);
}

// LDS image of one key block: K rows (read whole for the A operand) and V rows
// (read with transpose reads), both in the att_swz layout.
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
    const int c = pc ^ att_swz<D>(row);                       // logical chunk
    const bool in = key < N;
    const int offk = in ? static_cast<int>(((head_off + key) * D + c * 8) * 2) : kOobOffset;
    const int offv = in ? static_cast<int>(((head_off + key) * D + c * 8) * 2) : kOobOffset;
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
        const u32x4 kf = *reinterpret_cast<const u32x4*>(att_chunk<D>(kl, row, 4 * ks + g));
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
          // dropout (masked variant only): the row sum keeps every probability,
          // P V only the kept ones
          if constexpr (MASKED)
            pb[kt][r] = Elem<T>::bits(a.drop ? p * drop_factor(a, bh, q[qt], key0 + 16 * kt + r) : p);
          else
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
              (__attribute__((address_space(3))) s16x4_t*)(att_chunk<D>(vl, row, 2 * dt + (cq >> 1)) +
                                                           (cq & 1) * 8));
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
    if (a.lse && g == 0) a.lse[(int64_t)bh * a.lse_ld + q[qt]] = (m_run[qt] + log2f(l)) * 0.69314718055994531f;
  }
}

template <typename T, int D, int QT>
hipError_t launch_attn_fwd_qt(AttnArgs a, hipStream_t s) {
  constexpr int KT = D == 64 ? 8 : 4;       // 128 keys per block at D = 64 (two workgroups per CU fit in LDS)
  a.qblocks = (a.M + attn_wg_queries(QT) - 1) / attn_wg_queries(QT);
  const int64_t blocks = (int64_t)a.BH * a.qblocks;
  if (a.mask_kind != GEV2_MASK_NONE || !(a.scale > 0.f) || a.drop)
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
// softmax phases of a block), and always at D = 128, where the 32-query
// variant's registers allow only one wave per SIMD (measured: 140 against
// 156 us at B 2, H 16, M = N = 2048).
template <typename T, int D>
hipError_t launch_attn_fwd(const AttnArgs& a, hipStream_t s) {
  const int64_t wg2 = (int64_t)a.BH * ((a.M + attn_wg_queries(2) - 1) / attn_wg_queries(2));
  if (D == 64 && wg2 >= 512) return launch_attn_fwd_qt<T, D, 2>(a, s);
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

// dst = dropout(P) over the [B*H, M, N] probabilities of the fp32 path
// (dropout_run of launcher.cu:249-258 and 454-490); dst may be P itself.
__global__ void __launch_bounds__(256) attn_dropout_kernel(const float* __restrict__ P, float* dst, AttnArgs a) {
  const int64_t total = (int64_t)a.BH * a.M * a.N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / a.N;
    const int key = static_cast<int>(i - row * a.N);
    dst[i] = P[i] * drop_factor(a, static_cast<int>(row / a.M), static_cast<int>(row % a.M), key);
  }
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
  const int bh = static_cast<int>(row / a.M);
  if (a.drop) {
    // dP of the kept probabilities only (the reference's dropout backward, launcher.cu:566-590)
    for (int k = lane; k < a.N; k += 64) grow[k] *= drop_factor(a, bh, q, k);
  }
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

// ---------------------------------------------------------------------------
// Fused backward of the 16-bit forward (flash style): P is recomputed from the
// forward's row log-sum-exp, never stored.
//   attn_bwd_dot_kernel:  Dq[q] = sum_d dO[q][d] O[q][d]
//   attn_bwd_kv_kernel:   a workgroup owns 64 keys (16 per wave, K / V rows in
//     registers) and streams 64-query blocks of Q and dO through LDS:
//     S = Q K^T and dP = dO V^T come out with the key in the lane, so
//     P = exp(scale S - lse) and dS = P (dP - Dq) feed dV^T += dO^T P and
//     dK^T += Q^T dS as B operands straight from registers (dO and Q read with
//     transpose reads, queries in the matching permuted order).
//   attn_bwd_q_kernel:    the forward's layout (query in the lane, 16 per
//     wave): S^T = K Q^T, dP^T = V dO^T, dS^T, dQ^T += K^T dS^T.
// Masked entries get dS = 0, as the reference zeroes them (any non-zero
// external mask entry, or key > query with causal).
// ---------------------------------------------------------------------------
struct AttnBwdArgs {
  AttnArgs f;            // Q, K, V, scale, masks, dims (f.Y = O, f.lse = lse)
  const void* dO;
  const float* Dq;       // [BH, M]
  void* dQ;
  void* dK;
  void* dV;
};

// 8 lanes per row, 16 bytes each per step
template <typename T>
__global__ void __launch_bounds__(256) attn_bwd_dot_kernel(const T* __restrict__ dO, const T* __restrict__ O,
                                                           float* __restrict__ Dq, int64_t rows, int D, int M,
                                                           int ld) {
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  if (row >= rows) return;
  float acc = 0.f;
  for (int d = sub * 8; d < D; d += 64) {
    float a[8], b[8];
    chunk_to_f32<T>(*reinterpret_cast<const u32x4*>(dO + row * D + d), a);
    chunk_to_f32<T>(*reinterpret_cast<const u32x4*>(O + row * D + d), b);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += a[i] * b[i];
  }
  acc = xor_sum(xor_sum(xor_sum(acc, 1), 2), 4);
  if (sub == 0) Dq[(row / M) * ld + row % M] = acc;
}

// 16-byte row piece (8 elements from 8 * chunk) of an att_swz tile
template <int D>
__device__ __forceinline__ u32x4 row16(const char* base, int row, int chunk) {
  return *reinterpret_cast<const u32x4*>(att_chunk<D>(base, row, chunk));
}

// Transpose-read operand: lane 16g + i receives rows {r0 + 4g + e, r0 + 16 + 4g + e}
// (e = 0..3) of column 16 dt + i from an att_swz tile.
template <int D>
__device__ __forceinline__ u32x4 tr_operand(const char* base, int r0, int dt, int lane) {
  const int g = lane >> 4, e = (lane >> 2) & 3, cq = lane & 3;
  u32x4 f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = r0 + 16 * h + 4 * g + e;
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(att_chunk<D>(base, row, 2 * dt + (cq >> 1)) + (cq & 1) * 8));
    const u32x2 w2 = __builtin_bit_cast(u32x2, v);
    f[2 * h] = w2[0];
    f[2 * h + 1] = w2[1];
  }
  return f;
}

// Whether (query q, key) is masked for the dS zeroing (and the score).
__device__ __forceinline__ bool masked_entry(const AttnArgs& a, int b, int q, int key) {
  bool m = a.causal && key > q;
  if (a.mask_kind != GEV2_MASK_NONE) {
    const int64_t i = ((int64_t)b * a.M + q) * a.N + key;
    if (a.mask_kind == GEV2_MASK_I8) m |= static_cast<const int8_t*>(a.mask)[i] != 0;
    else if (a.mask_kind == GEV2_MASK_I32) m |= static_cast<const int32_t*>(a.mask)[i] != 0;
    else m |= static_cast<const float*>(a.mask)[i] != 0.f;
  }
  return m;
}

// DMA one 64-row tile of a [rows, D] tensor (rows past `limit` read as zero)
// into LDS in the att_swz layout; this wave's share.
template <int D>
__device__ __forceinline__ void load_rows(const i32x4_t& r, int64_t head_off, int row0, int limit, int wave,
                                                 int lane, uint32_t lds) {
  constexpr int kRowBytes = D * 2, kChunks = D / 8, rows_per_load = 1024 / kRowBytes;
  constexpr int loads = 64 * kRowBytes / 1024 / 4;
#pragma unroll
  for (int j = 0; j < loads; ++j) {
    const int ld = wave * loads + j;
    const int row = ld * rows_per_load + lane / kChunks;
    const int pc = lane % kChunks;
    const int c = pc ^ att_swz<D>(row);
    const int off = row0 + row < limit ? static_cast<int>(((head_off + row0 + row) * D + c * 8) * 2) : kOobOffset;
    dma16(r, off, 0, lds + ld * 1024);
  }
}

// STAGES = 2 prefetches the next query block while this one is used; STAGES = 1
// loads each block after the previous one is consumed and halves the LDS, so
// more workgroups fit per CU.
template <typename T, int D, bool MASKED, int STAGES>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(STAGES == 1 ? 3 : 1)))
attn_bwd_kv_kernel(AttnBwdArgs ba) {
  static_assert(STAGES == 1 || STAGES == 2, "one or two LDS stages");
  const AttnArgs& a = ba.f;
  constexpr int KS = D / 32, DT = D / 16, RB = D * 2, TILE = 64 * RB;
  constexpr int NL = 2 * (TILE / 1024 / 4);          // loads per wave per query block (Q and dO)
  __shared__ __attribute__((aligned(1024))) char lds[STAGES][2][TILE];
  // lse and Dq of a query block (first 256 bytes of each 1 KB load), wave 0's two extra loads
  __shared__ __attribute__((aligned(1024))) float aux[STAGES][2][256];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int kblocks = (a.N + 63) / 64;
  const int bh = blockIdx.x / kblocks, kb = blockIdx.x - bh * kblocks;
  const int b = bh / a.H;
  const int64_t qhead = (int64_t)bh * a.M, khead = (int64_t)bh * a.N;
  const int key = kb * 64 + wave * 16 + col;          // this lane's key column
  const bool key_ok = key < a.N;

  // K and V rows of this lane's key as B operands (k = d 32 ks + 8 g ..)
  u32x4 kf[KS], vf[KS];
  {
    const T* krow = static_cast<const T*>(a.K) + (khead + key) * D;
    const T* vrow = static_cast<const T*>(a.V) + (khead + key) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[ks] = key_ok ? *reinterpret_cast<const u32x4*>(krow + 32 * ks + 8 * g) : u32x4{0u, 0u, 0u, 0u};
      vf[ks] = key_ok ? *reinterpret_cast<const u32x4*>(vrow + 32 * ks + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);
  asm volatile("" ::: "memory");

  const float kLog2e = 1.4426950408889634f;
  const float xscale = a.scale * kLog2e;
  f32x4_t dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dk[dt] = dv[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nqb = (a.M + 63) / 64;
  // causal without other masks: query blocks wholly before this block's first key see none of it
  const int qb0 = (!MASKED && a.causal) ? min(nqb, (kb * 64) / 64) : 0;
  const i32x4_t rQ = rsrc_words(a.Q), rO = rsrc_words(ba.dO);
  const i32x4_t rL = rsrc_words(a.lse), rD = rsrc_words(ba.Dq);
  const uint32_t base = lds_addr(&lds[0][0][0]);
  const uint32_t abase = lds_addr(&aux[0][0][0]);
  auto q_lds = [&](int st) { return base + st * 2 * TILE; };
  auto o_lds = [&](int st) { return base + st * 2 * TILE + TILE; };
  // lse / Dq rows [q0, q0 + 64) of this head: 16 lanes x 4 floats; the arrays are padded to
  // lse_ld (a multiple of 64) rows per head, so every piece is inside them
  auto load_aux = [&](int q0, int st) {
    const int off = lane < 16 ? static_cast<int>(((int64_t)bh * a.lse_ld + q0 + 4 * lane) * 4) : kOobOffset;
    dma16(rL, off, 0, abase + st * 2048);
    dma16(rD, off, 0, abase + st * 2048 + 1024);
  };
  if (qb0 < nqb) {
    load_rows<D>(rQ, qhead, qb0 * 64, a.M, wave, lane, q_lds(0));
    load_rows<D>(rO, qhead, qb0 * 64, a.M, wave, lane, o_lds(0));
    if (wave == 0) load_aux(qb0 * 64, 0);
  }
  for (int qb = qb0; qb < nqb; ++qb) {
    const int st = STAGES == 2 ? (qb - qb0) & 1 : 0;
    if constexpr (STAGES == 2) {
      if (qb + 1 < nqb) {
        load_rows<D>(rQ, qhead, (qb + 1) * 64, a.M, wave, lane, q_lds(st ^ 1));
        load_rows<D>(rO, qhead, (qb + 1) * 64, a.M, wave, lane, o_lds(st ^ 1));
        if (wave == 0) {
          load_aux((qb + 1) * 64, st ^ 1);
          __builtin_amdgcn_s_waitcnt(0x3f70 | ((NL + 2) & 0xf) | (((NL + 2) >> 4) << 14));
        } else {
          __builtin_amdgcn_s_waitcnt(0x3f70 | (NL & 0xf) | ((NL >> 4) << 14));
        }
      } else {
        __builtin_amdgcn_s_waitcnt(0x3f70);
      }
    } else {
      // the barrier that ended the previous block's use of stage 0 is behind us
      if (qb > qb0) {
        load_rows<D>(rQ, qhead, qb * 64, a.M, wave, lane, q_lds(0));
        load_rows<D>(rO, qhead, qb * 64, a.M, wave, lane, o_lds(0));
        if (wave == 0) load_aux(qb * 64, 0);
      }
      __builtin_amdgcn_s_waitcnt(0x3f70);
    }
    __syncthreads();
    asm volatile("" ::: "memory");
    const char* ql = &lds[st][0][0];
    const char* ol = &lds[st][1][0];
    const float* lsel = &aux[st][0][0];
    const float* dql = &aux[st][1][0];
    uint32_t pw[4][2], sw[4][2];                      // P and dS of each 16-query tile, packed pairs
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f32x4_t sacc = f32x4_t{0.f, 0.f, 0.f, 0.f}, pacc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sacc = mfma_16x16x32<T>(row16<D>(ql, 16 * t + col, 4 * ks + g), kf[ks], sacc);
        pacc = mfma_16x16x32<T>(row16<D>(ol, 16 * t + col, 4 * ks + g), vf[ks], pacc);
      }
      float p[4], ds[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = qb * 64 + 16 * t + 4 * g + r;   // row of this accumulator entry
        const bool q_ok = q < a.M;
        // rows past M hold padding (never-written lse / Dq): their P and dS are set to 0 outright
        const float lse2 = lsel[16 * t + 4 * g + r] * kLog2e;
        const float dq = dql[16 * t + 4 * g + r];
        float pv;
        if constexpr (MASKED) {
          // dropout (masked variant only): dV takes the kept probabilities, dP
          // the kept gradient (launcher.cu:454-590 regenerates the forward's mask)
          const bool in = key_ok && q_ok;
          const float keep = a.drop && in ? drop_factor(a, bh, q, key) : 1.f;
          const float x = in ? mask_add(sacc[r] * a.scale, a, b, q, key) * kLog2e : 0.f;
          pv = in ? __builtin_amdgcn_exp2f(x - lse2) : 0.f;
          const bool m = in ? masked_entry(a, b, q, key) : true;
          ds[r] = m ? 0.f : pv * (pacc[r] * keep - dq);
          pv *= keep;
        } else {
          const bool live = key_ok && q_ok && !(a.causal && key > q);
          pv = live ? __builtin_amdgcn_exp2f(fmaf(sacc[r], xscale, -lse2)) : 0.f;
          ds[r] = live ? pv * (pacc[r] - dq) : 0.f;
        }
        p[r] = pv;
      }
      pw[t][0] = pack2(Elem<T>::bits(p[0]), Elem<T>::bits(p[1]));
      pw[t][1] = pack2(Elem<T>::bits(p[2]), Elem<T>::bits(p[3]));
      sw[t][0] = pack2(Elem<T>::bits(ds[0]), Elem<T>::bits(ds[1]));
      sw[t][1] = pack2(Elem<T>::bits(ds[2]), Elem<T>::bits(ds[3]));
    }
    // dV^T[d][key] += dO^T P ; dK^T[d][key] += Q^T dS  (queries 32 i + {4g + e, 16 + 4g + e})
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4 pb = {pw[2 * i][0], pw[2 * i][1], pw[2 * i + 1][0], pw[2 * i + 1][1]};
      const u32x4 sb = {sw[2 * i][0], sw[2 * i][1], sw[2 * i + 1][0], sw[2 * i + 1][1]};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dv[dt] = mfma_16x16x32<T>(tr_operand<D>(ol, 32 * i, dt, lane), pb, dv[dt]);
        dk[dt] = mfma_16x16x32<T>(tr_operand<D>(ql, 32 * i, dt, lane), sb, dk[dt]);
      }
    }
    __syncthreads();
  }
  if (!key_ok) return;
  T* dkr = static_cast<T*>(ba.dK) + (khead + key) * D;
  T* dvr = static_cast<T*>(ba.dV) + (khead + key) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    if (ba.dK) {
      u32x2 w;
      w[0] = pack2(Elem<T>::bits(dk[dt][0] * a.scale), Elem<T>::bits(dk[dt][1] * a.scale));
      w[1] = pack2(Elem<T>::bits(dk[dt][2] * a.scale), Elem<T>::bits(dk[dt][3] * a.scale));
      *reinterpret_cast<u32x2*>(dkr + 16 * dt + 4 * g) = w;
    }
    if (ba.dV) {
      u32x2 w;
      w[0] = pack2(Elem<T>::bits(dv[dt][0]), Elem<T>::bits(dv[dt][1]));
      w[1] = pack2(Elem<T>::bits(dv[dt][2]), Elem<T>::bits(dv[dt][3]));
      *reinterpret_cast<u32x2*>(dvr + 16 * dt + 4 * g) = w;
    }
  }
}

// STAGES as in attn_bwd_kv_kernel: 2 prefetches the next key block, 1 halves the LDS
template <typename T, int D, bool MASKED, int STAGES>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(STAGES == 1 ? 3 : 1)))
attn_bwd_q_kernel(AttnBwdArgs ba) {
  static_assert(STAGES == 1 || STAGES == 2, "one or two LDS stages");
  const AttnArgs& a = ba.f;
  constexpr int KS = D / 32, DT = D / 16, RB = D * 2, TILE = 64 * RB;
  constexpr int NL = 2 * (TILE / 1024 / 4);
  __shared__ __attribute__((aligned(1024))) char lds[STAGES][2][TILE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int qblocks = (a.M + 63) / 64;
  const int bh = blockIdx.x / qblocks, qb = blockIdx.x - bh * qblocks;
  const int b = bh / a.H;
  const int64_t qhead = (int64_t)bh * a.M, khead = (int64_t)bh * a.N;
  const int q = qb * 64 + wave * 16 + col;            // this lane's query column
  const bool q_ok = q < a.M;

  u32x4 qf[KS], of[KS];
  {
    const T* qrow = static_cast<const T*>(a.Q) + (qhead + q) * D;
    const T* orow = static_cast<const T*>(ba.dO) + (qhead + q) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = q_ok ? *reinterpret_cast<const u32x4*>(qrow + 32 * ks + 8 * g) : u32x4{0u, 0u, 0u, 0u};
      of[ks] = q_ok ? *reinterpret_cast<const u32x4*>(orow + 32 * ks + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const float kLog2e = 1.4426950408889634f;
  const float xscale = a.scale * kLog2e;
  const float lse2 = q_ok ? a.lse[(int64_t)bh * a.lse_ld + q] * kLog2e : INFINITY;
  const float dq = q_ok ? ba.Dq[(int64_t)bh * a.lse_ld + q] : 0.f;
  __builtin_amdgcn_s_waitcnt(0x3f70);
  asm volatile("" ::: "memory");

  f32x4_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int nkb = (a.N + 63) / 64;
  if (!MASKED && a.causal) nkb = min(nkb, (qb * 64 + 63) / 64 + 1);
  const i32x4_t rK = rsrc_words(a.K), rV = rsrc_words(a.V);
  const uint32_t base = lds_addr(&lds[0][0][0]);
  auto k_lds = [&](int st) { return base + st * 2 * TILE; };
  auto v_lds = [&](int st) { return base + st * 2 * TILE + TILE; };
  load_rows<D>(rK, khead, 0, a.N, wave, lane, k_lds(0));
  load_rows<D>(rV, khead, 0, a.N, wave, lane, v_lds(0));
  for (int kb = 0; kb < nkb; ++kb) {
    const int st = STAGES == 2 ? kb & 1 : 0;
    if constexpr (STAGES == 2) {
      if (kb + 1 < nkb) {
        load_rows<D>(rK, khead, (kb + 1) * 64, a.N, wave, lane, k_lds(st ^ 1));
        load_rows<D>(rV, khead, (kb + 1) * 64, a.N, wave, lane, v_lds(st ^ 1));
        __builtin_amdgcn_s_waitcnt(0x3f70 | (NL & 0xf) | ((NL >> 4) << 14));
      } else {
        __builtin_amdgcn_s_waitcnt(0x3f70);
      }
    } else {
      // the barrier that ended the previous block's use of stage 0 is behind us
      if (kb > 0) {
        load_rows<D>(rK, khead, kb * 64, a.N, wave, lane, k_lds(0));
        load_rows<D>(rV, khead, kb * 64, a.N, wave, lane, v_lds(0));
      }
      __builtin_amdgcn_s_waitcnt(0x3f70);
    }
    __syncthreads();
    asm volatile("" ::: "memory");
    const char* kl = &lds[st][0][0];
    const char* vl = &lds[st][1][0];
    uint32_t sw[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4_t sacc = f32x4_t{0.f, 0.f, 0.f, 0.f}, pacc = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const int row = 16 * kt + col;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sacc = mfma_16x16x32<T>(row16<D>(kl, row, 4 * ks + g), qf[ks], sacc);
        pacc = mfma_16x16x32<T>(row16<D>(vl, row, 4 * ks + g), of[ks], pacc);
      }
      float ds[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb * 64 + 16 * kt + 4 * g + r;
        const bool key_ok = key < a.N;
        if constexpr (MASKED) {
          const bool in = key_ok && q_ok;
          const float dp = a.drop && in ? pacc[r] * drop_factor(a, bh, q, key) : pacc[r];
          const float x = in ? mask_add(sacc[r] * a.scale, a, b, q, key) * kLog2e : 0.f;
          const float pv = in ? __builtin_amdgcn_exp2f(x - lse2) : 0.f;
          const bool m = in ? masked_entry(a, b, q, key) : true;
          ds[r] = m ? 0.f : pv * (dp - dq);
        } else {
          const bool live = key_ok && q_ok && !(a.causal && key > q);
          const float pv = live ? __builtin_amdgcn_exp2f(fmaf(sacc[r], xscale, -lse2)) : 0.f;
          ds[r] = live ? pv * (pacc[r] - dq) : 0.f;
        }
      }
      sw[kt][0] = pack2(Elem<T>::bits(ds[0]), Elem<T>::bits(ds[1]));
      sw[kt][1] = pack2(Elem<T>::bits(ds[2]), Elem<T>::bits(ds[3]));
    }
    // dQ^T[d][q] += K^T[d][key] dS^T[key][q]  (keys 32 j + {4g + e, 16 + 4g + e})
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 sb = {sw[2 * j][0], sw[2 * j][1], sw[2 * j + 1][0], sw[2 * j + 1][1]};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma_16x16x32<T>(tr_operand<D>(kl, 32 * j, dt, lane), sb, acc[dt]);
    }
    __syncthreads();
  }
  if (!q_ok) return;
  T* dqr = static_cast<T*>(ba.dQ) + (qhead + q) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    u32x2 w;
    w[0] = pack2(Elem<T>::bits(acc[dt][0] * a.scale), Elem<T>::bits(acc[dt][1] * a.scale));
    w[1] = pack2(Elem<T>::bits(acc[dt][2] * a.scale), Elem<T>::bits(acc[dt][3] * a.scale));
    *reinterpret_cast<u32x2*>(dqr + 16 * dt + 4 * g) = w;
  }
}

template <typename T, int D>
hipError_t launch_attn_bwd(const AttnBwdArgs& ba, hipStream_t s) {
  const AttnArgs& a = ba.f;
  const int64_t rows = (int64_t)a.BH * a.M;
  hipLaunchKernelGGL((attn_bwd_dot_kernel<T>), dim3(static_cast<unsigned>((rows + 31) / 32)), dim3(256), 0, s,
                     static_cast<const T*>(ba.dO), static_cast<const T*>(a.Y), const_cast<float*>(ba.Dq), rows, D,
                     a.M, a.lse_ld);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const bool masked = a.mask_kind != GEV2_MASK_NONE || !(a.scale > 0.f) || a.drop;
  if (ba.dK || ba.dV) {
    const dim3 grid(static_cast<unsigned>((int64_t)a.BH * ((a.N + 63) / 64)));
    // one LDS stage at D = 128 (3 waves per SIMD instead of 2: 582 -> 574 us at B 2, H 16,
    // M = N = 2048); at D = 64 both are equal (59.4 / 59.3 us at B 8, H 8, M = N = 512)
    constexpr bool one = D == 128;
    if (masked) {
      hipLaunchKernelGGL((attn_bwd_kv_kernel<T, D, true, one ? 1 : 2>), grid, dim3(256), 0, s, ba);
    } else {
      hipLaunchKernelGGL((attn_bwd_kv_kernel<T, D, false, one ? 1 : 2>), grid, dim3(256), 0, s, ba);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (ba.dQ) {
    const dim3 grid(static_cast<unsigned>((int64_t)a.BH * ((a.M + 63) / 64)));
    // one LDS stage at D = 128 (4 waves per SIMD instead of 2: 559 -> 539 us at B 2, H 16,
    // M = N = 2048); at D = 64 both are equal (60.1 / 60.4 us at B 8, H 8, M = N = 512)
    constexpr bool one = D == 128;
    if (masked) {
      hipLaunchKernelGGL((attn_bwd_q_kernel<T, D, true, one ? 1 : 2>), grid, dim3(256), 0, s, ba);
    } else {
      hipLaunchKernelGGL((attn_bwd_q_kernel<T, D, false, one ? 1 : 2>), grid, dim3(256), 0, s, ba);
    }
    e = hipGetLastError();
  }
  return e;
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
  if (!(d->dropout_p >= 0.f && d->dropout_p <= 1.f)) return attn_fail(GEV2_INVALID_ARGUMENT, "dropout_p must be in [0, 1]");
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
  a->drop = d->dropout_p > 0.f ? 1 : 0;
  a->drop_p = d->dropout_p;
  // dropout/kernels.cu:43-47: kept values scaled by 1/(1-p) when scale_in_train and 1-p > 0
  a->drop_scale = (d->scale_in_train && (1.0f - d->dropout_p) > 0.f) ? 1.0f / (1.0f - d->dropout_p) : 1.0f;
  a->seed = d->seed;
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

int64_t align256(int64_t n) { return ((n + 255) / 256) * 256; }

// fused 16-bit backward: O [BH, M, D] (16-bit), lse and Dq [BH, Mp] fp32 with
// Mp = M rounded up to 64 (whole 64-row pieces per head)
int64_t padded_rows(int64_t M) { return (M + 63) / 64 * 64; }
int64_t fused_bwd_bytes(int64_t BH, int64_t M, int64_t D) {
  return align256(BH * M * D * 2) + 2 * align256(BH * padded_rows(M) * 4);
}

// the fused backward unless GEV2_ATTN_BWD_WIDE=1 (comparison runs)
bool fused_bwd(int dtype, int D) {
  if (!fused_ok(dtype, D)) return false;
  const char* v = std::getenv("GEV2_ATTN_BWD_WIDE");
  return !(v && v[0] == '1');
}

int64_t gev2_sdpa_workspace_size(const gev2_sdpa_desc* d, int backward) {
  gev2::AttnArgs a{};
  if (attn_check(d, &a) != GEV2_OK) return -1;
  if (fused_ok(d->dtype, d->D) && !backward) return 0;
  if (!backward) return scores_bytes(a.BH, d->M, d->N);
  if (fused_bwd(d->dtype, d->D)) return fused_bwd_bytes(a.BH, d->M, d->D);
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
  a.Q = d->Q; a.K = d->K; a.V = d->V; a.Y = d->Y; a.lse = d->lse; a.lse_ld = d->M;
  const int64_t M = d->M, N = d->N, D = d->D;
  if (fused_ok(d->dtype, d->D)) {
    for (const void* p : {d->Q, d->K, d->V, static_cast<const void*>(d->Y)})
      if (reinterpret_cast<uintptr_t>(p) % 16) return attn_fail(GEV2_INVALID, "fused path needs 16-byte aligned tensors");
    if (a.BH * N * D * 2 > 0x7fffff00LL) return attn_fail(GEV2_INVALID, "fused path needs K / V under 2^31 bytes");
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
  if (a.drop) {
    hipLaunchKernelGGL(gev2::attn_dropout_kernel, dim3(4096), dim3(256), 0, s, S, S, a);
    st = hip_status(hipGetLastError(), "dropout");
    if (st != GEV2_OK) return st;
  }
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
  if (fused_bwd(d->dtype, d->D)) {
    // recompute O and lse with the fused forward, Dq = rowsum(dO O), then the dK/dV and dQ kernels
    if (!d->workspace || d->workspace_bytes < fused_bwd_bytes(BH, M, D))
      return attn_fail(GEV2_MISSING_INPUT, "backward needs a workspace of gev2_sdpa_workspace_size(desc, 1) bytes");
    for (const void* p : {d->Q, d->K, d->V, d->dY, static_cast<const void*>(d->dQ), static_cast<const void*>(d->dK),
                          static_cast<const void*>(d->dV)})
      if (reinterpret_cast<uintptr_t>(p) % 16) return attn_fail(GEV2_INVALID, "fused path needs 16-byte aligned tensors");
    if (BH * M * D * 2 > 0x7fffff00LL || BH * N * D * 2 > 0x7fffff00LL)
      return attn_fail(GEV2_INVALID, "fused path needs Q / K / V / dY under 2^31 bytes");
    char* w = static_cast<char*>(d->workspace);
    void* O = w;
    const int64_t Mp = padded_rows(M);
    float* lse = reinterpret_cast<float*>(w + align256(BH * M * D * 2));
    float* Dq = reinterpret_cast<float*>(w + align256(BH * M * D * 2) + align256(BH * Mp * 4));
    gev2::AttnArgs fa = a;
    fa.Q = d->Q; fa.K = d->K; fa.V = d->V; fa.Y = O; fa.lse = lse; fa.lse_ld = static_cast<int>(Mp);
    hipError_t e;
    if (d->dtype == GEV2_BF16) e = D == 64 ? gev2::launch_attn_fwd<__bf16, 64>(fa, s) : gev2::launch_attn_fwd<__bf16, 128>(fa, s);
    else e = D == 64 ? gev2::launch_attn_fwd<_Float16, 64>(fa, s) : gev2::launch_attn_fwd<_Float16, 128>(fa, s);
    st = hip_status(e, "attn_fwd (backward)");
    if (st != GEV2_OK) return st;
    gev2::AttnBwdArgs ba{};
    ba.f = fa;
    ba.dO = d->dY; ba.Dq = Dq; ba.dQ = d->dQ; ba.dK = d->dK; ba.dV = d->dV;
    if (d->dtype == GEV2_BF16) e = D == 64 ? gev2::launch_attn_bwd<__bf16, 64>(ba, s) : gev2::launch_attn_bwd<__bf16, 128>(ba, s);
    else e = D == 64 ? gev2::launch_attn_bwd<_Float16, 64>(ba, s) : gev2::launch_attn_bwd<_Float16, 128>(ba, s);
    return hip_status(e, "attn_bwd");
  }
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
  // dV = P^T dY, with the dropped P (in the dP buffer, free until dP below) under dropout
  if (d->dV) {
    const float* Pv = P;
    if (a.drop) {
      hipLaunchKernelGGL(gev2::attn_dropout_kernel, dim3(4096), dim3(256), 0, s, P, dP, a);
      st = hip_status(hipGetLastError(), "dropout");
      if (st != GEV2_OK) return st;
      Pv = dP;
    }
    st = slice_gemm(GEV2_F32, true, false, 1.f, BH, N, D, M, Pv, N, M * N, d->dY, D, M * D, d->dV, D, N * D, stream);
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
