// MFMA tile GEMM for gfx950 with fused bias/activation epilogue, optional
// act'-prologue on one operand and fused column sums (dBias).
//
// One kernel template serves the three operand layouts the operator needs:
//   forward   Y  = act(X W + b)      A = X  [M,K] (K-contig), B = W [K,N] (N-contig)
//   dX        gA = dY' W^T           A = dY'[M,N] (K-contig), B = W as [N,K] (K-contig)
//   dW        gB = X^T dY'           A = X as [K,M] (M-contig), B = dY' [M,N] (N-contig)
// plus the batched/strided SDPA and conv forms.  The reference computes the
// forward with an FFMA register-tiled kernel (regemm_gemm_bias_act.cu:254-395)
// and the backward with an element-wise act' pass plus two SGEMMs
// (regemm_backward.cu:91-130,271-291); here dY' is never materialised.
//
// Data path per K-tile (BK = 128 bytes of K):
//   global -> registers: 16-byte loads.  An operand that is contiguous along
//     M/N is loaded as EPCxEPC blocks (EPC = elements per 16 bytes) and
//     transposed in registers so LDS always holds K-contiguous rows.
//   registers -> LDS: rows of 8 chunks, chunk index XOR-swizzled with
//     (row & 7) ^ ((row >> 3) & 7) so that any 8 consecutive lanes of a store
//     or of an MFMA fragment read touch 8 different 16-byte bank groups.
//   LDS -> MFMA: v_mfma_f32_32x32x16_{bf16,f16} (one 16-byte fragment per
//     lane) or v_mfma_f32_32x32x2_f32 (four per fragment).  The W/B fragment
//     is passed as src0 so that each lane's accumulators hold 4 consecutive
//     N columns of one M row, which makes the epilogue store 4-wide.
// Two LDS buffers; the global loads for tile k+1 are issued before the MFMAs
// of tile k, one barrier per K-tile.
#pragma once
#include "gev2_device.hpp"
#include "gev2_kernels.hpp"

namespace gev2 {

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 7); }

// Map a linear workgroup id to a (tile_m, tile_n) pair.  Workgroups are
// dispatched round-robin over the 8 XCDs; remapping gives each XCD a
// contiguous range of tiles, and the group-of-4 row ordering keeps the tiles
// an XCD owns compact so its L2 sees A-row and B-column reuse.
__device__ __forceinline__ void map_tile(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  constexpr int GM = 4;
  const int width = GM * tiles_n;
  const int group = pid / width;
  const int first = group * GM;
  const int gsz = min(tiles_m - first, GM);
  const int r = pid - group * width;
  tm = first + r % gsz;
  tn = r / gsz;
}

// Staging of one operand tile: ROWS x BK elements, ROWS along M (or N).
// MNC: the operand is contiguous along M/N in memory (needs the transpose).
template <typename T, int ROWS, bool MNC, int NT, bool VEC>
struct Stage {
  static constexpr int EPC = Elem<T>::kPerChunk;
  static constexpr int NBLK = (ROWS / EPC) * 8;                 // EPC x EPC blocks per tile
  static constexpr int BPT = (NBLK + NT - 1) / NT;              // blocks per thread (MNC)
  static constexpr int LPT = MNC ? BPT * EPC : (ROWS * 8) / NT; // 16-byte loads per thread
  static_assert(MNC || (ROWS * 8) % NT == 0, "tile rows must cover the workgroup");
  u32x4 r[LPT];

  __device__ __forceinline__ static u32x4 load_chunk(const T* p, bool row_ok, int lim_left) {
    // lim_left = number of valid elements from p along the contiguous dim
    if constexpr (VEC) {
      if (row_ok && lim_left > 0) return *reinterpret_cast<const u32x4*>(p);
      return u32x4{0, 0, 0, 0};
    } else {
      float v[EPC];
#pragma unroll
      for (int e = 0; e < EPC; ++e) v[e] = (row_ok && e < lim_left) ? Elem<T>::load1(p + e) : 0.f;
      return f32_to_chunk<T>(v);
    }
  }

  // base: slice origin; (mn0, k0): tile origin; MNlim/Klim: matrix extents.
  __device__ __forceinline__ void load(const T* base, int64_t ld, int mn0, int k0, int MNlim,
                                       int Klim, int tid) {
    if constexpr (!MNC) {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int c = tid + i * NT;
        const int mn = mn0 + (c >> 3);
        const int k = k0 + (c & 7) * EPC;
        const bool ok = mn < MNlim;
        const T* p = base + (ok ? (int64_t)mn * ld + k : 0);
        r[i] = load_chunk(p, ok, Klim - k);
      }
    } else {
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int b = tid + bi * NT;
        const int bc = b % (ROWS / EPC), br = b / (ROWS / EPC);
        const int mn = mn0 + bc * EPC;
#pragma unroll
        for (int j = 0; j < EPC; ++j) {
          const int k = k0 + br * EPC + j;
          const bool ok = (NBLK % NT == 0 || b < NBLK) && k < Klim;
          const T* p = base + (ok ? (int64_t)k * ld + mn : 0);
          r[bi * EPC + j] = load_chunk(p, ok, MNlim - mn);
        }
      }
    }
  }

  // dY' = dY * act'(Z) on the staged registers; for MNC operands also add the
  // column sums (over K rows) into colsum[BPT][EPC].
  template <int ACT, bool SUMS>
  __device__ __forceinline__ void prologue(const Stage& z, float slope, float (*colsum)[EPC]) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      float g[EPC], zz[EPC];
      chunk_to_f32<T>(r[i], g);
      chunk_to_f32<T>(z.r[i], zz);
#pragma unroll
      for (int e = 0; e < EPC; ++e) g[e] *= act_grad_t<ACT>(zz[e], slope);
      if constexpr (SUMS && MNC) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) colsum[i / EPC][e] += g[e];
      }
      r[i] = f32_to_chunk<T>(g);
    }
  }

  __device__ __forceinline__ void store(u32x4* lds, int tid) const {
    if constexpr (!MNC) {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int c = tid + i * NT;
        const int row = c >> 3;
        lds[row * 8 + ((c & 7) ^ swz(row))] = r[i];
      }
    } else {
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int b = tid + bi * NT;
        if (NBLK % NT != 0 && b >= NBLK) continue;
        const int bc = b % (ROWS / EPC), br = b / (ROWS / EPC);
        const u32x4* in = r + bi * EPC;
        if constexpr (EPC == 8) {
          // 8x8 transpose of 16-bit elements: out[e] word j = (in[2j][e], in[2j+1][e])
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            u32x4 t;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t lo = in[2 * j][e >> 1], hi = in[2 * j + 1][e >> 1];
              t[j] = (e & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
            }
            const int row = bc * 8 + e;
            lds[row * 8 + (br ^ swz(row))] = t;
          }
        } else {
          // 4x4 transpose of fp32
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u32x4 t = {in[0][e], in[1][e], in[2][e], in[3][e]};
            const int row = bc * 4 + e;
            lds[row * 8 + (br ^ swz(row))] = t;
          }
        }
      }
    }
  }
};

template <typename T>
__device__ __forceinline__ void mfma_step(f32x16_t& acc, const u32x4& a, const u32x4& b) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(b[j]), __uint_as_float(a[j]), acc, 0, 0, 0);
  } else if constexpr (__is_same(T, __bf16)) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, b),
                                                  __builtin_bit_cast(bf16x8_t, a), acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, b),
                                                 __builtin_bit_cast(f16x8_t, a), acc, 0, 0, 0);
  }
}

// Store 4 consecutive values of row m starting at column n.
template <typename T>
__device__ __forceinline__ void store4(T* row, int n, int N, const float* v, bool vec) {
  if (vec && n + 3 < N) {
    if constexpr (sizeof(T) == 4) {
      *reinterpret_cast<f32x4_t*>(row + n) = f32x4_t{v[0], v[1], v[2], v[3]};
    } else {
      const u32x2 w = {Elem<T>::bits(v[0]) | (Elem<T>::bits(v[1]) << 16),
                       Elem<T>::bits(v[2]) | (Elem<T>::bits(v[3]) << 16)};
      *reinterpret_cast<u32x2*>(row + n) = w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < N) Elem<T>::store1(row + n + i, v[i]);
  }
}

// PRO: 0 none, 1 prologue on A, 2 prologue on B (+ fused column sums when B is N-contig).
template <typename T, int BM, int BN, int WM, int WN, bool TA, bool TB, int PRO, bool VEC>
__global__ void __launch_bounds__(WM * WN * 64)
gemm_tile_kernel(TileArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int EPC = Elem<T>::kPerChunk;
  constexpr int BK = 8 * EPC;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  static_assert(FM >= 1 && FN >= 1, "wave tile must be a multiple of 32");
  using SA = Stage<T, BM, TA, NT, VEC>;
  using SB = Stage<T, BN, !TB, NT, VEC>;
  constexpr bool kSums = (PRO == 2) && !TB;

  __shared__ u32x4 lds[2 * (BM + BN) * 8];
  u32x4* As = lds;
  u32x4* Bs = lds + 2 * BM * 8;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  int tm, tn;
  map_tile(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int bz = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;

  const T* Ab = reinterpret_cast<const T*>(p.A) + (int64_t)bz * p.sA;
  const T* Bb = reinterpret_cast<const T*>(p.B) + (int64_t)bz * p.sB;
  const T* Zb = reinterpret_cast<const T*>(p.Zi) + (int64_t)bz * p.sZi;

  SA sa;
  SB sb;
  SA za;  // prologue Z for A (PRO == 1)
  SB zb;  // prologue Z for B (PRO == 2)
  float colsum[SB::BPT][EPC];
  if constexpr (kSums) {
#pragma unroll
    for (int i = 0; i < SB::BPT; ++i)
#pragma unroll
      for (int e = 0; e < EPC; ++e) colsum[i][e] = 0.f;
  }
  const bool do_sums = kSums && p.dbias != nullptr && tm == 0;

  // A is [M,K] (K-contig) or [K,M] (M-contig); B is [K,N] (N-contig) or [N,K] (K-contig).
  auto load_tile = [&](int k0) __attribute__((always_inline)) {
    sa.load(Ab, p.lda, m0, k0, p.M, p.K, tid);
    sb.load(Bb, p.ldb, n0, k0, p.N, p.K, tid);
    if constexpr (PRO == 1) za.load(Zb, p.ldzi, m0, k0, p.M, p.K, tid);
    if constexpr (PRO == 2) zb.load(Zb, p.ldzi, n0, k0, p.N, p.K, tid);
  };
  auto stage_tile = [&](int buf) __attribute__((always_inline)) {
    if constexpr (PRO == 1)
      dispatch_act(p.pro_act, [&]<int ACT>() __attribute__((always_inline)) { sa.template prologue<ACT, false>(za, p.slope, nullptr); });
    if constexpr (PRO == 2) {
      if (do_sums)
        dispatch_act(p.pro_act, [&]<int ACT>() __attribute__((always_inline)) { sb.template prologue<ACT, kSums>(zb, p.slope, colsum); });
      else
        dispatch_act(p.pro_act, [&]<int ACT>() __attribute__((always_inline)) { sb.template prologue<ACT, false>(zb, p.slope, nullptr); });
    }
    sa.store(As + buf * BM * 8, tid);
    sb.store(Bs + buf * BN * 8, tid);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int KT = (p.K + BK - 1) / BK;
  if (KT > 0) {
    load_tile(0);
    stage_tile(0);
  }
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) load_tile((kt + 1) * BK);
    const u32x4* Ac = As + cur * BM * 8;
    const u32x4* Bc = Bs + cur * BN * 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ch = 2 * q + (lane >> 5);
      u32x4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * WTM + i * 32 + (lane & 31);
        af[i] = Ac[row * 8 + (ch ^ swz(row))];
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * WTN + j * 32 + (lane & 31);
        bfr[j] = Bc[row * 8 + (ch ^ swz(row))];
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mfma_step<T>(acc[i][j], af[i], bfr[j]);
    }
    if (more) stage_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- fused dBias: column sums of dY' over all M (workgroups of tile row 0) ----
  if constexpr (kSums) {
    if (do_sums) {
      float* red = reinterpret_cast<float*>(lds);  // [8][BN]
#pragma unroll
      for (int bi = 0; bi < SB::BPT; ++bi) {
        const int b = tid + bi * NT;
        if (SB::NBLK % NT != 0 && b >= SB::NBLK) continue;
        const int bc = b % (BN / EPC), br = b / (BN / EPC);
#pragma unroll
        for (int e = 0; e < EPC; ++e) red[br * BN + bc * EPC + e] = colsum[bi][e];
      }
      __syncthreads();
      for (int c = tid; c < BN; c += NT) {
        float s = 0.f;
#pragma unroll
        for (int br = 0; br < 8; ++br) s += red[br * BN + c];
        const int n = n0 + c;
        if (n < p.N) p.dbias[(int64_t)bz * p.sDbias + n] = s;
      }
    }
  }

  // ---- epilogue: pre = alpha*acc + bias; Z = pre; D = act(pre) ----
  T* Db = reinterpret_cast<T*>(p.D) + (int64_t)bz * p.sD;
  T* Zob = p.Zo ? reinterpret_cast<T*>(p.Zo) + (int64_t)bz * p.sZo : nullptr;
  const float* biasb = p.bias ? p.bias + (int64_t)bz * p.sBias : nullptr;
  const int bk = biasb ? p.bias_kind : kBiasNone;
  const bool vec = p.store_vec != 0;
  const float alpha = p.alpha;
  dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * WTM + i * 32 + (lane & 31);
      if (m >= p.M) continue;
      T* drow = Db + (int64_t)m * p.ldd;
      T* zrow = Zob ? Zob + (int64_t)m * p.ldzo : nullptr;
      const float brow = bk == kBiasPerM ? biasb[m] : bk == kBiasScalar ? biasb[0] : 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + wn * WTN + j * 32 + q * 8 + (lane >> 5) * 4;
          if (n >= p.N) continue;
          float pre[4], y[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float v = acc[i][j][q * 4 + t];
            if (alpha != 1.f) v = alpha * v;
            v += bk == kBiasPerN ? biasb[min(n + t, p.N - 1)] : brow;
            pre[t] = v;
            y[t] = act_fwd_t<ACT>(v, p.slope);
          }
          if (zrow) store4<T>(zrow, n, p.N, pre, vec);
          store4<T>(drow, n, p.N, y, vec);
        }
      }
    }
  });
}

// ---------------------------------------------------------------------------
// Host-side launch (instantiation table)
// ---------------------------------------------------------------------------
template <int CFG> struct CfgShape;
template <> struct CfgShape<kCfg256x256> { static constexpr int BM = 256, BN = 256, WM = 2, WN = 4; };
template <> struct CfgShape<kCfg128x128> { static constexpr int BM = 128, BN = 128, WM = 2, WN = 2; };
template <> struct CfgShape<kCfg64x64> { static constexpr int BM = 64, BN = 64, WM = 2, WN = 2; };
template <> struct CfgShape<kCfg128x256> { static constexpr int BM = 128, BN = 256, WM = 2, WN = 2; };

template <typename T, int CFG, bool TA, bool TB, int PRO, bool VEC>
static hipError_t launch_one(const TileArgs& a, int batch, hipStream_t s) {
  using C = CfgShape<CFG>;
  dim3 grid(a.tiles_m * a.tiles_n, batch);
  dim3 block(C::WM * C::WN * 64);
  hipLaunchKernelGGL((gemm_tile_kernel<T, C::BM, C::BN, C::WM, C::WN, TA, TB, PRO, VEC>), grid,
                     block, 0, s, a);
  return hipGetLastError();
}

// Layout combos in use: NN (forward, conv, P.V), NT (dX, QK^T), TN (dW, SDPA dV/dK).
template <typename T, int CFG, bool VEC>
static hipError_t launch_layout(bool ta, bool tb, int pro, const TileArgs& a, int batch,
                                hipStream_t s) {
  if (!ta && !tb && pro == 0) return launch_one<T, CFG, false, false, 0, VEC>(a, batch, s);
  if (!ta && tb && pro == 0) return launch_one<T, CFG, false, true, 0, VEC>(a, batch, s);
  if (!ta && tb && pro == 1) return launch_one<T, CFG, false, true, 1, VEC>(a, batch, s);
  if (ta && !tb && pro == 0) return launch_one<T, CFG, true, false, 0, VEC>(a, batch, s);
  if (ta && !tb && pro == 2) return launch_one<T, CFG, true, false, 2, VEC>(a, batch, s);
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t launch_cfg(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                             int batch, hipStream_t s) {
  if (!vec) return launch_layout<T, kCfg64x64, false>(ta, tb, pro, a, batch, s);
  switch (cfg) {
    case kCfg128x128: return launch_layout<T, kCfg128x128, true>(ta, tb, pro, a, batch, s);
    case kCfg64x64: return launch_layout<T, kCfg64x64, true>(ta, tb, pro, a, batch, s);
    case kCfg128x256: return launch_layout<T, kCfg128x256, true>(ta, tb, pro, a, batch, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
