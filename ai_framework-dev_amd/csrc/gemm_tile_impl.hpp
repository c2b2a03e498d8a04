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
__device__ __forceinline__ void map_tile_grouped(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GM = 4;
  const int width = GM * tiles_n;
  const int group = pid / width;
  const int first = group * GM;
  const int gsz = min(tiles_m - first, GM);
  const int r = pid - group * width;
  tm = first + r % gsz;
  tn = r / gsz;
}

__device__ __forceinline__ void map_tile(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  map_tile_grouped(pid, tiles_m, tiles_n, tm, tn);
}

// Tile and batch slice of this workgroup in a (tiles, batch) grid.  The
// dispatcher hands workgroups to the 8 XCDs in turn by flattened id (x
// fastest), so the tiles of one slice would sit on different XCDs and each
// fetch the slice's shared operand rows past its own L2.  When the grid's
// workgroup count is a multiple of 8, each XCD instead takes a contiguous run
// of (slice, tile) items: e.g. the 5 dW tiles of one image of a 3x3
// convolution's backward (128 x 576 x 3136 per image) read that image's dY'
// rows through one L2.  One-slice grids keep map_tile's spread.
__device__ __forceinline__ void map_tile_batched(int tiles_m, int tiles_n, int& tm, int& tn, int& bz) {
  const int tiles = tiles_m * tiles_n;           // == gridDim.x
  const int total = tiles * static_cast<int>(gridDim.y);
  if (gridDim.y > 1 && (total & 7) == 0) {
    const int L = static_cast<int>(blockIdx.x) + static_cast<int>(blockIdx.y) * tiles;
    const int g = (L & 7) * (total >> 3) + (L >> 3);
    bz = g / tiles;
    map_tile_grouped(g - bz * tiles, tiles_m, tiles_n, tm, tn);
  } else {
    bz = blockIdx.y;
    map_tile(blockIdx.x, tiles_m, tiles_n, tm, tn);
  }
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

  __device__ __forceinline__ void store(u32x4* lds, int tid) const { store_regs(r, lds, tid); }

  __device__ __forceinline__ static void store_regs(const u32x4 (&r)[LPT], u32x4* lds, int tid) {
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
// Pipelined kernel for the vector path (16-byte aligned operands).
//
// Differences from gemm_tile_kernel above:
//   - global loads are raw buffer loads with no branches: a chunk outside the
//     matrix gets an offset beyond the buffer's range and reads as zero;
//   - the K loop is software-pipelined: fragments for k16 step q+1 are read
//     from LDS while the MFMAs of step q run, the next K tile's global loads
//     are in flight during the whole tile, and its LDS stores (with the
//     transpose and the act' prologue) are issued between the MFMAs of steps
//     1 and 2 into the other LDS buffer; one barrier per K tile;
//   - the backward's epilogue (PRO != 0) is compiled for act = none only.
// ---------------------------------------------------------------------------

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  // range 2^31 - 1 bytes: every valid offset is below it (checked by the
  // host), kOobOffset + any tile offset is not.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), 0x7fffffff,
                                           0x00020000);
}

// Staging of one operand tile (ROWS x BK elements) through registers with raw
// buffer loads.  The per-thread part of each chunk's byte offset is computed
// once (rows outside the matrix fold to kOobOffset); a K tile adds its k0 term.
template <typename T, int ROWS, bool MNC, int NT>
struct PipeStage {
  static constexpr int EPC = Elem<T>::kPerChunk;
  static constexpr int ES = sizeof(T);
  static constexpr int NBLK = (ROWS / EPC) * 8;
  static constexpr int BPT = (NBLK + NT - 1) / NT;
  static constexpr int LPT = MNC ? BPT * EPC : (ROWS * 8) / NT;
  static constexpr int NOFF = MNC ? BPT : LPT;
  static constexpr bool kMNC = MNC;
  static_assert(MNC || (ROWS * 8) % NT == 0, "tile rows must cover the workgroup");
  static_assert(!MNC || NT % (ROWS / EPC) == 0 || BPT == 1, "block columns must be fixed per thread");
  using Base = Stage<T, ROWS, MNC, NT, true>;   // LDS layout (store_regs)
  u32x4 r[LPT];
  int voff[NOFF];   // per-thread byte offsets at k0 = 0
  int kpos;         // K position of this thread's first chunk within a tile
  int ldb_bytes;    // ld * ES (MNC: step between the EPC rows of a block)

  __device__ __forceinline__ void init(int64_t ld, int mn0, int MNlim, int tid) {
    ldb_bytes = static_cast<int>(ld * ES);
    if constexpr (!MNC) {
      kpos = (tid & 7) * EPC;
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int mn = mn0 + ((tid + i * NT) >> 3);
        voff[i] = mn < MNlim ? static_cast<int>(((int64_t)mn * ld + kpos) * ES) : kOobOffset;
      }
    } else {
      kpos = (tid / (ROWS / EPC)) * EPC;   // br * EPC of block 0 (block bi adds bi * NT / (ROWS/EPC) * EPC)
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int b = tid + bi * NT;
        const int bc = b % (ROWS / EPC), br = b / (ROWS / EPC);
        const int mn = mn0 + bc * EPC;
        const bool ok = (NBLK % NT == 0 || b < NBLK) && mn < MNlim;
        voff[bi] = ok ? static_cast<int>(((int64_t)br * EPC * ld + mn) * ES) : kOobOffset;
      }
    }
  }

  // Issue the loads of the K tile starting at k0 (k >= Klim reads zeros).
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rsrc, int k0, int Klim) {
    if constexpr (!MNC) {
      const bool kok = k0 + kpos < Klim;
      const int kb = k0 * ES;
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int off = kok ? voff[i] + kb : kOobOffset;
        r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
      }
    } else {
      const int kb = k0 * ldb_bytes;
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int k1 = k0 + kpos + bi * (NT / (ROWS / EPC)) * EPC;
#pragma unroll
        for (int j = 0; j < EPC; ++j) {
          const int off = (k1 + j < Klim) ? voff[bi] + kb + j * ldb_bytes : kOobOffset;
          r[bi * EPC + j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
        }
      }
    }
  }

  // ---- per-chunk forms, for hand-interleaving with the MFMAs ----
  // load_one<L>: input chunk L (MNC: block L / EPC, row L % EPC of the block).
  template <int L>
  __device__ __forceinline__ void load_one(__amdgpu_buffer_rsrc_t rsrc, int k0, int Klim) {
    if constexpr (!MNC) {
      const int off = (k0 + kpos < Klim) ? voff[L] + k0 * ES : kOobOffset;
      r[L] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    } else {
      constexpr int BI = L / EPC, J = L % EPC;
      const int k = k0 + kpos + BI * (NT / (ROWS / EPC)) * EPC + J;
      const int off = (k < Klim) ? voff[BI] + k0 * ldb_bytes + J * ldb_bytes : kOobOffset;
      r[L] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    }
  }

  // pro_one<L>: dY' = dY * act'(Z) on input chunk L (+ its column sums).
  template <int L, int ACT, bool SUMS>
  __device__ __forceinline__ void pro_one(const PipeStage& z, float slope, float (*colsum)[EPC]) {
    float g[EPC], zz[EPC];
    chunk_to_f32<T>(r[L], g);
    chunk_to_f32<T>(z.r[L], zz);
#pragma unroll
    for (int e = 0; e < EPC; ++e) g[e] *= act_grad_t<ACT>(zz[e], slope);
    if constexpr (SUMS && MNC) {
#pragma unroll
      for (int e = 0; e < EPC; ++e) colsum[L / EPC][e] += g[e];
    }
    r[L] = f32_to_chunk<T>(g);
  }

  // store_one<O>: LDS chunk O (MNC: transposed row O % EPC of block O / EPC).
  template <int O>
  __device__ __forceinline__ void store_one(u32x4* lds, int tid) const {
    if constexpr (!MNC) {
      const int c = tid + O * NT;
      const int row = c >> 3;
      lds[row * 8 + ((c & 7) ^ swz(row))] = r[O];
    } else {
      constexpr int BI = O / EPC, E = O % EPC;
      const int b = tid + BI * NT;
      if (NBLK % NT != 0 && b >= NBLK) return;
      const int bc = b % (ROWS / EPC), br = b / (ROWS / EPC);
      const u32x4* in = r + BI * EPC;
      u32x4 t;
      if constexpr (EPC == 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = in[2 * j][E >> 1], hi = in[2 * j + 1][E >> 1];
          t[j] = (E & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
      } else {
        t = u32x4{in[0][E], in[1][E], in[2][E], in[3][E]};
      }
      const int row = bc * EPC + E;
      lds[row * 8 + (br ^ swz(row))] = t;
    }
  }

  template <int ACT, bool SUMS>
  __device__ __forceinline__ void prologue(const PipeStage& z, float slope, float (*colsum)[EPC]) {
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

  __device__ __forceinline__ void store(u32x4* lds, int tid) const { Base::store_regs(r, lds, tid); }
};

// Compile-time loop: f.template operator()<I>() for I in [B, E).  Register
// arrays indexed with I stay in registers however large the unrolled body is.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f.template operator()<B>();
    static_for<B + 1, E>(f);
  }
}

// Fused bias/act epilogue of one wave's FM x FN grid of 32x32 accumulators.
// Each lane holds 4 consecutive N columns of one M row per group of 4 values
// (the W/B fragment is MFMA src0).
template <typename T, int FM, int FN, int WTM, int WTN, int ACT>
__device__ __forceinline__ void store_tile(const f32x16_t (&acc)[FM][FN], const TileArgs& p, int bz, int m0,
                                           int n0, int wm, int wn, int lane) {
  T* Db = reinterpret_cast<T*>(p.D) + (int64_t)bz * p.sD;
  T* Zob = p.Zo ? reinterpret_cast<T*>(p.Zo) + (int64_t)bz * p.sZo : nullptr;
  const float* biasb = p.bias ? p.bias + (int64_t)bz * p.sBias : nullptr;
  const int bk = biasb ? p.bias_kind : kBiasNone;
  const bool vec = p.store_vec != 0;
  const float alpha = p.alpha;
  static_for<0, FM>([&]<int I>() __attribute__((always_inline)) {
    const int m = m0 + wm * WTM + I * 32 + (lane & 31);
    if (m < p.M) {
      T* drow = Db + (int64_t)m * p.ldd;
      T* zrow = Zob ? Zob + (int64_t)m * p.ldzo : nullptr;
      const float brow = bk == kBiasPerM ? biasb[m] : bk == kBiasScalar ? biasb[0] : 0.f;
      static_for<0, FN * 4>([&]<int JQ>() __attribute__((always_inline)) {
        constexpr int J = JQ / 4, Q = JQ % 4;
        const int n = n0 + wn * WTN + J * 32 + Q * 8 + (lane >> 5) * 4;
        if (n < p.N) {
          float pre[4], y[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float v = acc[I][J][Q * 4 + t];
            if (alpha != 1.f) v = alpha * v;
            v += bk == kBiasPerN ? biasb[min(n + t, p.N - 1)] : brow;
            pre[t] = v;
            y[t] = act_fwd_t<ACT>(v, p.slope);
          }
          if (zrow) store4<T>(zrow, n, p.N, pre, vec);
          store4<T>(drow, n, p.N, y, vec);
        }
      });
    }
  });
}

// Staging work of one K tile, as an ordered list of per-chunk items that the
// main loop spreads over the MFMA slots: for each operand, the LDS stores of
// the chunks in registers (with the act' prologue first when it applies) and
// the reloads of the same registers with the tile after.  For a transposed
// (MN-contiguous) operand a block's EPC inputs make EPC outputs, so all of a
// block's stores precede its reloads.
enum WKind : int { kStoreA, kLoadA, kLoadZA, kProB, kStoreB, kLoadB, kLoadZB };
struct WItem { int kind, idx; };
template <int N>
struct WList { WItem it[N]; };

template <bool MNC_A, bool MNC_B, int PRO, int LA, int LB, int EPC>
struct WSched {
  static constexpr int N = 2 * LA + 2 * LB + (PRO == 1 ? LA : 0) + (PRO == 2 ? 2 * LB : 0);
  static constexpr WList<N> make() {
    WList<N> w{};
    int n = 0;
    if constexpr (!MNC_A) {
      for (int i = 0; i < LA; ++i) {
        w.it[n++] = {kStoreA, i};
        w.it[n++] = {kLoadA, i};
        if (PRO == 1) w.it[n++] = {kLoadZA, i};
      }
    } else {
      for (int b = 0; b < LA / EPC; ++b) {
        for (int e = 0; e < EPC; ++e) w.it[n++] = {kStoreA, b * EPC + e};
        for (int j = 0; j < EPC; ++j) w.it[n++] = {kLoadA, b * EPC + j};
        if (PRO == 1)
          for (int j = 0; j < EPC; ++j) w.it[n++] = {kLoadZA, b * EPC + j};
      }
    }
    if constexpr (MNC_B) {
      for (int b = 0; b < LB / EPC; ++b) {
        if (PRO == 2)
          for (int j = 0; j < EPC; ++j) w.it[n++] = {kProB, b * EPC + j};
        for (int e = 0; e < EPC; ++e) w.it[n++] = {kStoreB, b * EPC + e};
        for (int j = 0; j < EPC; ++j) w.it[n++] = {kLoadB, b * EPC + j};
        if (PRO == 2)
          for (int j = 0; j < EPC; ++j) w.it[n++] = {kLoadZB, b * EPC + j};
      }
    } else {
      for (int i = 0; i < LB; ++i) {
        if (PRO == 2) w.it[n++] = {kProB, i};
        w.it[n++] = {kStoreB, i};
        w.it[n++] = {kLoadB, i};
        if (PRO == 2) w.it[n++] = {kLoadZB, i};
      }
    }
    return w;
  }
  static constexpr WList<N> list = make();
};

// Scheduling hints (LLVM AMDGPU sched_group_barrier masks).
constexpr int kSgMfma = 0x008, kSgValu = 0x002, kSgVmemRead = 0x020, kSgDsRead = 0x100, kSgDsWrite = 0x200;
#define GEV2_SG(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)

// Epilogue of the vector path: no branches around loads or stores.  A PerN
// bias comes from LDS (staged once per workgroup), PerM / Scalar from
// registers loaded up front; Y and Z are written with raw buffer stores whose
// offset is moved out of range for rows >= M or column groups >= N (the host
// guarantees N % 4 == 0 and 16-byte aligned rows for this path).
template <typename T, int FM, int FN, int WTM, int WTN, int ACT>
__device__ __forceinline__ void store_tile_vec(const f32x16_t (&acc)[FM][FN], const TileArgs& p, int bz, int m0,
                                               int n0, int wm, int wn, int lane, const float* bias_lds) {
  constexpr int ES = sizeof(T);
  const __amdgpu_buffer_rsrc_t rD = make_rsrc(reinterpret_cast<T*>(p.D) + (int64_t)bz * p.sD);
  const bool hz = p.Zo != nullptr;
  const __amdgpu_buffer_rsrc_t rZ = make_rsrc(hz ? reinterpret_cast<T*>(p.Zo) + (int64_t)bz * p.sZo
                                                 : reinterpret_cast<T*>(p.D));
  const float* biasb = p.bias ? p.bias + (int64_t)bz * p.sBias : nullptr;
  const int bk = biasb ? p.bias_kind : kBiasNone;
  const float alpha = p.alpha;
  const float bscalar = bk == kBiasScalar ? biasb[0] : 0.f;
  float brow[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * WTM + i * 32 + (lane & 31);
    brow[i] = bk == kBiasPerM ? (m < p.M ? biasb[m] : 0.f) : bscalar;
  }
  const int h4 = (lane >> 5) * 4;
  static_for<0, FM>([&]<int I>() __attribute__((always_inline)) {
    const int m = m0 + wm * WTM + I * 32 + (lane & 31);
    const bool mok = m < p.M;
    const int64_t dro = (int64_t)m * p.ldd, zro = (int64_t)m * p.ldzo;
    static_for<0, FN * 4>([&]<int JQ>() __attribute__((always_inline)) {
      constexpr int J = JQ / 4, Q = JQ % 4;
      const int nl = wn * WTN + J * 32 + Q * 8 + h4;   // column within the tile
      const int n = n0 + nl;
      f32x4_t bv = {brow[I], brow[I], brow[I], brow[I]};
      if (bk == kBiasPerN) bv = *reinterpret_cast<const f32x4_t*>(bias_lds + nl);
      float pre[4], y[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        pre[t] = fmaf(alpha, acc[I][J][Q * 4 + t], bv[t]);
        y[t] = act_fwd_t<ACT>(pre[t], p.slope);
      }
      const bool ok = mok && n < p.N;
      const int od = ok ? static_cast<int>((dro + n) * ES) : kOobOffset;
      if constexpr (ES == 4) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4_t{y[0], y[1], y[2], y[3]}), rD, od, 0, 0);
      } else {
        const u32x2 w = {Elem<T>::bits(y[0]) | (Elem<T>::bits(y[1]) << 16),
                         Elem<T>::bits(y[2]) | (Elem<T>::bits(y[3]) << 16)};
        __builtin_amdgcn_raw_buffer_store_b64(w, rD, od, 0, 0);
      }
      if (hz) {
        const int oz = ok ? static_cast<int>((zro + n) * ES) : kOobOffset;
        if constexpr (ES == 4) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4_t{pre[0], pre[1], pre[2], pre[3]}), rZ, oz, 0, 0);
        } else {
          const u32x2 w = {Elem<T>::bits(pre[0]) | (Elem<T>::bits(pre[1]) << 16),
                           Elem<T>::bits(pre[2]) | (Elem<T>::bits(pre[3]) << 16)};
          __builtin_amdgcn_raw_buffer_store_b64(w, rZ, oz, 0, 0);
        }
      }
    });
  });
}

template <typename T, int BM, int BN, int WM, int WN, bool TA, bool TB, int PRO>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_pipe_kernel(TileArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int EPC = Elem<T>::kPerChunk;
  constexpr int BK = 8 * EPC;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  static_assert(FM >= 1 && FN >= 1, "wave tile must be a multiple of 32");
  using SA = PipeStage<T, BM, TA, NT>;
  using SB = PipeStage<T, BN, !TB, NT>;
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

  const __amdgpu_buffer_rsrc_t rA = make_rsrc(reinterpret_cast<const T*>(p.A) + (int64_t)bz * p.sA);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(reinterpret_cast<const T*>(p.B) + (int64_t)bz * p.sB);
  const __amdgpu_buffer_rsrc_t rZ =
      make_rsrc(PRO ? reinterpret_cast<const T*>(p.Zi) + (int64_t)bz * p.sZi : reinterpret_cast<const T*>(p.A));

  SA sa;
  SB sb;
  SA za;  // prologue Z for A (PRO == 1)
  SB zb;  // prologue Z for B (PRO == 2)
  sa.init(p.lda, m0, p.M, tid);
  sb.init(p.ldb, n0, p.N, tid);
  if constexpr (PRO == 1) za.init(p.ldzi, m0, p.M, tid);
  if constexpr (PRO == 2) zb.init(p.ldzi, n0, p.N, tid);
  float colsum[SB::BPT][EPC];
  if constexpr (kSums) {
#pragma unroll
    for (int i = 0; i < SB::BPT; ++i)
#pragma unroll
      for (int e = 0; e < EPC; ++e) colsum[i][e] = 0.f;
  }
  // Only the workgroups of tile row 0 emit the column sums (each covers all M).
  const bool do_sums = kSums && p.dbias != nullptr && tm == 0;

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int KT = (p.K + BK - 1) / BK;

  auto main_loop = [&]<int PACT, bool SUMS>() __attribute__((always_inline)) {
    auto load_tile = [&](int k0) __attribute__((always_inline)) {
      sa.load(rA, k0, p.K);
      sb.load(rB, k0, p.K);
      if constexpr (PRO == 1) za.load(rZ, k0, p.K);
      if constexpr (PRO == 2) zb.load(rZ, k0, p.K);
    };
    auto stage_tile = [&](int buf) __attribute__((always_inline)) {
      if constexpr (PRO == 1) sa.template prologue<PACT, false>(za, p.slope, nullptr);
      if constexpr (PRO == 2) sb.template prologue<PACT, SUMS>(zb, p.slope, colsum);
      sa.store(As + buf * BM * 8, tid);
      sb.store(Bs + buf * BN * 8, tid);
    };
    auto read_frags = [&](int buf, int q, u32x4 (&af)[FM], u32x4 (&bfr)[FN]) __attribute__((always_inline)) {
      const u32x4* Ac = As + buf * BM * 8;
      const u32x4* Bc = Bs + buf * BN * 8;
      const int ch = 2 * q + (lane >> 5);
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
    };
    constexpr int NMF = FM * FN;                      // MFMA groups per k16 step
    constexpr int NFR = FM + FN;                      // fragment reads per k16 step
    constexpr int MF_PER_K = sizeof(T) == 4 ? 4 : 1;  // MFMAs per fragment pair

    constexpr int NMI = NMF * MF_PER_K;      // MFMA instructions per k16 step
    constexpr int LA = SA::LPT, LB = SB::LPT;
    constexpr int H = (NMI + 1) / 2;          // fragment reads go in the first half
    using WS = WSched<SA::kMNC, SB::kMNC, PRO, LA, LB, EPC>;
    constexpr int NW = WS::N;                 // staging items per K tile
    constexpr int NSLOT = 4 * NMI;            // MFMA slots per K tile

    auto mfma_one = [&]<int X>(const u32x4 (&af)[FM], const u32x4 (&bfr)[FN]) __attribute__((always_inline)) {
      if constexpr (sizeof(T) == 4) {
        // element-major order: consecutive MFMAs update different accumulators
        constexpr int E = X / NMF, P = X % NMF, I = P / FN, J = P % FN;
        acc[I][J] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bfr[J][E]), __uint_as_float(af[I][E]),
                                                         acc[I][J], 0, 0, 0);
      } else {
        constexpr int I = X / FN, J = X % FN;
        mfma_step<T>(acc[I][J], af[I], bfr[J]);
      }
    };
    auto read_one = [&]<int F>(int buf, int q, u32x4 (&af)[FM], u32x4 (&bfr)[FN]) __attribute__((always_inline)) {
      const int ch = 2 * q + (lane >> 5);
      if constexpr (F < FM) {
        const int row = wm * WTM + F * 32 + (lane & 31);
        af[F] = (As + buf * BM * 8)[row * 8 + (ch ^ swz(row))];
      } else {
        const int row = wn * WTN + (F - FM) * 32 + (lane & 31);
        bfr[F - FM] = (Bs + buf * BN * 8)[row * 8 + (ch ^ swz(row))];
      }
    };
    auto load_one = [&]<int L>(int k0) __attribute__((always_inline)) {
      if constexpr (L < LA) sa.template load_one<L>(rA, k0, p.K);
      else if constexpr (L < LA + LB) sb.template load_one<L - LA>(rB, k0, p.K);
      else if constexpr (PRO == 1) za.template load_one<L - LA - LB>(rZ, k0, p.K);
      else zb.template load_one<L - LA - LB>(rZ, k0, p.K);
    };
    auto store_one = [&]<int S>(int buf) __attribute__((always_inline)) {
      if constexpr (S < LA) {
        if constexpr (PRO == 1) sa.template pro_one<S, PACT, false>(za, p.slope, nullptr);
        sa.template store_one<S>(As + buf * BM * 8, tid);
      } else {
        sb.template store_one<S - LA>(Bs + buf * BN * 8, tid);
      }
    };

    // staging item W of a window: buffer `buf` receives the tile held in
    // registers, which are then reloaded from K offset `kload`
    auto witem = [&]<int W>(int buf, int kload) __attribute__((always_inline)) {
      constexpr WItem it = WS::list.it[W];
      if constexpr (it.kind == kStoreA) {
        if constexpr (PRO == 1) sa.template pro_one<it.idx, PACT, false>(za, p.slope, nullptr);
        sa.template store_one<it.idx>(As + buf * BM * 8, tid);
      } else if constexpr (it.kind == kLoadA) {
        sa.template load_one<it.idx>(rA, kload, p.K);
      } else if constexpr (it.kind == kLoadZA) {
        if constexpr (PRO == 1) za.template load_one<it.idx>(rZ, kload, p.K);
      } else if constexpr (it.kind == kProB) {
        if constexpr (PRO == 2) sb.template pro_one<it.idx, PACT, SUMS>(zb, p.slope, colsum);
      } else if constexpr (it.kind == kStoreB) {
        sb.template store_one<it.idx>(Bs + buf * BN * 8, tid);
      } else if constexpr (it.kind == kLoadB) {
        sb.template load_one<it.idx>(rB, kload, p.K);
      } else {
        if constexpr (PRO == 2) zb.template load_one<it.idx>(rZ, kload, p.K);
      }
    };
    // the items of slot G (of NSLOT) of a window
    auto wslot = [&]<int G>(int buf, int kload) __attribute__((always_inline)) {
      static_for<G * NW / NSLOT, (G + 1) * NW / NSLOT>([&]<int W>() __attribute__((always_inline)) {
        witem.template operator()<W>(buf, kload);
      });
    };

    // Software pipeline over K tiles (tile t in LDS buffer t % 2), hand-
    // interleaved: every MFMA slot is followed by the LDS fragment reads and
    // staging items assigned to it and a scheduling fence, so this order holds:
    //   q0..q2: MFMAs of steps 0..2 | fragment reads of steps 1..3 (first half
    //           of each step) | staging window t-1, slots NMI..4*NMI-1
    //   barrier: every wave is done reading buffer t % 2, and window t-1 (tile
    //           t+1 into buffer (t+1) % 2) is complete
    //   q3:     MFMAs of step 3 | step-0 fragment reads of tile t+1 | staging
    //           window t, slots 0..NMI-1
    // Staging window w stores tile w+2 (in registers) into buffer w % 2 and
    // reloads the registers with tile w+3, spread over a whole tile of MFMA
    // slots: a global load has one K tile to arrive, an LDS store until the
    // next barrier.  Tiles at or beyond K read as zeros.
    load_tile(0);
    stage_tile(0);
    load_tile(BK);
    static_for<0, NMI>([&]<int G>() __attribute__((always_inline)) {   // window -1, first part
      wslot.template operator()<G>(1, 2 * BK);
    });
    __syncthreads();
    u32x4 af[2][FM], bfr[2][FN];
    read_frags(0, 0, af[0], bfr[0]);

    for (int kt = 0; kt < KT; ++kt) {
      const int cur = kt & 1;
      const int kprev = (kt + 2) * BK;   // window kt-1 reloads tile kt+2
      static_for<0, NMI>([&]<int X>() __attribute__((always_inline)) {
        mfma_one.template operator()<X>(af[0], bfr[0]);
        if constexpr (X < H)
          static_for<X * NFR / H, (X + 1) * NFR / H>([&]<int F>() __attribute__((always_inline)) {
            read_one.template operator()<F>(cur, 1, af[1], bfr[1]);
          });
        wslot.template operator()<NMI + X>(cur ^ 1, kprev);
        __builtin_amdgcn_sched_barrier(0);
      });
      static_for<0, NMI>([&]<int X>() __attribute__((always_inline)) {
        mfma_one.template operator()<X>(af[1], bfr[1]);
        if constexpr (X < H)
          static_for<X * NFR / H, (X + 1) * NFR / H>([&]<int F>() __attribute__((always_inline)) {
            read_one.template operator()<F>(cur, 2, af[0], bfr[0]);
          });
        wslot.template operator()<2 * NMI + X>(cur ^ 1, kprev);
        __builtin_amdgcn_sched_barrier(0);
      });
      static_for<0, NMI>([&]<int X>() __attribute__((always_inline)) {
        mfma_one.template operator()<X>(af[0], bfr[0]);
        if constexpr (X < H)
          static_for<X * NFR / H, (X + 1) * NFR / H>([&]<int F>() __attribute__((always_inline)) {
            read_one.template operator()<F>(cur, 3, af[1], bfr[1]);
          });
        wslot.template operator()<3 * NMI + X>(cur ^ 1, kprev);
        __builtin_amdgcn_sched_barrier(0);
      });
      __syncthreads();
      const int knext = (kt + 3) * BK;   // window kt reloads tile kt+3
      static_for<0, NMI>([&]<int X>() __attribute__((always_inline)) {
        mfma_one.template operator()<X>(af[1], bfr[1]);
        if constexpr (X < H)
          static_for<X * NFR / H, (X + 1) * NFR / H>([&]<int F>() __attribute__((always_inline)) {
            read_one.template operator()<F>(cur ^ 1, 0, af[0], bfr[0]);
          });
        wslot.template operator()<X>(cur, knext);
        __builtin_amdgcn_sched_barrier(0);
      });
    }
  };

  if constexpr (PRO == 0) {
    main_loop.template operator()<kActNone, false>();
  } else {
    // Only the piecewise-linear activations are fused into the operand load
    // (a compare and a select per element); the host materialises dY' for the
    // transcendental ones, whose act' would be recomputed by every workgroup
    // that loads the element.
    dispatch_act_linear(p.pro_act, [&]<int PACT>() __attribute__((always_inline)) {
      if (do_sums) main_loop.template operator()<PACT, kSums>();
      else main_loop.template operator()<PACT, false>();
    });
  }

  if constexpr (kSums) {
    if (do_sums) {
      __syncthreads();
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

  if (p.store_vec) {
    // stage a PerN bias slice in LDS (every wave is past its last LDS read)
    float* bias_lds = reinterpret_cast<float*>(lds);
    __syncthreads();
    if (p.bias && p.bias_kind == kBiasPerN) {
      const float* biasb = p.bias + (int64_t)bz * p.sBias;
      for (int c = tid; c < BN; c += NT) bias_lds[c] = n0 + c < p.N ? biasb[n0 + c] : 0.f;
    }
    __syncthreads();
    if constexpr (PRO != 0) {
      store_tile_vec<T, FM, FN, WTM, WTN, kActNone>(acc, p, bz, m0, n0, wm, wn, lane, bias_lds);
    } else {
      dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
        store_tile_vec<T, FM, FN, WTM, WTN, ACT>(acc, p, bz, m0, n0, wm, wn, lane, bias_lds);
      });
    }
  } else if constexpr (PRO != 0) {
    store_tile<T, FM, FN, WTM, WTN, kActNone>(acc, p, bz, m0, n0, wm, wn, lane);
  } else {
    dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
      store_tile<T, FM, FN, WTM, WTN, ACT>(acc, p, bz, m0, n0, wm, wn, lane);
    });
  }
}

// ---------------------------------------------------------------------------
// Host-side launch (instantiation table)
// ---------------------------------------------------------------------------
template <int CFG> struct CfgShape;
template <> struct CfgShape<kCfg256x256> { static constexpr int BM = 256, BN = 256, WM = 2, WN = 2; };
template <> struct CfgShape<kCfg128x128> { static constexpr int BM = 128, BN = 128, WM = 2, WN = 2; };
template <> struct CfgShape<kCfg128x64> { static constexpr int BM = 128, BN = 64, WM = 4, WN = 1; };
template <> struct CfgShape<kCfg64x64> { static constexpr int BM = 64, BN = 64, WM = 2, WN = 2; };
template <> struct CfgShape<kCfg128x256> { static constexpr int BM = 128, BN = 256, WM = 2, WN = 2; };

template <typename T, int CFG, bool TA, bool TB, int PRO, bool VEC>
static hipError_t launch_one(const TileArgs& a, int batch, hipStream_t s) {
  using C = CfgShape<CFG>;
  dim3 grid(a.tiles_m * a.tiles_n, batch);
  dim3 block(C::WM * C::WN * 64);
  if constexpr (VEC)
    hipLaunchKernelGGL((gemm_pipe_kernel<T, C::BM, C::BN, C::WM, C::WN, TA, TB, PRO>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((gemm_tile_kernel<T, C::BM, C::BN, C::WM, C::WN, TA, TB, PRO, VEC>), grid, block, 0, s, a);
  return hipGetLastError();
}

// Layout combos in use: NN (forward, conv, P.V), NT (dX, QK^T), TN (dW, SDPA dV/dK).
// The fused-prologue variants (pro != 0) are not built for 256x256 (the host
// never selects that tile for them: the extra operand registers would spill).
template <typename T, int CFG, bool VEC>
static hipError_t launch_layout(bool ta, bool tb, int pro, const TileArgs& a, int batch,
                                hipStream_t s) {
  if (!ta && !tb && pro == 0) return launch_one<T, CFG, false, false, 0, VEC>(a, batch, s);
  if (!ta && tb && pro == 0) return launch_one<T, CFG, false, true, 0, VEC>(a, batch, s);
  if (ta && !tb && pro == 0) return launch_one<T, CFG, true, false, 0, VEC>(a, batch, s);
  if constexpr (CFG != kCfg256x256) {
    if (!ta && tb && pro == 1) return launch_one<T, CFG, false, true, 1, VEC>(a, batch, s);
    if (ta && !tb && pro == 2) return launch_one<T, CFG, true, false, 2, VEC>(a, batch, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t launch_cfg(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                             int batch, hipStream_t s) {
  if (!vec) return launch_layout<T, kCfg64x64, false>(ta, tb, pro, a, batch, s);
  switch (cfg) {
    case kCfg256x256: return launch_layout<T, kCfg256x256, true>(ta, tb, pro, a, batch, s);
    case kCfg128x128: return launch_layout<T, kCfg128x128, true>(ta, tb, pro, a, batch, s);
    case kCfg64x64: return launch_layout<T, kCfg64x64, true>(ta, tb, pro, a, batch, s);
    case kCfg128x256: return launch_layout<T, kCfg128x256, true>(ta, tb, pro, a, batch, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
