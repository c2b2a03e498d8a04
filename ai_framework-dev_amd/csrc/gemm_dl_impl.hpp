// MFMA GEMM for 16-bit data with direct-to-LDS operand loads (gfx950).
//
// Same contract as gemm_pipe_kernel (TileArgs, tile order, vector epilogue)
// for the prologue-free layouts, but neither operand passes through registers
// on its way to LDS:
//   - every operand chunk is fetched with `buffer_load_dwordx4 ... lds`, which
//     writes a wave's 64 x 16 bytes to 1 KB of consecutive LDS at M0; the LDS
//     layout is chosen by which global chunk each lane fetches;
//   - an operand contiguous along K ("K rows") is stored as rows of BK
//     elements with the 16-byte chunk index XOR-swizzled by the row, and its MFMA
//     fragments are read with one ds_read_b128 each;
//   - an operand contiguous along M/N ("MN rows") is stored as it lies in
//     memory, one row per k, with the 32-byte block index XOR-swizzled by
//     2 (k & 3) (k & 3 for 128-byte rows), and its fragments are read with
//     two ds_read_b64_tr_b16, which
//     transpose 4x16 blocks of 16-bit elements across each 16-lane group:
//     lane 16g+i receives element e of the 8-byte chunk addressed by lane
//     16g+4e+i/4, at position i%4.
// No VALU transpose, no ds_write and no staging registers remain in the loop.
// The LDS holds S stages of BK k each, so loads run S-1 tiles ahead.
//
// The loads are issued from inline assembly so that the compiler does not
// treat them as pending writes to every LDS read that follows (it would wait
// for all outstanding loads before each transpose read).  Completion is
// explicit instead: each wave waits for its own loads (vmcnt) before the
// barrier that publishes a K tile.
#pragma once
#include "gemm_tile_impl.hpp"

namespace gev2 {

// Chunk swizzle of K rows by row length: 128-byte rows (8 chunks) use the
// tile kernel's swz(); 64-byte rows (4 chunks) use ((row >> 1) ^ (row >> 3)) & 3,
// which gives the rows of equal parity in any aligned 8 (and the rows of equal
// row & 3 in any aligned 16) distinct chunk positions, so fragment reads are
// conflict free whether a bank cycle serves 128 or 256 bytes.
template <int RBK>
__device__ __forceinline__ int swz_k(int row) {
  static_assert(RBK == 64 || RBK == 128, "K row bytes");
  if constexpr (RBK == 128) return swz(row);
  else return ((row >> 1) ^ (row >> 3)) & 3;
}

// One operand tile of ROWS (M or N extent) x BKB bytes of K, elements of ES
// bytes (2: bf16 / f16, 4: fp32).  A fragment is one u32x4 per lane: the
// 16-bit MFMA's 8 k values, or four fp32 k values (one per 32x32x2 MFMA), of
// row r0 + lane % 32 at k = KF * q + (KF / 2) * (lane / 32) + 0.. within the
// tile, KF = 32 / ES k per fragment step q.
template <int ROWS, bool MNC, int NT, int BKB, int ES>
struct DlStage {
  static_assert(BKB == 64 || BKB == 128, "K tile bytes");
  static_assert(ES == 2 || ES == 4, "element size");
  static constexpr int BK = BKB / ES;                         // k per tile
  static constexpr int EPC = 16 / ES;                         // elements per 16-byte chunk
  static constexpr int BYTES = ROWS * BKB;
  static constexpr int LOADS = BYTES / 1024;                  // wave instructions per tile
  static constexpr int LPW = LOADS / (NT / 64);               // per wave
  static constexpr int RB = MNC ? ROWS * ES : BKB;            // LDS row bytes
  static_assert(LOADS % (NT / 64) == 0, "tile loads must divide among the waves");
  static_assert(!MNC || ES == 4 || RB >= 128, "16-bit MN rows need at least 4 32-byte blocks");

  int voff[LPW];    // per-lane byte offset of each load at k0 = 0 (kOobOffset if outside)
  int kpos[LPW];    // k of the lane's chunk within the tile

  // 32-byte block swizzle of 16-bit MN rows.  A half-wave of a transpose read
  // takes two adjacent blocks (an even-odd pair) from each of four consecutive
  // rows; XOR with 2 * (k & 3) puts those eight blocks in eight different
  // 32-byte bank groups when a row has at least 8 blocks (with k & 3 alone,
  // rows k and k ^ 1 share the pair's two groups).  Rows of 4 blocks keep k & 3.
  __device__ __forceinline__ static int mn_swz(int k) { return RB >= 256 ? 2 * (k & 3) : (k & 3); }

  // mn0: tile origin along M/N; MNlim: extent; ld: leading dimension (elements)
  __device__ __forceinline__ void init(int64_t ld, int mn0, int MNlim, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int byte = (wave * LPW + i) * 1024 + lane * 16;   // LDS byte this lane fills
      const int row = byte / RB, off = byte % RB;
      if constexpr (!MNC) {
        // row = M/N index within the tile; logical chunk = physical ^ swizzle
        const int c = (off / 16) ^ swz_k<BKB>(row);
        const int mn = mn0 + row;
        kpos[i] = c * EPC;
        voff[i] = mn < MNlim ? static_cast<int>(((int64_t)mn * ld + c * EPC) * ES) : kOobOffset;
      } else if constexpr (ES == 2) {
        // row = k within the tile; logical 32-byte block = physical ^ mn_swz(k)
        const int lb = (off / 32) ^ mn_swz(row);
        const int n = lb * 16 + ((off / 16) & 1) * 8;
        const int mn = mn0 + n;
        kpos[i] = row;
        voff[i] = mn < MNlim ? static_cast<int>(((int64_t)row * ld + mn) * 2) : kOobOffset;
      } else {
        // fp32: row = k within the tile, stored as it lies in memory
        const int mn = mn0 + off / 4;
        kpos[i] = row;
        voff[i] = mn < MNlim ? static_cast<int>(((int64_t)row * ld + mn) * 4) : kOobOffset;
      }
    }
  }

  // Byte offset of K tile k0 from the tile's k = 0 (uniform).
  __device__ __forceinline__ static int kbytes(int k0, int64_t ld) {
    return MNC ? static_cast<int>(k0 * ld * ES) : k0 * ES;
  }

  // Issue load I of the K tile at k0 into the LDS buffer at `buf` (uniform).
  template <int I>
  __device__ __forceinline__ void load(const i32x4_t& rsrc, uint32_t buf, int wave, int k0, int Klim,
                                       int kb) const {
    const int off = (k0 + kpos[I] < Klim) ? voff[I] : kOobOffset;
    dma16(rsrc, off, kb, buf + (wave * LPW + I) * 1024);
  }

  // MFMA fragment of step q for rows/cols [r0, r0 + 32).
  __device__ __forceinline__ u32x4 frag(const char* buf, int r0, int q, int lane) const {
    if constexpr (!MNC) {
      const int row = r0 + (lane & 31);
      const int ch = 2 * q + (lane >> 5);
      return *reinterpret_cast<const u32x4*>(buf + row * RB + ((ch ^ swz_k<BKB>(row)) * 16));
    } else if constexpr (ES == 2) {
      const int g = lane >> 4, e = (lane >> 2) & 3, qq = lane & 3;
      const int n = r0 + 16 * (g & 1) + 4 * qq;
      u32x4 out;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = 16 * q + 8 * (g >> 1) + 4 * h + e;
        const char* p = buf + k * RB + (((n >> 4) ^ mn_swz(k)) << 5) + (n & 15) * 2;
        const s16x4_t v =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)(p));
        const u32x2 w = __builtin_bit_cast(u32x2, v);
        out[2 * h] = w[0];
        out[2 * h + 1] = w[1];
      }
      return out;
    } else {
      // fp32: four k rows, 32 consecutive columns per half-wave
      const int n = r0 + (lane & 31);
      const int kb = 8 * q + 4 * (lane >> 5);
      u32x4 out;
#pragma unroll
      for (int j = 0; j < 4; ++j) out[j] = *reinterpret_cast<const uint32_t*>(buf + (kb + j) * RB + n * 4);
      return out;
    }
  }
};

// Epilogue through LDS (16-bit outputs with 16-byte aligned rows, N % 8 == 0).
// The MFMA result layout gives each lane 4 consecutive columns of one row, so
// a direct store writes 8-byte pieces of 32 different rows.  Instead each wave
// converts one 32-row slab of its results to 16-bit values in its own LDS
// region (16-byte chunks XOR-swizzled by row), then reads it back row-major
// and writes 16 bytes per lane with consecutive lanes on consecutive bytes of
// a row.  Only the wave's own region is touched, and LDS instructions of one
// wave execute in order, so no barrier is needed between the two phases.
template <typename T, int FM, int FN, int WTM, int WTN, int ACT>
__device__ __forceinline__ void store_tile_lds(const f32x16_t (&acc)[FM][FN], const TileArgs& p, int bz, int m0,
                                               int n0, int wm, int wn, int lane, const float* bias_lds,
                                               char* stage) {
  constexpr int RBY = WTN * 2;     // bytes per staged row
  constexpr int CPR = RBY / 16;    // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;    // rows per read-back instruction
  static_assert(64 % CPR == 0 && 32 % RPI == 0, "staged row shape");
  char* ys = stage;
  char* zs = stage + 32 * RBY;
  const __amdgpu_buffer_rsrc_t rD = make_rsrc(reinterpret_cast<T*>(p.D) + (int64_t)bz * p.sD);
  const bool hz = p.Zo != nullptr;
  const __amdgpu_buffer_rsrc_t rZ = make_rsrc(hz ? reinterpret_cast<T*>(p.Zo) + (int64_t)bz * p.sZo
                                                 : reinterpret_cast<T*>(p.D));
  const float* biasb = p.bias ? p.bias + (int64_t)bz * p.sBias : nullptr;
  const int bk = biasb ? p.bias_kind : kBiasNone;
  const float alpha = p.alpha;
  const float bscalar = bk == kBiasScalar ? biasb[0] : 0.f;
  const int h = lane >> 5, rr = lane & 31;
  static_for<0, FM>([&]<int I>() __attribute__((always_inline)) {
    const int mw = m0 + wm * WTM + I * 32;   // first row of the slab
    const float brow = bk == kBiasPerM ? (mw + rr < p.M ? biasb[mw + rr] : 0.f) : bscalar;
    static_for<0, FN * 4>([&]<int JQ>() __attribute__((always_inline)) {
      constexpr int J = JQ / 4, Q = JQ % 4;
      const int nl = wn * WTN + J * 32 + Q * 8 + h * 4;   // column within the tile
      f32x4_t bv = {brow, brow, brow, brow};
      if (bk == kBiasPerN) bv = *reinterpret_cast<const f32x4_t*>(bias_lds + nl);
      float pre[4], y[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        pre[t] = fmaf(alpha, acc[I][J][Q * 4 + t], bv[t]);
        y[t] = act_fwd_t<ACT>(pre[t], p.slope);
      }
      const int off = rr * RBY + (((J * 4 + Q) ^ (rr & (CPR - 1))) * 16) + h * 8;
      *reinterpret_cast<u32x2*>(ys + off) = u32x2{Elem<T>::bits(y[0]) | (Elem<T>::bits(y[1]) << 16),
                                                  Elem<T>::bits(y[2]) | (Elem<T>::bits(y[3]) << 16)};
      if (hz)
        *reinterpret_cast<u32x2*>(zs + off) = u32x2{Elem<T>::bits(pre[0]) | (Elem<T>::bits(pre[1]) << 16),
                                                    Elem<T>::bits(pre[2]) | (Elem<T>::bits(pre[3]) << 16)};
    });
    asm volatile("" ::: "memory");
    static_for<0, 32 / RPI>([&]<int R>() __attribute__((always_inline)) {
      const int row = R * RPI + lane / CPR, ch = lane % CPR;
      const int off = row * RBY + ((ch ^ (row & (CPR - 1))) * 16);
      const int m = mw + row;
      const int n = n0 + wn * WTN + ch * 8;
      const bool ok = m < p.M && n < p.N;
      const u32x4 yv = *reinterpret_cast<const u32x4*>(ys + off);
      __builtin_amdgcn_raw_buffer_store_b128(yv, rD, ok ? static_cast<int>(((int64_t)m * p.ldd + n) * 2) : kOobOffset,
                                             0, 0);
      if (hz) {
        const u32x4 zv = *reinterpret_cast<const u32x4*>(zs + off);
        __builtin_amdgcn_raw_buffer_store_b128(zv, rZ, ok ? static_cast<int>(((int64_t)m * p.ldzo + n) * 2) : kOobOffset,
                                               0, 0);
      }
    });
    asm volatile("" ::: "memory");
  });
}

// S LDS stages of BK k each; tile t lives in stage t % S.  Per tile:
//   q = 0 .. NQ-2: MFMAs of step q | fragment reads of step q+1
//   wait for this wave's loads of tile t+1 (the S-2 younger tiles stay in
//   flight), barrier: tile t+1 is complete in LDS and every wave is done
//   reading stage t % S
//   q = NQ-1: MFMAs of the last step | step-0 reads of tile t+1 | loads of
//   tile t+S into stage t % S
// so a tile's loads are issued S-1 tiles before it is read.
//
// SUMS (TN layout): after its tile, each workgroup of the first tile row also
// finishes the PerN bias gradient of its BN columns from the fp32 row-block
// column sums of B (dbias_part, written by the pass that formed B = dY'):
// thread groups add disjoint runs of row blocks in order, then the runs are
// added in order, so no separate launch is needed for the final sum.
template <typename T, int BM, int BN, int WM, int WN, bool TA, bool TB, int BKB, int S, int WPE, bool SUMS>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_dl_kernel(TileArgs p) {
  constexpr int ES = sizeof(T);
  constexpr int NT = WM * WN * 64;
  constexpr int BK = BKB / ES;                 // k per tile
  constexpr int NQ = BKB / 32;                 // fragment steps per tile
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int NMF = FM * FN, NFR = FM + FN;
  constexpr int H = (NMF + 1) / 2;
  using SA = DlStage<BM, TA, NT, BKB, ES>;
  using SB = DlStage<BN, !TB, NT, BKB, ES>;
  constexpr int ABYTES = SA::BYTES, BBYTES = SB::BYTES;
  constexpr int NL = SA::LPW + SB::LPW;   // load instructions per wave per tile
  static_assert(S >= 2 && (S - 1) * NL <= 63, "vmcnt range");
  static_assert(S * (ABYTES + BBYTES) <= 160 * 1024, "LDS");

  __shared__ __attribute__((aligned(1024))) char lds[S * (ABYTES + BBYTES)];
  char* As = lds;
  char* Bs = lds + S * ABYTES;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  int tm, tn, bz;
  map_tile_batched(p.tiles_m, p.tiles_n, tm, tn, bz);
  const int m0 = tm * BM, n0 = tn * BN;

  const i32x4_t rA = rsrc_words(reinterpret_cast<const T*>(p.A) + (int64_t)bz * p.sA);
  const i32x4_t rB = rsrc_words(reinterpret_cast<const T*>(p.B) + (int64_t)bz * p.sB);
  SA sa;
  SB sb;
  sa.init(p.lda, m0, p.M, wave, lane);
  sb.init(p.ldb, n0, p.N, wave, lane);
  const uint32_t a_lds = lds_addr(As), b_lds = lds_addr(Bs);

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int KT = (p.K + BK - 1) / BK;
  auto load_one = [&]<int L>(int st, int k0, int kba, int kbb) __attribute__((always_inline)) {
    if constexpr (L < SA::LPW) sa.template load<L>(rA, a_lds + st * ABYTES, wave, k0, p.K, kba);
    else sb.template load<L - SA::LPW>(rB, b_lds + st * BBYTES, wave, k0, p.K, kbb);
  };
  auto load_tile = [&](int st, int k0) __attribute__((always_inline)) {
    const int kba = SA::kbytes(k0, p.lda), kbb = SB::kbytes(k0, p.ldb);
    static_for<0, NL>([&]<int L>() __attribute__((always_inline)) { load_one.template operator()<L>(st, k0, kba, kbb); });
  };
  auto read_one = [&]<int F>(int st, int q, u32x4 (&af)[FM], u32x4 (&bfr)[FN]) __attribute__((always_inline)) {
    if constexpr (F < FM) af[F] = sa.frag(As + st * ABYTES, wm * WTM + F * 32, q, lane);
    else bfr[F - FM] = sb.frag(Bs + st * BBYTES, wn * WTN + (F - FM) * 32, q, lane);
  };
  auto mfma_one = [&]<int X>(const u32x4 (&af)[FM], const u32x4 (&bfr)[FN]) __attribute__((always_inline)) {
    constexpr int I = X / FN, J = X % FN;
    mfma_step<T>(acc[I][J], af[I], bfr[J]);
  };

  static_for<0, S>([&]<int P>() __attribute__((always_inline)) { load_tile(P, P * BK); });
  // vmcnt((S-1) * NL): this wave's loads of tile 0 have landed
  constexpr int kWaitFirst = (S - 1) * NL, kWaitLoop = (S - 2) * NL;
  __builtin_amdgcn_s_waitcnt(0x3f70 | (kWaitFirst & 0xf) | ((kWaitFirst >> 4) << 14));
  __syncthreads();
  u32x4 af[2][FM], bfr[2][FN];
  static_for<0, NFR>([&]<int F>() __attribute__((always_inline)) {
    read_one.template operator()<F>(0, 0, af[0], bfr[0]);
  });

  // With two stages the loads of tile t+2 may only start once every wave has
  // finished reading tile t (the barrier), and issuing all of them among the
  // few MFMAs after it stalls MFMA issue.  So only the first NLP go there; the
  // rest follow in the first k16 step of the next tile (still before the
  // barrier that needs them), spread over its MFMAs.  Per-wave timestamps at
  // 4096^3: 2628 -> 2512 cycles per 64-deep tile.
  constexpr int NLP = S == 2 ? NL / 2 : NL;
  int pst = 0, pkload = 0, pkba = 0, pkbb = 0;   // the deferred loads' stage and K tile
  int cur = 0;   // stage of tile kt
  for (int kt = 0; kt < KT; ++kt) {
    const int nxt = cur + 1 == S ? 0 : cur + 1;
    const bool deferred = kt > 0;
    static_for<0, NQ - 1>([&]<int Q>() __attribute__((always_inline)) {
      static_for<0, NMF>([&]<int X>() __attribute__((always_inline)) {
        if constexpr (Q == 0 && NLP < NL) {
          static_for<NLP + X * (NL - NLP) / NMF, NLP + (X + 1) * (NL - NLP) / NMF>(
              [&]<int L>() __attribute__((always_inline)) {
                if (deferred) load_one.template operator()<L>(pst, pkload, pkba, pkbb);
              });
        }
        mfma_one.template operator()<X>(af[Q & 1], bfr[Q & 1]);
        if constexpr (X < H)
          static_for<X * NFR / H, (X + 1) * NFR / H>([&]<int F>() __attribute__((always_inline)) {
            read_one.template operator()<F>(cur, Q + 1, af[(Q + 1) & 1], bfr[(Q + 1) & 1]);
          });
        __builtin_amdgcn_sched_barrier(0);
      });
    });
    __builtin_amdgcn_s_waitcnt(0x3f70 | (kWaitLoop & 0xf) | ((kWaitLoop >> 4) << 14));
    __syncthreads();
    const int kload = (kt + S) * BK;
    const int kba = SA::kbytes(kload, p.lda), kbb = SB::kbytes(kload, p.ldb);
    constexpr int QL = (NQ - 1) & 1;
    static_for<0, NMF>([&]<int X>() __attribute__((always_inline)) {
      mfma_one.template operator()<X>(af[QL], bfr[QL]);
      if constexpr (X < H)
        static_for<X * NFR / H, (X + 1) * NFR / H>([&]<int F>() __attribute__((always_inline)) {
          read_one.template operator()<F>(nxt, 0, af[0], bfr[0]);
        });
      static_for<X * NLP / NMF, (X + 1) * NLP / NMF>([&]<int L>() __attribute__((always_inline)) {
        load_one.template operator()<L>(cur, kload, kba, kbb);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    pst = cur; pkload = kload; pkba = kba; pkbb = kbb;
    cur = nxt;
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);   // the loads past the last tile (all out of range)

  // epilogue (the host selects this kernel only with store_vec != 0; 2 =
  // 16-bit rows with 16-byte aligned starts and N % 8 == 0, staged through
  // LDS; 1 = 4-column vector stores from the accumulators)
  float* bias_lds = reinterpret_cast<float*>(lds);
  __syncthreads();
  if (p.bias && p.bias_kind == kBiasPerN) {
    const float* biasb = p.bias + (int64_t)bz * p.sBias;
    for (int c = tid; c < BN; c += NT) bias_lds[c] = n0 + c < p.N ? biasb[n0 + c] : 0.f;
  }
  __syncthreads();
  bool staged = false;
  if constexpr (ES == 2) {
    if (p.store_vec == 2) {
      static_assert(1024 + NT / 64 * 64 * WTN * 2 <= S * (ABYTES + BBYTES), "epilogue staging");
      char* stage = lds + 1024 + wave * (64 * WTN * 2);
      dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
        store_tile_lds<T, FM, FN, WTM, WTN, ACT>(acc, p, bz, m0, n0, wm, wn, lane, bias_lds, stage);
      });
      staged = true;
    }
  }
  if (!staged) {
    dispatch_act(p.act, [&]<int ACT>() __attribute__((always_inline)) {
      store_tile_vec<T, FM, FN, WTM, WTN, ACT>(acc, p, bz, m0, n0, wm, wn, lane, bias_lds);
    });
  }
  if constexpr (SUMS) {
    if (tm == 0) {                                   // uniform over the workgroup
      constexpr int G = NT / BN;                     // thread groups per column
      static_assert(G >= 1 && NT % BN == 0, "column groups");
      const int c = tid % BN, g = tid / BN;
      const int per = (p.dbias_rb + G - 1) / G;
      const int rb0 = g * per, rb1 = min(p.dbias_rb, rb0 + per);
      const int n = n0 + c;
      float sum = 0.f;
      if (n < p.N) {
        const float* pp = p.dbias_part + (int64_t)bz * p.sDbiasPart + n;
        for (int r = rb0; r < rb1; r += 16) {
          float v[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] = r + u < rb1 ? pp[(int64_t)(r + u) * p.N] : 0.f;
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (r + u < rb1) sum += v[u];
        }
      }
      float* red = reinterpret_cast<float*>(lds);
      __syncthreads();                               // the epilogue's LDS staging is done
      red[g * BN + c] = sum;
      __syncthreads();
      if (g == 0 && n < p.N) {
        float s = red[c];
#pragma unroll
        for (int q = 1; q < G; ++q) s += red[q * BN + c];
        p.dbias[(int64_t)bz * p.sDbias + n] = s;
      }
    }
  }
}

// Waves, K depth and stage count per tile shape.
//   256x256: 8 waves of 128x64 (2 per SIMD, accumulators in VGPRs), two stages
//     of BK = 64 (128 KB).  A second wave per SIMD keeps the MFMA pipe fed
//     while the other waits on its fragment reads or the tile barrier, and
//     halves each wave's share of the epilogue: measured at 4096^3 bf16
//     (interleaved runs, medians) 123.9 us against 129.1 us for 4 waves of
//     128x128 (one per SIMD); per-wave timestamps put the 4-wave epilogue at
//     27.8k cycles and the 8-wave one at 18.0k.  BK = 32 with 4 stages gave
//     127.7 us, 16 waves with 5 stages 143 us.
//   128x256 / 128x128: 4 waves, the most stages of BK = 32 that fit in LDS
//     (two 128x128 workgroups share a CU).
//   64x64 (fp32 only): 4 waves of 32x32, four stages of 32 k; a 1024^2 output
//     is 256 such tiles, one per CU.
//   128x64: 4 waves of 32x64, three stages of 128 bytes of K (72 KB for 16-bit,
//     so two workgroups share a CU): narrow outputs such as attention's P.V
//     (N = 64), which a 128-wide tile would half waste.
// The K depth is given in bytes (BKB), so fp32 tiles hold half the k of 16-bit
// ones in the same LDS.
template <int CFG> struct DlPipe;
template <> struct DlPipe<kCfg256x256> { static constexpr int BKB = 128, S = 2, WM = 2, WN = 4, WPE = 2; };
template <> struct DlPipe<kCfg128x256> { static constexpr int BKB = 64, S = 6, WM = 2, WN = 2, WPE = 1; };
template <> struct DlPipe<kCfg128x128> { static constexpr int BKB = 64, S = 4, WM = 2, WN = 2, WPE = 1; };
template <> struct DlPipe<kCfg64x64> { static constexpr int BKB = 128, S = 4, WM = 2, WN = 2, WPE = 1; };
template <> struct DlPipe<kCfg128x64> { static constexpr int BKB = 128, S = 3, WM = 4, WN = 1, WPE = 1; };

template <typename T, int CFG, bool TA, bool TB, bool SUMS = false>
static hipError_t launch_dl_one(const TileArgs& a, int batch, hipStream_t s) {
  using C = CfgShape<CFG>;
  using P = DlPipe<CFG>;
  dim3 grid(a.tiles_m * a.tiles_n, batch);
  hipLaunchKernelGGL((gemm_dl_kernel<T, C::BM, C::BN, P::WM, P::WN, TA, TB, P::BKB, P::S, P::WPE, SUMS>), grid,
                     dim3(P::WM * P::WN * 64), 0, s, a);
  return hipGetLastError();
}

// a.dbias_part set: the TN launch also finishes the PerN dBias (SUMS).
template <typename T, int CFG>
static hipError_t launch_dl_layout(bool ta, bool tb, const TileArgs& a, int batch, hipStream_t s) {
  const bool sums = a.dbias_part != nullptr;
  if (sums && (!(ta && !tb) || !a.dbias || a.dbias_rb < 1)) return hipErrorInvalidValue;
  if (!ta && !tb) return launch_dl_one<T, CFG, false, false>(a, batch, s);
  if (!ta && tb) return launch_dl_one<T, CFG, false, true>(a, batch, s);
  if (ta && !tb) {
    if (sums) return launch_dl_one<T, CFG, true, false, true>(a, batch, s);
    return launch_dl_one<T, CFG, true, false>(a, batch, s);
  }
  return hipErrorInvalidValue;
}

// Used for prologue-free layouts with 16-byte-aligned operands and vector
// stores: 16-bit data on the 256x256 / 128x256 / 128x128 tiles, fp32 on those
// and 64x64.
template <typename T>
static hipError_t launch_dl_cfg(int cfg, bool ta, bool tb, const TileArgs& a, int batch, hipStream_t s) {
  switch (cfg) {
    case kCfg256x256: return launch_dl_layout<T, kCfg256x256>(ta, tb, a, batch, s);
    case kCfg128x256: return launch_dl_layout<T, kCfg128x256>(ta, tb, a, batch, s);
    case kCfg128x128: return launch_dl_layout<T, kCfg128x128>(ta, tb, a, batch, s);
    case kCfg128x64: return launch_dl_layout<T, kCfg128x64>(ta, tb, a, batch, s);
    case kCfg64x64:
      if constexpr (sizeof(T) == 4) return launch_dl_layout<T, kCfg64x64>(ta, tb, a, batch, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
