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
#include <cstdlib>

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
        const int off = (nok && k < p.K) ? static_cast<int>(((int64_t)k * p.ldb + n) * sizeof(T)) : kOobOffset;
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

// ---------------------------------------------------------------------------
// 16-bit skinny forward: split-K over 256 x 256 blocks of W, streamed straight
// into LDS, v_mfma_f32_16x16x32, fixed-order reduction in a second pass.
//
// Reading W in 32-byte pieces per row (one column slab per workgroup over all
// of K) caps a 32 MB read near 2.3 TB/s on this part, while 512-byte row
// segments reach ~4.9 TB/s.  So a workgroup owns a block of 256 rows x 256
// columns (512 bytes of each row, 128 KB), and wave w takes its 64 columns
// over all 256 rows: each wave loads, transposes and multiplies only its own
// data, with no cross-wave reduction.  Per wave, 32 buffer_load ... lds of
// 1 KB (8 rows x 128 bytes) are all in flight from the start; the rows sit in
// LDS with the 32-byte block index XOR-swizzled by (k & 3), so the transpose
// reads of a 16-lane group (4 rows x 32 bytes) hit distinct banks.  The X
// block (16 rows, rows past M zero, as 8-k blocks of 16 rows x 16 bytes) is
// loaded the same way, a quarter per wave.  The K loop waits for the first
// 128 rows, runs their 4 k-steps, then waits for the rest.
//   One K block: the workgroup applies bias / activation / Z / Y itself.
//   Otherwise it writes fp32 partials in the MFMA result layout (16 bytes per
//   lane, only lanes holding rows < M) and skinny_reduce_kernel adds the K
//   blocks in order and applies the epilogue.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ f32x4_t mfma16(const u32x4& a, const u32x4& b, const f32x4_t& c) {
  if constexpr (__is_same(T, __bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
}

// W block per workgroup: COLS columns x ROWS rows, 128 KB (COLS 256 or 512);
// wave w takes COLS / 4 columns over all ROWS rows.
template <int COLS, int ROWS = 65536 / COLS>
struct SplitShape {
  static_assert(ROWS * COLS <= 65536 && ROWS % 128 == 0, "at most 128 KB of W, whole X loads per wave");
  static constexpr int kCols = COLS;
  static constexpr int kRows = ROWS;                         // 128 KB of 16-bit W (64 KB at 128 rows)
  static constexpr int kWaveCols = COLS / 4;
  static constexpr int kRowBytes = kWaveCols * 2;            // bytes per W row per wave
  static constexpr int kTiles = kWaveCols / 16;              // 16-column MFMA tiles per wave
  static constexpr int kSteps = kRows / 32;                  // k-steps of 32
  static constexpr int kLoads = kRows * kRowBytes / 1024;    // W loads per wave (32)
  static constexpr int kXBlocks = kRows / 8;                 // 8-k X blocks (16 rows x 16 B)
  static constexpr int kXLoads = kXBlocks / 4 / 4;           // X loads per wave
};

// 256 columns unless GEV2_SKINNY_COLS=512 (the kernel, the reduction and the
// workspace size all follow this choice).
int skinny_split_cols() {
  static const int c = [] {
    const char* v = std::getenv("GEV2_SKINNY_COLS");
    return (v && std::atoi(v) == 512) ? 512 : 256;
  }();
  return c;
}

// b: the bias term of (m, n), read beforehand (ignored without a bias)
template <typename T>
__device__ __forceinline__ void skinny_out_b(const SkinnyArgs& p, int m, int n, float acc, float b) {
  T* Y = reinterpret_cast<T*>(p.D);
  T* Zo = reinterpret_cast<T*>(p.Zo);
  float pre = p.alpha == 1.f ? acc : p.alpha * acc;
  if (p.bias) pre += b;
  if (Zo) Elem<T>::store1(Zo + (int64_t)m * p.ldzo + n, pre);
  Elem<T>::store1(Y + (int64_t)m * p.ldd + n, act_fwd(pre, p.act, p.slope));
}

template <typename T>
__device__ __forceinline__ void skinny_out(const SkinnyArgs& p, int m, int n, float acc) {
  skinny_out_b<T>(p, m, n, acc, p.bias ? load_bias(p.bias, p.bias_kind, m, n) : 0.f);
}

// partial of (split, 16-column tile, lane): lanes 0 .. 16*MQ-1 (rows < 4*MQ)
__device__ __forceinline__ int64_t skinny_part_index(int split, int ntile, int tile, int lane, int mq) {
  return ((int64_t)split * ntile + tile) * (16 * mq) + lane;
}

template <typename T, int COLS, int ROWS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_skinny_split_kernel(SkinnyArgs p, f32x4_t* part, int nslab) {
  using S = SplitShape<COLS, ROWS>;
  constexpr int RB = S::kRowBytes;
  constexpr int NWL = S::kLoads;
  constexpr int WBYTES = S::kRows * RB;                      // 32 KB per wave
  constexpr int XBYTES = S::kXBlocks * 256;
  constexpr int RPL = 1024 / RB;                             // W rows per load
  constexpr int BPR = RB / 32;                               // 32-byte blocks per row
  __shared__ __attribute__((aligned(1024))) char lds[4 * WBYTES + XBYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slab = blockIdx.x % nslab, split = blockIdx.x / nslab;
  const int c0 = slab * S::kCols + wave * S::kWaveCols;      // this wave's first column
  const int k0 = split * S::kRows;
  char* wl = lds + wave * WBYTES;
  char* xl = lds + 4 * WBYTES;

  // X: load i fills k-blocks 4i .. 4i+3: lane -> block 4i + lane/16, row m = lane % 16.
  // A K block lies wholly in A or in A2 (K1 is a multiple of the block).
  const bool second = p.A2 != nullptr && k0 >= p.K1;
  const i32x4_t rX = rsrc_words(second ? p.A2 : p.A);
  const int64_t ldx = second ? p.lda2 : p.lda;
  const int kx = second ? p.K1 : 0;                          // first X column of the source
  {
    const int m = lane & 15;
#pragma unroll
    for (int ii = 0; ii < S::kXLoads; ++ii) {
      const int i = S::kXLoads * wave + ii;
      const int k = k0 + 8 * (4 * i + (lane >> 4));
      const int off = (m < p.M && k < p.K) ? static_cast<int>(((int64_t)m * ldx + (k - kx)) * sizeof(T)) : kOobOffset;
      dma16(rX, off, 0, lds_addr(xl) + i * 1024);
    }
  }
  // W: load j fills rows RPL j .. of this wave's rows; the lane's 16 bytes hold
  // logical 32-byte block (physical ^ (row & 3))
  const i32x4_t rW = rsrc_words(p.B);
  {
    const int rsub = lane / (2 * BPR), pb = (lane % (2 * BPR)) >> 1, half = lane & 1;
    const uint32_t wl_addr = lds_addr(wl);
#pragma unroll
    for (int j = 0; j < NWL; ++j) {
      const int row = RPL * j + rsub;
      const int col = c0 + ((pb ^ (row & 3)) << 4) + half * 8;
      const int k = k0 + row;
      const int off = (k < p.K && col < p.N) ? static_cast<int>(((int64_t)k * p.ldb + col) * sizeof(T)) : kOobOffset;
      dma16(rW, off, 0, wl_addr + j * 1024);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x3f70 | (NWL & 0xf) | ((NWL >> 4) << 14));   // vmcnt(NWL): X loads done
  __syncthreads();                                                          // X block complete

  f32x4_t acc[S::kTiles];
#pragma unroll
  for (int t = 0; t < S::kTiles; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // transpose reads: lane 16g + 4e + c addresses columns 16t + 4c.. of row
  // 32s + 8g + 4h + e
  const int g = lane >> 4, e = (lane >> 2) & 3, cq = lane & 3;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    // the first half of the rows are the first NWL / 2 W loads
    if (half == 0) __builtin_amdgcn_s_waitcnt(0x3f70 | (NWL / 2 & 0xf) | ((NWL / 2) >> 4 << 14));
    else __builtin_amdgcn_s_waitcnt(0x3f70);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int ss = 0; ss < S::kSteps / 2; ++ss) {
      const int s = S::kSteps / 2 * half + ss;
      const u32x4 xa = *reinterpret_cast<const u32x4*>(xl + s * 1024 + lane * 16);
#pragma unroll
      for (int t = 0; t < S::kTiles; ++t) {
        u32x4 wf;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int k = 32 * s + 8 * g + 4 * h + e;
          const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4_t*)(wl + k * RB + ((t ^ (k & 3)) << 5) + cq * 8));
          const u32x2 w2 = __builtin_bit_cast(u32x2, v);
          wf[2 * h] = w2[0];
          wf[2 * h + 1] = w2[1];
        }
        acc[t] = mfma16<T>(xa, wf, acc[t]);
      }
    }
  }

  // D[m][n]: n = c0 + 16 t + lane % 16, m = 4 (lane / 16) + r
  const int nsplit = gridDim.x / nslab;
  if (nsplit == 1) {
#pragma unroll
    for (int t = 0; t < S::kTiles; ++t) {
      const int n = c0 + 16 * t + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * (lane >> 4) + r;
        if (m < p.M && n < p.N) skinny_out<T>(p, m, n, acc[t][r]);
      }
    }
  } else {
    const int mq = (p.M + 3) / 4;
    if (lane < 16 * mq) {
#pragma unroll
      for (int t = 0; t < S::kTiles; ++t)
        part[skinny_part_index(split, nslab * (S::kCols / 16), slab * (S::kCols / 16) + wave * S::kTiles + t, lane,
                               mq)] = acc[t];
    }
  }
}

// Y = act(alpha * sum_s part[s] + bias), K blocks added in order s = 0, 1, ...
// One thread per (16-column tile, lane, row pair) of the MFMA result layout,
// i.e. per 2 rows of one column, so that the 2 MiB of partials of an
// 8x4096x4096 problem spread over 256 single-wave workgroups; every K block's
// partial is loaded at once.
constexpr int kReduceThreads = 64;
typedef float f32x2_t __attribute__((ext_vector_type(2)));

template <typename T>
__global__ void __launch_bounds__(kReduceThreads) skinny_reduce_kernel(SkinnyArgs p, const f32x4_t* part, int nsplit,
                                                                       int ntile) {
  const int mq = (p.M + 3) / 4;
  const int64_t i = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;
  const int64_t per_split = (int64_t)ntile * 16 * mq;   // f32x4 vectors per K block
  if (i >= 2 * per_split) return;
  const int64_t v = i >> 1;
  const int half = static_cast<int>(i & 1);
  const int tile = static_cast<int>(v / (16 * mq)), lane = static_cast<int>(v % (16 * mq));
  const int n = tile * 16 + (lane & 15);
  const int m0 = 4 * (lane >> 4) + 2 * half;
  if (m0 >= p.M || n >= p.N) return;
  // The bias terms (one vector load each, index chosen without a branch) and
  // the first 16 K blocks' partials are all in flight together: one memory
  // round trip for the common K <= 4096.
  const int bk = p.bias ? p.bias_kind : kBiasNone;
  float bv[2] = {0.f, 0.f};
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int bi = bk == kBiasPerN ? n : (bk == kBiasPerM ? m0 + r : 0);
    if (bk != kBiasNone && m0 + r < p.M) bv[r] = p.bias[bi];
  }
  const f32x2_t* src = reinterpret_cast<const f32x2_t*>(part) + 2 * v + half;
  f32x2_t sum = {0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += 16) {
    f32x2_t w[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)   // past the last K block: a reload of it, not added (no branch, no copy)
      w[u] = src[2 * (int64_t)min(s0 + u, nsplit - 1) * per_split];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (s0 + u < nsplit) {
        if (s0 + u == 0) {
          sum = w[u];
        } else {
          sum[0] += w[u][0];
          sum[1] += w[u][1];
        }
      }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r)
    if (m0 + r < p.M) skinny_out_b<T>(p, m0 + r, n, sum[r], bv[r]);
}

// K-block rows: the 128 KB block (65536 / cols rows), or 128 rows of a
// 256-column slab when the 128 KB blocks would give fewer than 128 workgroups
// (half the CUs), e.g. an RNN step's 8x1536x1024: 24 workgroups of 128 KB
// become 48 of 64 KB.  K <= 256 stays one K block (its epilogue runs in the
// kernel, one launch).  GEV2_SKINNY_ROWS=256 / 128 picks one of the two
// (tuning runs).
static int skinny_split_rows(int cols, int N, int K) {
  const int rows = 65536 / cols;
  if (cols != 256 || K <= 256) return rows;
  const char* v = std::getenv("GEV2_SKINNY_ROWS");
  if (v && std::atoi(v) == 256) return rows;
  if (v && std::atoi(v) == 128) return 128;
  const int64_t wgs = (int64_t)((N + cols - 1) / cols) * ((K + rows - 1) / rows);
  return wgs < 128 ? 128 : rows;
}

template <typename T, int COLS, int ROWS>
static hipError_t launch_skinny_split_c(const SkinnyArgs& a, float* part, hipStream_t s) {
  using S = SplitShape<COLS, ROWS>;
  const int nslab = (a.N + S::kCols - 1) / S::kCols;
  const int nsplit = (a.K + S::kRows - 1) / S::kRows;
  f32x4_t* pv = reinterpret_cast<f32x4_t*>(part);
  hipLaunchKernelGGL((gemm_skinny_split_kernel<T, COLS, ROWS>), dim3(nslab * nsplit), dim3(256), 0, s, a, pv, nslab);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  const int ntile = nslab * (S::kCols / 16);
  const int64_t threads = (int64_t)ntile * 16 * ((a.M + 3) / 4) * 2;
  hipLaunchKernelGGL((skinny_reduce_kernel<T>), dim3(static_cast<unsigned>((threads + kReduceThreads - 1) / kReduceThreads)),
                     dim3(kReduceThreads), 0, s, a, pv, nsplit, ntile);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_skinny_split(const SkinnyArgs& a, float* part, hipStream_t s) {
  if (skinny_split_cols() == 512) return launch_skinny_split_c<T, 512, 128>(a, part, s);
  return skinny_split_rows(256, a.N, a.K) == 128 ? launch_skinny_split_c<T, 256, 128>(a, part, s)
                                                 : launch_skinny_split_c<T, 256, 256>(a, part, s);
}

// nsplit x (nslab x tiles per slab) x 16*ceil(M/4) lanes x 16 bytes
int64_t skinny_split_workspace_bytes(int M, int N, int K) {
  const int cols = skinny_split_cols(), rows = skinny_split_rows(cols, N, K);
  const int64_t nsplit = (K + rows - 1) / rows;
  const int64_t nslab = (N + cols - 1) / cols;
  return nsplit > 1 ? nsplit * nslab * (cols / 16) * 16 * ((M + 3) / 4) * 16 : 0;
}

// The split kernel takes 16-bit data with 16-byte aligned X rows spanning
// < 2^31 bytes (x_vec == 2) and M <= 16; GEV2_SKINNY_DOT=1 selects the
// dot-product kernel below instead (comparison runs).
bool skinny_split_eligible(const SkinnyArgs& a) {
  if (a.x_vec != 2 || a.M > 16) return false;
  if (a.A2) return true;                      // [A | A2] exists only for the split kernel
  const char* v = std::getenv("GEV2_SKINNY_DOT");
  return !(v && v[0] == '1');
}

template <typename T>
static hipError_t launch_skinny_t(const SkinnyArgs& a, float* part, hipStream_t s) {
  if (a.A2 && (sizeof(T) != 2 || !skinny_split_eligible(a) || a.K1 <= 0 || a.K1 >= a.K || a.K1 % 256 != 0 || !part))
    return hipErrorInvalidValue;
  if constexpr (sizeof(T) == 2) {
    // x_vec == 2: X rows are 16-byte aligned and span < 2^31 bytes (host)
    if (skinny_split_eligible(a)) return launch_skinny_split<T>(a, part, s);
  }
  constexpr int COLS = sk_cols<T>();
  dim3 grid((a.N + COLS - 1) / COLS);
  if (a.M <= 8)
    hipLaunchKernelGGL((gemm_skinny_kernel<T, 8>), grid, dim3(kSkThreads), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<T, 16>), grid, dim3(kSkThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_skinny(int dtype, const SkinnyArgs& a, float* part, hipStream_t s) {
  switch (dtype) {
    case kF32: return launch_skinny_t<float>(a, part, s);
    case kBF16: return launch_skinny_t<__bf16>(a, part, s);
    case kF16: return launch_skinny_t<_Float16>(a, part, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gev2
