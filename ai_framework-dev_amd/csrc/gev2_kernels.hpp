// Kernel argument blocks and launcher declarations shared between the HIP
// kernels (gemm_tile.hip, gemm_skinny.hip, gemm_aux.hip) and the C-ABI
// dispatcher (capi.hip).  All strides and leading dimensions are in elements.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct gev2_gemm_fwd_desc;   // include/gev2_gemm.h

namespace gev2 {

// One launch of the MFMA tile kernel computes, for each batch slice b,
//   D = epilogue( alpha * op(A) @ op(B) )
// where op(A) is [M,K] and op(B) is [K,N].  Operand layouts:
//   trans_a = 0: A is [M,K] row-major (lda >= K);  1: A is [K,M] (lda >= M)
//   trans_b = 0: B is [K,N] row-major (ldb >= N);  1: B is [N,K] (ldb >= K)
// A "prologue" may replace one operand element-wise by  g * act'(z)  with z
// read from Zi at the same logical position (the backward pass's dY' = dY (.)
// act'(Z)), and, for the [K,N] operand, also emit its column sums (dBias).
struct TileArgs {
  const void* A; const void* B; void* D; void* Zo;
  const void* Zi;        // prologue pre-activation (same layout as the operand it scales)
  const float* bias;     // epilogue bias (kind below)
  float* dbias;          // PerN dBias: column sums of the prologue operand (PRO == 2), or the
                         // sum of dbias_part's row blocks (direct-to-LDS TN launch)
  const float* dbias_part;   // [batch][dbias_rb][N] fp32 row-block column sums of B (or null)
  int64_t sDbiasPart;
  int dbias_rb;
  int64_t lda, ldb, ldd, ldzo, ldzi;
  int64_t sA, sB, sD, sZo, sZi, sBias, sDbias;   // batch strides
  int M, N, K;
  int act, bias_kind;    // epilogue
  float slope, alpha;
  int pro_act;           // prologue activation kind (derivative applied)
  int tiles_m, tiles_n;
  int store_vec;         // D/Zo rows: 0 scalar, 1 4-wide vector stores, 2 16-byte row segments (16-bit)
};

// Skinny forward (M <= kSkinnyMaxM): for 16-bit data a split-K kernel over
// 256 x 256 blocks of W with fp32 partials in a workspace and a fixed-order
// reduction pass; otherwise one workgroup per 32-byte column slab of W over
// all of K (no cross-workgroup reduction, no workspace).
constexpr int kSkinnyMaxM = 16;
struct SkinnyArgs {
  const void* A; const void* B; void* D; void* Zo;
  const float* bias;
  int64_t lda, ldb, ldd, ldzo;
  int M, N, K;
  int act, bias_kind;
  float slope, alpha;
  int x_vec;             // 1: X rows 16-byte aligned, K % chunk == 0; 2: also spans < 2^31 bytes
  // Optional second part of X (split kernel only): columns K1 .. K-1 of X are
  // columns 0 .. K-K1-1 of A2 (row stride lda2), so X = [A | A2] is never
  // gathered.  K1 must be a multiple of 256 (a whole number of K blocks);
  // A2 null: X is A alone.
  const void* A2;
  int64_t lda2;
  int K1;
};

// Element-wise gZ = gY * act'(Z) (optionally scaled by beta) -> out, and
// deterministic bias-gradient reductions.
struct GradArgs {
  const void* gY; const void* Z; void* out;      // out may be null
  float* gbias;                                   // may be null
  int64_t ldgy, ldz, ldout;
  int64_t sgY, sZ, sOut, sGbias;
  int M, N;
  int act; float slope; float beta;
  int bias_kind;
};

// Vectorised dY' = dY (.) act'(Z) into a dense [M,N] buffer (16-byte chunks;
// N a multiple of the chunk, rows 16-byte aligned) plus, when `partial` is
// set, fixed-order column sums per block of kPrepRows rows: partial[rb][n].
// finish_col_sums adds the row-block partials of each column in order.
// With `rowsum` set instead (a PerM bias), one wave forms each whole row and
// writes its fixed-order sum to rowsum[batch * sRowsum + m].
constexpr int kPrepRows = 64;
struct PrepArgs {
  const void* gY; const void* Z; void* out; float* partial;
  int64_t ldgy, ldz;              // out has ld = N; partial has ld = N
  int64_t sgY, sZ, sOut, sPartial;
  int M, N;
  int act; float slope;
  float* rowsum; int64_t sRowsum;
};
hipError_t launch_grad_prep(int dtype, const PrepArgs& a, int batch, hipStream_t s);

// gA of the backward when M <= 16 (one slice): D[M,K] = alpha * (G (.) act'(Z)) B^T
// with B [K,N]; Z null when G is already dY'.  Rows of G, Z and B must be
// 16-byte aligned with N a multiple of the chunk.
struct SkinnyNtArgs {
  const void* G; const void* Z; const void* B; void* D;
  int64_t ldg, ldz, ldb, ldd;
  int M, N, K;
  int act; float slope, alpha;
};
hipError_t launch_skinny_nt(int dtype, const SkinnyNtArgs& a, hipStream_t s);
// Second pass of the fp32 split-K forward: Z = alpha * sum_s part[s] + bias
// (slices added in order s = 0, 1, ...), Y = act(Z).  part is [ks][M][N]
// dense; Y / Z are row-major with leading dimensions ldy / ldz (Z may be null).
struct SplitkReduceArgs {
  const float* part;
  int ks, M, N;
  float alpha;
  const float* bias; int bias_kind;
  int act; float slope;
  float* Y; int64_t ldy;
  float* Z; int64_t ldz;
};
hipError_t launch_splitk_reduce(const SplitkReduceArgs& a, hipStream_t s);

// Small fp32 problems in one launch (gemm_small.hip).  Operand element (i, k)
// (i: output row for the left operand, output column for the right one; k:
// reduction index) is p[i * rs + k * ks], times act'(z[i * zrs + k * zks])
// when z is set (dY' formed while loading).  vec: ks = 1 (and zks = 1), p
// (and z) 16-byte aligned, rs (and zrs) multiples of 4, so that four
// consecutive k from a multiple of 4 are one 16-byte load.
struct SmallOperand {
  const float* p; int64_t rs, ks;
  const float* z; int64_t zrs, zks;
  int vec;
  // Optional second part (no z with it): reduction indices k1 .. of rows i are
  // p2[i * rs2 + (k - k1) * ks]; k1 a multiple of 4.  p2 null: p alone.
  const float* p2; int64_t rs2; int k1;
};
// out[rows, cols] (leading dimension ldo) = scale * sum_k a(row, k) b(col, k);
// kind 0: forward, 1: dX (a is dY'), 2: dW (b is dY').  own (backward only):
// each wave takes a whole tile (wgs = ceil(tiles / waves)); otherwise the
// waves of a workgroup split one tile's reduction (wgs = tiles).
struct SmallJob {
  SmallOperand a, b;
  int kind, own;
  int rows, cols, red;
  int tiles_c, tiles;   // 16x16 tiles along cols, in all
  int wgs;
  float scale;
  float* out; int64_t ldo;
};
// fwd: job 0 is the forward, Z = scale * acc + bias, out = act(Z).
// Otherwise jobs 0 and 1 (dX, dW) store scale * acc, and when gbias is set
// further workgroups (64 columns each) sum dY' = gY (.) act'(Zin) over the M
// rows of each of the N columns (PerN dBias).
struct SmallArgs {
  SmallJob job[2];
  int njobs, fwd;
  int act; float slope;
  const float* bias; int bias_kind;
  float* Z; int64_t ldz;
  const float* gY; int64_t ldgy;
  const float* Zin; int64_t ldzin;
  float* gbias;
  int M, N;
};
// waves per workgroup: 4 or 16
hipError_t launch_small(const SmallArgs& a, int waves, hipStream_t s);
// waves per workgroup for a reduction of length red: 16 from 512 on, else 4
int small_waves_for(int64_t red);
hipError_t launch_finish_col_sums(const float* partial, int64_t sPartial, int row_blocks, int N,
                                  float* gbias, int64_t sGbias, int batch, hipStream_t s);

// Launcher entry points (each returns hipError_t from the launch).
// Tile configuration ids, chosen by the host dispatcher.
enum TileCfg : int {
  kCfg256x256 = 0,   // 256x256 (direct-to-LDS: 8 waves of 128x64; register-staged: 4 of 128x128)
  kCfg128x128 = 1,   // 128x128, 4 waves (64x64 per wave)
  kCfg64x64 = 2,     // 64x64, 4 waves (32x32 per wave)
  kCfg128x256 = 3,   // 128x256, 4 waves (64x128 per wave)
  kCfg128x64 = 4,    // 128x64, 4 waves (32x64 per wave; direct-to-LDS kernel only)
};

hipError_t launch_tile(int dtype, int cfg, bool trans_a, bool trans_b, int prologue,
                       bool vec, const TileArgs& a, int batch, hipStream_t s);
hipError_t launch_tile_f32(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                           int batch, hipStream_t s);
hipError_t launch_tile_bf16(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                            int batch, hipStream_t s);
hipError_t launch_tile_f16(int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                           int batch, hipStream_t s);
hipError_t launch_dl_bf16(int cfg, bool ta, bool tb, const TileArgs& a, int batch, hipStream_t s);
hipError_t launch_dl_f16(int cfg, bool ta, bool tb, const TileArgs& a, int batch, hipStream_t s);
hipError_t launch_dl_f32(int cfg, bool ta, bool tb, const TileArgs& a, int batch, hipStream_t s);
bool dl_selected(int dtype, int cfg, int pro, bool vec, const TileArgs& a);
// part: fp32 partial sums for the split-K 16-bit kernel (skinny_split_workspace_bytes)
hipError_t launch_skinny(int dtype, const SkinnyArgs& a, float* part, hipStream_t s);

// Size of the fixed device array that gev2_gemm_fwd_noalloc takes its split-K
// scratch from (noalloc.hip): 16 MiB, the partials of skinny problems up to
// N * K = 2^26 at M = 16 (2 MiB at M = 8, N = K = 4096).
constexpr int64_t kNoAllocScratchBytes = int64_t{16} << 20;

// The forward of gev2_gemm_fwd (capi.hip).  fixed_bytes < 0: split-K scratch
// from the caller's workspace or the library's per-stream buffer; fixed_bytes
// >= 0: only from `fixed` (no allocation; larger needs are refused).
int gemm_fwd_run(const ::gev2_gemm_fwd_desc* d, void* stream, void* fixed, int64_t fixed_bytes);
// Records a HIP error as the calling thread's last error; returns GEV2_HIP_ERROR.
int report_hip_error(hipError_t e, const char* where);
bool skinny_split_eligible(const SkinnyArgs& a);
int64_t skinny_split_workspace_bytes(int M, int N, int K);
hipError_t launch_grad_elementwise(int dtype, const GradArgs& a, int batch, hipStream_t s);
hipError_t launch_bias_grad(int dtype, const GradArgs& a, int batch, hipStream_t s);

// Tile extents of each configuration (scalar-load variants always use 64x64).
inline int tile_bm(int cfg, bool vec) {
  if (!vec) return 64;
  return cfg == kCfg256x256 ? 256 : cfg == kCfg64x64 ? 64 : 128;
}
inline int tile_bn(int cfg, bool vec) {
  if (!vec) return 64;
  return cfg == kCfg256x256 ? 256 : cfg == kCfg64x64 || cfg == kCfg128x64 ? 64 : cfg == kCfg128x256 ? 256 : 128;
}

}  // namespace gev2
