// C ABI of libgev2.so: descriptor validation, kernel selection and launch.
// The kernels themselves live in gemm_tile_*.hip, gemm_skinny.hip and
// gemm_aux.hip.  Nothing here throws across the ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/gev2_gemm.h"
#include "gev2_kernels.hpp"

namespace gev2 {

// The direct-to-LDS kernel (gemm_dl_impl.hpp) takes prologue-free launches
// with vector loads and stores: 16-bit data on the three large tiles, fp32 on
// those and 64x64.  GEV2_DL=0 selects the register-staged kernel instead
// (comparison runs).
bool dl_selected(int dtype, int cfg, int pro, bool vec, const TileArgs& a) {
  if (!vec || pro != 0 || !a.store_vec) return false;
  if (cfg == kCfg64x64 && dtype != GEV2_F32) return false;
  const char* v = std::getenv("GEV2_DL");
  return !(v && v[0] == '0');
}

hipError_t launch_tile(int dtype, int cfg, bool ta, bool tb, int pro, bool vec, const TileArgs& a,
                       int batch, hipStream_t s) {
  if (dl_selected(dtype, cfg, pro, vec, a)) {
    switch (dtype) {
      case GEV2_BF16: return launch_dl_bf16(cfg, ta, tb, a, batch, s);
      case GEV2_F16: return launch_dl_f16(cfg, ta, tb, a, batch, s);
      default: return launch_dl_f32(cfg, ta, tb, a, batch, s);
    }
  }
  if (cfg == kCfg128x64) {
    // the register-staged kernel has no 128x64 tile: 128x128 over the same rows
    TileArgs b = a;
    b.tiles_n = (a.N + tile_bn(kCfg128x128, vec) - 1) / tile_bn(kCfg128x128, vec);
    return launch_tile(dtype, kCfg128x128, ta, tb, pro, vec, b, batch, s);
  }
  switch (dtype) {
    case GEV2_F32: return launch_tile_f32(cfg, ta, tb, pro, vec, a, batch, s);
    case GEV2_BF16: return launch_tile_bf16(cfg, ta, tb, pro, vec, a, batch, s);
    case GEV2_F16: return launch_tile_f16(cfg, ta, tb, pro, vec, a, batch, s);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace gev2

namespace {

thread_local std::string t_last_error;
thread_local const char* t_last_path = "";
// captures this thread has open (gev2_graph_begin .. gev2_graph_end), and the
// device frees requested meanwhile (a free during capture would invalidate it;
// e.g. a Python array whose last reference goes away inside the capture block)
thread_local int t_captures = 0;
thread_local std::vector<void*> t_deferred_frees;

int fail(int status, const std::string& msg) {
  t_last_error = msg;
  return status;
}

int hip_fail(hipError_t e, const char* where) {
  t_last_error = std::string(where) + ": " + hipGetErrorString(e);
  return GEV2_HIP_ERROR;
}

size_t elem_size(int dtype) { return dtype == GEV2_F32 ? 4 : 2; }
int elems_per_chunk(int dtype) { return dtype == GEV2_F32 ? 4 : 8; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Vector (16-byte) loads of an operand are legal when its base is 16-byte
// aligned and every row start and every chunk start is too.
// The vector path also addresses each operand slice with 32-bit byte offsets
// from the slice origin (raw buffer loads), so a slice must span < 2^31 bytes.
bool vec_ok(const void* p, int64_t ld, int64_t stride, int64_t contig_extent, int64_t rows, int batch,
            int dtype) {
  if (!p) return true;
  const int epc = elems_per_chunk(dtype);
  if (!aligned16(p) || ld % epc != 0 || contig_extent % epc != 0) return false;
  if (batch > 1 && stride % epc != 0) return false;
  const int64_t span = (rows > 0 ? (rows - 1) * ld : 0) + contig_extent;
  if (span * static_cast<int64_t>(elem_size(dtype)) > 0x7fffff00LL) return false;
  return true;
}

bool fits_i32(int64_t v) { return v >= 0 && v <= 0x7fffffffLL; }

// Vector epilogue: 4-column groups (whole, N % 4 == 0) at 16-byte aligned
// rows, written with 32-bit offsets from the slice origin (< 2^31 bytes).
bool out_vec_ok(const void* p, int64_t ld, int64_t stride, int64_t rows, int64_t cols, int batch, int dtype) {
  if (!p) return true;
  if (!aligned16(p) || ld % 4 != 0 || cols % 4 != 0) return false;
  if (batch > 1 && stride % 4 != 0) return false;
  const int64_t span = (rows > 0 ? (rows - 1) * ld : 0) + cols;
  return span * static_cast<int64_t>(elem_size(dtype)) <= 0x7fffff00LL;
}

// Epilogue level of an output: 0 = scalar stores, 1 = 4-column vector
// stores, 2 = 16-byte row segments (16-bit data with 8-column groups whose
// starts are 16-byte aligned), which the direct-to-LDS kernel stages
// through LDS.
int out_level(const void* p, int64_t ld, int64_t stride, int64_t rows, int64_t cols, int batch, int dtype) {
  if (!out_vec_ok(p, ld, stride, rows, cols, batch, dtype)) return 0;
  if (!p) return 2;
  if (dtype == GEV2_F32 || ld % 8 != 0 || cols % 8 != 0 || (batch > 1 && stride % 8 != 0)) return 1;
  return 2;
}

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  if (!v || !*v) return dflt;
  return std::atoi(v);
}

// Tile configuration: the candidate with the least estimated time, where a
// launch takes ceil(workgroups / (256 CUs x workgroups resident per CU))
// rounds, and a round costs (workgroups sharing a CU x tile area) divided by a
// per-size MFMA efficiency (larger tiles reuse more of each LDS fragment).
// GEV2_TILE_CFG overrides it (tuning runs).
// `fused` (an act' prologue on one operand) excludes 256x256: its extra
// operand registers would spill with 256 accumulators per lane.
int pick_cfg(int dtype, int64_t M, int64_t N, int64_t batch, bool fused = false) {
  const int forced = env_int("GEV2_TILE_CFG", -1);
  if (forced >= 0) return (fused && forced == gev2::kCfg256x256) ? gev2::kCfg128x256 : forced;
  struct Cand { int cfg, bm, bn, per_cu; double eff; };
  static const Cand cands[] = {
      {gev2::kCfg256x256, 256, 256, 1, 1.0},
      {gev2::kCfg128x256, 128, 256, 1, 0.85},
      {gev2::kCfg128x128, 128, 128, 2, 0.7},
      {gev2::kCfg128x64, 128, 64, 2, 0.6},
      {gev2::kCfg64x64, 64, 64, 4, 0.35},
  };
  (void)dtype;
  int best = gev2::kCfg64x64;
  double best_cost = 1e300;
  for (const Cand& c : cands) {
    if (fused && c.cfg == gev2::kCfg256x256) continue;
    const int64_t tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch;
    const int64_t rounds = (tiles + 256 * c.per_cu - 1) / (256 * c.per_cu);
    const int64_t resident = std::min<int64_t>(c.per_cu, (tiles + 255) / 256);
    const double cost = static_cast<double>(rounds) * resident * c.bm * c.bn / c.eff;
    if (cost < best_cost * 0.999) { best_cost = cost; best = c.cfg; }
  }
  return best;
}

const char* cfg_name(int cfg, bool vec, bool dl = false) {
  if (!vec) return "tile:64x64:scalar";
  if (dl) {
    switch (cfg) {
      case gev2::kCfg256x256: return "dl:256x256";
      case gev2::kCfg128x128: return "dl:128x128";
      case gev2::kCfg128x256: return "dl:128x256";
      case gev2::kCfg64x64: return "dl:64x64";
      case gev2::kCfg128x64: return "dl:128x64";
      default: return "dl:?";
    }
  }
  switch (cfg) {
    case gev2::kCfg256x256: return "tile:256x256";
    case gev2::kCfg128x128: return "tile:128x128";
    case gev2::kCfg64x64: return "tile:64x64";
    case gev2::kCfg128x256: return "tile:128x256";
    case gev2::kCfg128x64: return "tile:128x128";   // launched as 128x128
    default: return "tile:?";
  }
}

std::mutex g_ws_mu;

// True while `s` is being recorded into a HIP graph.  A stream whose capture
// state cannot be read (the null stream while another thread captures in
// global mode) counts as capturing.
bool stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

bool aligned256(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 255u) == 0; }

// Scratch for the forward's split-K partial sums and the backward's dY' when
// the caller passes no workspace: one buffer per (device, stream), grown on
// demand (a stream runs its calls in order, so they can share it).  hipFree
// waits for queued work that may still read the old buffer.
// While the stream is being captured nothing is allocated: a buffer that an
// earlier eager call left large enough is used (so the graph records the same
// kernels as the eager call), and from then on it is pinned: a later growth
// or gev2_stream_destroy retires it without freeing it, since a graph may
// still use it.  Without such a buffer the caller takes a scratch-free path.
struct StreamWs {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool pinned = false;
};
std::map<std::pair<int, hipStream_t>, StreamWs> g_stream_ws;
std::vector<void*> g_pinned_retired;   // kept until the process ends

// *out = the stream's buffer of at least `bytes`, or nullptr when the stream
// is being captured and no such buffer exists yet.
int acquire_stream_ws(hipStream_t s, size_t bytes, void** out) {
  *out = nullptr;
  const bool capturing = stream_capturing(s);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  StreamWs& ws = g_stream_ws[{dev, s}];
  if (ws.bytes < bytes) {
    if (capturing) return GEV2_OK;
    if (ws.ptr) {
      if (ws.pinned) g_pinned_retired.push_back(ws.ptr);
      else (void)hipFree(ws.ptr);
    }
    ws = StreamWs{};
    e = hipMalloc(&ws.ptr, bytes);
    if (e != hipSuccess) {
      ws = StreamWs{};
      return hip_fail(e, "hipMalloc(workspace)");
    }
    ws.bytes = bytes;
  }
  if (capturing) ws.pinned = true;
  *out = ws.ptr;
  return GEV2_OK;
}

int check_common(int dtype, int act, int bias_kind, int64_t M, int64_t N, int64_t K, int64_t batch) {
  if (dtype != GEV2_F32 && dtype != GEV2_F16 && dtype != GEV2_BF16)
    return fail(GEV2_DTYPE_MISMATCH, "dtype must be F32, F16 or BF16");
  if (act < GEV2_ACT_NONE || act > GEV2_ACT_TANH) return fail(GEV2_INVALID_ARGUMENT, "bad act kind");
  if (bias_kind < GEV2_BIAS_NONE || bias_kind > GEV2_BIAS_PER_N)
    return fail(GEV2_INVALID_ARGUMENT, "bad bias kind");
  if (M < 0 || N < 0 || K < 0 || batch < 1) return fail(GEV2_SHAPE_MISMATCH, "negative dims or batch < 1");
  if (!fits_i32(M) || !fits_i32(N) || !fits_i32(K) || !fits_i32(batch))
    return fail(GEV2_INVALID, "dims must fit int32");
  return GEV2_OK;
}

int64_t dense_ld(int64_t ld, int64_t cols) { return ld == 0 ? cols : ld; }

// Validation and path choice of a forward call, shared by gev2_gemm_fwd and
// gev2_gemm_fwd_workspace_size so that the size query always matches the call.
struct FwdPlan {
  bool empty = false;     // M == 0 or N == 0: nothing to launch
  bool skinny = false, split = false;
  int64_t lda = 0, ldb = 0, ldy = 0, ldz = 0;
  int64_t ws_bytes = 0;
  gev2::SkinnyArgs sk{};
  // fp32 split-K on the tile path: ksplit slices of kc (the last kc_last),
  // partial products [ksplit][M][N] fp32 in the workspace (ws_bytes)
  int ksplit = 0;
  int64_t kc = 0, kc_last = 0;
  // small fp32 problem: one launch of the small kernel with this many waves
  // per workgroup (0: not taken)
  int small_waves = 0;
};

// Small fp32 problems run in one launch of the small kernel (16x16 output
// tiles, the reduction split over the waves of a workgroup): at most 512
// tiles, a reduction of 128-2048 and 2^26 multiply-adds, where the tile
// kernels would run as a handful of workgroups (or split K over a second
// pass).  GEV2_NO_SMALL=1 turns it off.

// a small-kernel operand, with its 16-byte-load flag
gev2::SmallOperand small_op(const void* p, int64_t rs, int64_t ks, const void* z = nullptr, int64_t zrs = 0,
                            int64_t zks = 0) {
  gev2::SmallOperand o{static_cast<const float*>(p), rs, ks, static_cast<const float*>(z), zrs, zks, 0};
  o.vec = ks == 1 && rs % 4 == 0 && aligned16(p) && (!z || (zks == 1 && zrs % 4 == 0 && aligned16(z)));
  return o;
}

void plan_small(const gev2_gemm_fwd_desc* d, FwdPlan* pl) {
  const int64_t M = d->M, N = d->N, K = d->K;
  if (d->dtype != GEV2_F32 || d->batch != 1 || env_int("GEV2_NO_SMALL", 0) != 0) return;
  const int64_t tiles = ((M + 15) / 16) * ((N + 15) / 16);
  if (tiles > 512 || K < 128 || K > 2048 || static_cast<double>(M) * N * K > 67108864.0) return;
  pl->small_waves = gev2::small_waves_for(K);
}

// Slices of a split reduction of depth R over `tiles` output tiles: enough
// slices for about 128 workgroups, each at least 16 deep.  A slice depth (a
// multiple of 4) that divides R, with a count within [want/2, 2 want] nearest
// want, keeps every slice in one batched launch; otherwise slices of a
// multiple of 16 and a separate launch for the shorter tail.  False: no split.
bool splitk_slices(int64_t R, int64_t tiles, int64_t* kc_out, int64_t* ks_out) {
  const int64_t want = std::max<int64_t>(2, std::min<int64_t>(R / 32, 128 / std::max<int64_t>(tiles, 1)));
  int64_t kc = 0;
  for (int64_t c = 16; c <= R / 2; c += 4) {
    const int64_t n = R / c;
    if (R % c || 2 * n < want || n > 2 * want) continue;
    if (!kc || std::llabs(n - want) < std::llabs(R / kc - want)) kc = c;
  }
  if (!kc) kc = ((R + want - 1) / want + 15) / 16 * 16;
  const int64_t ks = (R + kc - 1) / kc;
  if (ks < 2) return false;
  *kc_out = kc;
  *ks_out = ks;
  return true;
}

// fp32 problems too small to occupy the GPU with 64x64 tiles (the 64x256
// output of a 784-input MLP layer: 4 tiles on 256 CUs, each running K = 784
// alone) split K over workgroups: slices of kc
// run as one batched launch into fp32 partials, and a
// second pass adds the slices in order and applies alpha, bias, Z and act.
void plan_splitk(const gev2_gemm_fwd_desc* d, FwdPlan* pl) {
  const int64_t M = d->M, N = d->N, K = d->K;
  if (d->dtype != GEV2_F32 || d->batch != 1 || d->trans_a || d->trans_b || env_int("GEV2_NO_SPLITK", 0) != 0)
    return;
  const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
  if (tiles > 32 || K < 256) return;
  if (!vec_ok(d->A, pl->lda, 0, K, M, 1, d->dtype) || !vec_ok(d->B, pl->ldb, 0, N, K, 1, d->dtype)) return;
  if (out_level(d->Y, pl->ldy, 0, M, N, 1, d->dtype) == 0 || out_level(d->Z, pl->ldz, 0, M, N, 1, d->dtype) == 0)
    return;
  int64_t kc = 0, ks = 0;
  if (!splitk_slices(K, tiles, &kc, &ks)) return;
  pl->ksplit = static_cast<int>(ks);
  pl->kc = kc;
  pl->kc_last = K - (ks - 1) * kc;
  pl->ws_bytes = ks * M * N * 4;
}

int plan_fwd(const gev2_gemm_fwd_desc* d, FwdPlan* pl) {
  if (!d) return fail(GEV2_INVALID_ARGUMENT, "null descriptor");
  int st = check_common(d->dtype, d->act, d->bias_kind, d->M, d->N, d->K, d->batch);
  if (st != GEV2_OK) return st;
  const int64_t M = d->M, N = d->N, K = d->K;
  if (!d->Y) return fail(GEV2_MISSING_OUTPUT, "Y is null");
  if (K > 0 && (!d->A || !d->B)) return fail(GEV2_MISSING_INPUT, "A/B is null");
  if (M == 0 || N == 0) {
    pl->empty = true;
    return GEV2_OK;
  }
  const bool ta = d->trans_a != 0, tb = d->trans_b != 0;
  pl->lda = dense_ld(d->lda, ta ? M : K);
  pl->ldb = dense_ld(d->ldb, tb ? K : N);
  pl->ldy = dense_ld(d->ldy, N);
  pl->ldz = dense_ld(d->ldz, N);
  if (pl->lda < (ta ? M : K) || pl->ldb < (tb ? K : N) || pl->ldy < N || (d->Z && pl->ldz < N))
    return fail(GEV2_STRIDE_MISMATCH, "leading dimension smaller than the row length");
  // small fp32 problems, M <= 16 included: the one-launch kernel measured
  // 1.2-2.5x faster than the fp32 skinny dot-product kernel (8x1024x1536:
  // 7.6 against 9.3 us; 16x1024x1024: 5.6 against 13.7 us)
  plan_small(d, pl);
  if (pl->small_waves) return GEV2_OK;
  const int epc = elems_per_chunk(d->dtype);
  pl->skinny = d->batch == 1 && !ta && !tb && M <= gev2::kSkinnyMaxM && K >= 64 && N % epc == 0 &&
               vec_ok(d->B, pl->ldb, 0, N, K, 1, d->dtype) && env_int("GEV2_NO_SKINNY", 0) == 0;
  if (!pl->skinny) {
    plan_splitk(d, pl);
    return GEV2_OK;
  }
  const bool has_bias = d->bias && d->bias_kind != GEV2_BIAS_NONE;
  gev2::SkinnyArgs& a = pl->sk;
  a.A = d->A; a.B = d->B; a.D = d->Y; a.Zo = d->Z;
  a.bias = has_bias ? d->bias : nullptr;
  a.lda = pl->lda; a.ldb = pl->ldb; a.ldd = pl->ldy; a.ldzo = pl->ldz;
  a.M = static_cast<int>(M); a.N = static_cast<int>(N); a.K = static_cast<int>(K);
  a.act = d->act; a.bias_kind = has_bias ? d->bias_kind : GEV2_BIAS_NONE;
  a.slope = d->leaky_slope; a.alpha = d->alpha;
  a.x_vec = (aligned16(d->A) && pl->lda % epc == 0 && K % epc == 0)
                ? (vec_ok(d->A, pl->lda, 0, K, M, 1, d->dtype) ? 2 : 1) : 0;
  pl->split = d->dtype != GEV2_F32 && gev2::skinny_split_eligible(a);
  pl->ws_bytes = pl->split ? gev2::skinny_split_workspace_bytes(a.M, a.N, a.K) : 0;
  return GEV2_OK;
}

}  // namespace

extern "C" {

int gev2_abi_version(void) { return GEV2_ABI_VERSION; }

const char* gev2_last_error(void) { return t_last_error.c_str(); }

int64_t gev2_gemm_fwd_workspace_size(const gev2_gemm_fwd_desc* d) {
  t_last_error.clear();
  FwdPlan pl;
  if (plan_fwd(d, &pl) != GEV2_OK) return -1;
  return pl.empty ? 0 : pl.ws_bytes;
}
const char* gev2_last_path(void) { return t_last_path; }

const char* gev2_status_string(int s) {
  switch (s) {
    case GEV2_OK: return "Ok";
    case GEV2_INVALID: return "Invalid";
    case GEV2_UNIMPLEMENTED: return "Unimplemented";
    case GEV2_RUNTIME_ERROR: return "RuntimeError";
    case GEV2_INVALID_ARGUMENT: return "InvalidArgument";
    case GEV2_MISSING_INPUT: return "MissingInput";
    case GEV2_MISSING_OUTPUT: return "MissingOutput";
    case GEV2_DEVICE_MISMATCH: return "DeviceMismatch";
    case GEV2_DTYPE_MISMATCH: return "DtypeMismatch";
    case GEV2_LAYOUT_MISMATCH: return "LayoutMismatch";
    case GEV2_SHAPE_MISMATCH: return "ShapeMismatch";
    case GEV2_STRIDE_MISMATCH: return "StrideMismatch";
    case GEV2_TRANSPOSE_NOT_SUPPORTED: return "TransposeNotSupported";
    case GEV2_HIP_ERROR: return "HipError";
    default: return "Unknown";
  }
}

int gev2_gemm_fwd(const gev2_gemm_fwd_desc* d, void* stream) { return gev2::gemm_fwd_run(d, stream, nullptr, -1); }

}  // extern "C"

namespace gev2 {

int report_hip_error(hipError_t e, const char* where) { return hip_fail(e, where); }

// The forward.  fixed_bytes < 0: scratch from the caller's workspace, else the
// per-stream buffer (or the scratch-free kernel under capture).  fixed_bytes
// >= 0: scratch only from `fixed` (fixed_bytes of it), nothing allocated, and
// a problem that needs more is refused.
int gemm_fwd_run(const gev2_gemm_fwd_desc* d, void* stream, void* fixed, int64_t fixed_bytes) {
  t_last_error.clear();
  FwdPlan pl;
  int st = plan_fwd(d, &pl);
  if (st != GEV2_OK || pl.empty) return st;
  const int64_t M = d->M, N = d->N, K = d->K;
  const int batch = static_cast<int>(d->batch);
  const bool ta = d->trans_a != 0, tb = d->trans_b != 0;
  const int64_t lda = pl.lda, ldb = pl.ldb, ldy = pl.ldy, ldz = pl.ldz;
  const bool has_bias = d->bias && d->bias_kind != GEV2_BIAS_NONE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  // ---- skinny path ----
  if (pl.skinny) {
    float* part = nullptr;
    if (pl.ws_bytes > 0 && fixed_bytes >= 0) {
      if (pl.ws_bytes > fixed_bytes)
        return fail(GEV2_INVALID_ARGUMENT, "the problem needs " + std::to_string(pl.ws_bytes) +
                                               " bytes of split-K scratch, more than the " +
                                               std::to_string(fixed_bytes) + " bytes available");
      part = static_cast<float*>(fixed);
    } else if (pl.ws_bytes > 0) {
      if (aligned256(d->workspace) && d->workspace_bytes >= pl.ws_bytes) {
        part = static_cast<float*>(d->workspace);
      } else {
        void* w = nullptr;
        st = acquire_stream_ws(s, static_cast<size_t>(pl.ws_bytes), &w);
        if (st != GEV2_OK) return st;
        part = static_cast<float*>(w);
        if (!part) {
          // no scratch under capture: the dot-product kernel, which needs none
          pl.sk.x_vec = std::min(pl.sk.x_vec, 1);
          pl.split = false;
        }
      }
    }
    hipError_t e = gev2::launch_skinny(d->dtype, pl.sk, part, s);
    if (e != hipSuccess) return hip_fail(e, "skinny launch");
    t_last_path = pl.split ? "skinny:split" : "skinny";
    return GEV2_OK;
  }

  // ---- small fp32 problems: one launch, no scratch ----
  if (pl.small_waves > 0) {
    gev2::SmallArgs a{};
    gev2::SmallJob& J = a.job[0];
    J.a = small_op(d->A, ta ? 1 : lda, ta ? lda : 1);
    J.b = small_op(d->B, tb ? ldb : 1, tb ? 1 : ldb);
    J.kind = 0;
    J.rows = static_cast<int>(M); J.cols = static_cast<int>(N); J.red = static_cast<int>(K);
    J.tiles_c = static_cast<int>((N + 15) / 16);
    J.tiles = static_cast<int>((M + 15) / 16) * J.tiles_c;
    J.wgs = J.tiles;
    J.scale = d->alpha;
    J.out = static_cast<float*>(d->Y); J.ldo = ldy;
    a.njobs = 1; a.fwd = 1;
    a.act = d->act; a.slope = d->leaky_slope;
    a.bias = has_bias ? d->bias : nullptr; a.bias_kind = has_bias ? d->bias_kind : GEV2_BIAS_NONE;
    a.Z = static_cast<float*>(d->Z); a.ldz = ldz;
    hipError_t e = gev2::launch_small(a, pl.small_waves, s);
    if (e != hipSuccess) return hip_fail(e, "small launch");
    t_last_path = "small";
    return GEV2_OK;
  }

  // ---- fp32 split-K (small problems): partials in the workspace, else the
  // per-stream buffer; under capture (or past the no-allocation array) the
  // plain tile path below ----
  if (pl.ksplit > 0) {
    float* part = nullptr;
    if (fixed_bytes >= 0) {
      if (pl.ws_bytes <= fixed_bytes) part = static_cast<float*>(fixed);
    } else if (aligned256(d->workspace) && d->workspace_bytes >= pl.ws_bytes) {
      part = static_cast<float*>(d->workspace);
    } else {
      void* w = nullptr;
      st = acquire_stream_ws(s, static_cast<size_t>(pl.ws_bytes), &w);
      if (st != GEV2_OK) return st;
      part = static_cast<float*>(w);
    }
    if (part) {
      const int ks = pl.ksplit;
      const int full = pl.kc_last == pl.kc ? ks : ks - 1;   // slices of depth kc
      const int cfg = pick_cfg(GEV2_F32, M, N, full);
      gev2::TileArgs a{};
      a.A = d->A; a.B = d->B; a.D = part;
      a.lda = lda; a.ldb = ldb; a.ldd = N;
      a.sA = pl.kc; a.sB = pl.kc * ldb; a.sD = M * N;
      a.M = static_cast<int>(M); a.N = static_cast<int>(N); a.K = static_cast<int>(pl.kc);
      a.act = GEV2_ACT_NONE; a.bias_kind = GEV2_BIAS_NONE; a.alpha = 1.f; a.slope = 0.f; a.pro_act = 0;
      const int bm = gev2::tile_bm(cfg, true), bn = gev2::tile_bn(cfg, true);
      a.tiles_m = static_cast<int>((M + bm - 1) / bm);
      a.tiles_n = static_cast<int>((N + bn - 1) / bn);
      a.store_vec = 1;
      hipError_t e = gev2::launch_tile(GEV2_F32, cfg, false, false, 0, true, a, full, s);
      if (e != hipSuccess) return hip_fail(e, "split-K launch");
      if (full < ks) {
        gev2::TileArgs r = a;
        r.A = static_cast<const float*>(d->A) + (int64_t)full * pl.kc;
        r.B = static_cast<const float*>(d->B) + (int64_t)full * pl.kc * ldb;
        r.D = part + (int64_t)full * M * N;
        r.K = static_cast<int>(pl.kc_last);
        e = gev2::launch_tile(GEV2_F32, cfg, false, false, 0, true, r, 1, s);
        if (e != hipSuccess) return hip_fail(e, "split-K launch");
      }
      gev2::SplitkReduceArgs ra{};
      ra.part = part; ra.ks = ks; ra.M = static_cast<int>(M); ra.N = static_cast<int>(N);
      ra.alpha = d->alpha; ra.bias = has_bias ? d->bias : nullptr; ra.bias_kind = has_bias ? d->bias_kind : 0;
      ra.act = d->act; ra.slope = d->leaky_slope;
      ra.Y = static_cast<float*>(d->Y); ra.ldy = ldy; ra.Z = static_cast<float*>(d->Z); ra.ldz = ldz;
      e = gev2::launch_splitk_reduce(ra, s);
      if (e != hipSuccess) return hip_fail(e, "split-K reduction launch");
      t_last_path = "tile:splitk";
      return GEV2_OK;
    }
  }

  // ---- tile path ----
  const bool vec = vec_ok(d->A, lda, d->stride_a, ta ? M : K, ta ? K : M, batch, d->dtype) &&
                   vec_ok(d->B, ldb, d->stride_b, tb ? K : N, tb ? N : K, batch, d->dtype) &&
                   env_int("GEV2_SCALAR_LOADS", 0) == 0;
  const int cfg = pick_cfg(d->dtype, M, N, batch);
  gev2::TileArgs a{};
  a.A = d->A; a.B = d->B; a.D = d->Y; a.Zo = d->Z; a.Zi = nullptr;
  a.bias = has_bias ? d->bias : nullptr; a.dbias = nullptr;
  a.lda = lda; a.ldb = ldb; a.ldd = ldy; a.ldzo = ldz; a.ldzi = 0;
  a.sA = d->stride_a; a.sB = d->stride_b; a.sD = d->stride_y; a.sZo = d->stride_z;
  a.sZi = 0; a.sBias = d->stride_bias; a.sDbias = 0;
  a.M = static_cast<int>(M); a.N = static_cast<int>(N); a.K = static_cast<int>(K);
  a.act = d->act; a.bias_kind = has_bias ? d->bias_kind : GEV2_BIAS_NONE;
  a.slope = d->leaky_slope; a.alpha = d->alpha; a.pro_act = 0;
  const int bm = gev2::tile_bm(cfg, vec), bn = gev2::tile_bn(cfg, vec);
  a.tiles_m = static_cast<int>((M + bm - 1) / bm);
  a.tiles_n = static_cast<int>((N + bn - 1) / bn);
  a.store_vec = std::min(out_level(d->Y, ldy, d->stride_y, M, N, batch, d->dtype),
                         out_level(d->Z, ldz, d->stride_z, M, N, batch, d->dtype));
  if (static_cast<int64_t>(a.tiles_m) * a.tiles_n > 0x7fffffffLL || batch > 65535)
    return fail(GEV2_INVALID, "grid too large");
  hipError_t e = gev2::launch_tile(d->dtype, cfg, ta, tb, 0, vec, a, batch, s);
  if (e != hipSuccess) return hip_fail(e, "tile launch");
  t_last_path = cfg_name(cfg, vec, gev2::dl_selected(d->dtype, cfg, 0, vec, a));
  return GEV2_OK;
}

}  // namespace gev2

namespace {

// Whether the backward materialises dY' = dY (.) act'(Z), the scratch it then
// needs, and where the PerN dBias partials of that pass go.  Shared by
// gev2_gemm_bwd and gev2_gemm_bwd_workspace_size.
//
// The partials (batch x row blocks x N fp32) are parked in an output that is
// written only afterwards: the dX output when it is a dense array (ld = K,
// slices back to back) large enough, else the dW output on the same terms,
// else after dY' in the workspace.  The workspace therefore needs no more than
// dY' itself (batch*M*N elements) in the usual case, which is never more than
// the M*N fp32 dZ buffer the reference's capture-safe backward passes.
enum PartHome { kPartNone = 0, kPartWorkspace = 1, kPartDx = 2, kPartDw = 3 };

struct BwdScratch {
  bool materialise{false}, prep_vec{false}, sums{false};
  // the dW (TN) pass finishes dBias from the partials itself (direct-to-LDS
  // kernel, partials not parked in its own output); it then runs before dX
  bool sums_in_dw{false};
  int row_blocks{0};
  int part_home{kPartNone};
  int64_t gz_bytes{0};     // dY': batch*M*N elements
  int64_t part_bytes{0};   // dBias partials (sums only)
  int64_t need{0};         // what gev2_gemm_bwd_workspace_size reports
  // fp32 dX split over the reduction (N) when dY' is formed while loading:
  // dx_ks slices of dx_kc (the last dx_kc_last), partials [dx_ks][M][K] fp32
  int dx_ks{0};
  int64_t dx_kc{0}, dx_kc_last{0}, dx_bytes{0};
  // the whole backward in one launch of the small kernel, with this many
  // waves per workgroup (0: not taken); needs no scratch
  int small_waves{0};
};

// Small fp32 backward in one launch (dX and dW tiles with dY' formed while
// loading, then the PerN dBias columns): no gC, no PerM / Scalar dBias, at most
// 2048 output tiles, 65536 dY' elements, reductions of at most 2048 and 2^26
// multiply-adds.
// A job whose reduction is at most kSmallOwnRed gives each wave a tile of its
// own; longer ones split each tile's reduction over the workgroup's waves.
constexpr int64_t kSmallOwnRed = 64;

int small_bwd_waves(const gev2_gemm_bwd_desc* d) {
  const int64_t M = d->M, N = d->N, K = d->K;
  const bool want_bias = d->gBias && d->bias_kind != GEV2_BIAS_NONE;
  if (d->dtype != GEV2_F32 || d->batch != 1 || d->gC || env_int("GEV2_NO_SMALL", 0) != 0) return 0;
  if (want_bias && d->bias_kind != GEV2_BIAS_PER_N) return 0;
  if (!d->gA && !d->gB && !want_bias) return 0;
  if (M * N > 65536 || M > 2048 || N > 2048 || static_cast<double>(M) * N * K > 67108864.0) return 0;
  // waves from the longest split reduction (dX: N, dW: M)
  int64_t split_red = 0;
  if (d->gA && N > kSmallOwnRed) split_red = std::max(split_red, N);
  if (d->gB && M > kSmallOwnRed) split_red = std::max(split_red, M);
  const int w = gev2::small_waves_for(split_red);
  // at most 2048 output tiles in all: past that (the rank-8 dW of an RNN step,
  // 6144 tiles) one launch measured no faster than the multi-launch path
  const int64_t tiles = (d->gA ? ((M + 15) / 16) * ((K + 15) / 16) : 0) +
                        (d->gB ? ((K + 15) / 16) * ((N + 15) / 16) : 0);
  return tiles <= 2048 ? w : 0;
}

int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }

BwdScratch bwd_scratch(const gev2_gemm_bwd_desc* d) {
  BwdScratch r;
  const int64_t M = d->M, N = d->N, K = d->K;
  const int batch = static_cast<int>(d->batch), dt = d->dtype;
  const int64_t es = static_cast<int64_t>(elem_size(dt));
  const int64_t ldgy = dense_ld(d->ldgy, N), ldz = dense_ld(d->ldz, N);
  const bool scalar_loads = env_int("GEV2_SCALAR_LOADS", 0) != 0;
  const bool want_bias = d->gBias && d->bias_kind != GEV2_BIAS_NONE;
  const bool linear = d->act == GEV2_ACT_NONE || d->act == GEV2_ACT_RELU || d->act == GEV2_ACT_LEAKY_RELU;
  const double work = static_cast<double>(M) * N * K * batch;
  r.small_waves = small_bwd_waves(d);
  if (r.small_waves > 0) return r;
  r.materialise = (!linear || work >= (1u << 30)) && (d->gA || d->gB) && env_int("GEV2_FUSED_BWD", 0) == 0;
  if (!r.materialise) {
    // small fp32 problems: dX (few 64x64 tiles, long reduction over N) split
    // over workgroups, with the partials in the otherwise unused workspace
    const int64_t lda_b = dense_ld(d->ldb, N), ldga = dense_ld(d->ldga, K);
    const int64_t tiles = ((M + 63) / 64) * ((K + 63) / 64);
    if (dt == GEV2_F32 && batch == 1 && d->gA && M > gev2::kSkinnyMaxM && tiles <= 32 && N >= 256 &&
        !scalar_loads && env_int("GEV2_NO_SPLITK", 0) == 0 && vec_ok(d->gY, ldgy, 0, N, M, 1, dt) &&
        vec_ok(d->Z, ldz, 0, N, M, 1, dt) && vec_ok(d->B, lda_b, 0, N, K, 1, dt) &&
        out_level(d->gA, ldga, 0, M, K, 1, dt) > 0) {
      int64_t kc = 0, ks = 0;
      if (splitk_slices(N, tiles, &kc, &ks)) {
        r.dx_ks = static_cast<int>(ks);
        r.dx_kc = kc;
        r.dx_kc_last = N - (ks - 1) * kc;
        r.dx_bytes = ks * M * K * 4;
        r.need = r.dx_bytes;
      }
    }
    return r;
  }
  const int epc = elems_per_chunk(dt);
  r.prep_vec = !scalar_loads && N % epc == 0 && vec_ok(d->gY, ldgy, d->stride_gy, N, M, batch, dt) &&
               vec_ok(d->Z, ldz, d->stride_z, N, M, batch, dt);
  r.sums = r.prep_vec && want_bias && d->bias_kind == GEV2_BIAS_PER_N;
  r.row_blocks = static_cast<int>((M + gev2::kPrepRows - 1) / gev2::kPrepRows);
  r.gz_bytes = static_cast<int64_t>(batch) * M * N * es;
  r.need = r.gz_bytes;
  if (!r.sums) return r;
  r.part_bytes = static_cast<int64_t>(batch) * r.row_blocks * N * 4;
  const auto dense_home = [&](const void* p, int64_t ld, int64_t stride, int64_t rows, int64_t cols) {
    if (!p || (reinterpret_cast<uintptr_t>(p) & 15u) != 0) return false;
    if (dense_ld(ld, cols) != cols || (batch > 1 && stride != rows * cols)) return false;
    return static_cast<int64_t>(batch) * rows * cols * es >= r.part_bytes;
  };
  if (dense_home(d->gA, d->ldga, d->stride_ga, M, K)) {
    r.part_home = kPartDx;
  } else if (dense_home(d->gB, d->ldgb, d->stride_gb, K, N)) {
    r.part_home = kPartDw;
  } else {
    r.part_home = kPartWorkspace;
    r.need = round256(r.gz_bytes) + r.part_bytes;
  }
  if (d->gB && r.part_home != kPartDw) {
    // the dW pass reads dY' (dense, 16-byte rows) as its B operand
    gev2::TileArgs t{};
    t.store_vec = out_level(d->gB, dense_ld(d->ldgb, N), d->stride_gb, K, N, batch, dt);
    const bool vec = vec_ok(d->A, dense_ld(d->lda, K), d->stride_a, K, M, batch, dt);
    r.sums_in_dw = gev2::dl_selected(dt, pick_cfg(dt, K, N, batch, false), 0, vec, t);
  }
  return r;
}

}  // namespace

extern "C" {

int64_t gev2_gemm_bwd_workspace_size(const gev2_gemm_bwd_desc* d) {
  if (!d || check_common(d->dtype, d->act, d->bias_kind, d->M, d->N, d->K, d->batch) != GEV2_OK) return -1;
  return bwd_scratch(d).need;
}

int gev2_gemm_bwd(const gev2_gemm_bwd_desc* d, void* stream) {
  t_last_error.clear();
  t_last_path = "bwd";
  if (!d) return fail(GEV2_INVALID_ARGUMENT, "null descriptor");
  int st = check_common(d->dtype, d->act, d->bias_kind, d->M, d->N, d->K, d->batch);
  if (st != GEV2_OK) return st;
  const int64_t M = d->M, N = d->N, K = d->K;
  const int batch = static_cast<int>(d->batch);
  if (!d->gY || !d->Z) return fail(GEV2_MISSING_INPUT, "gY/Z is null");
  if (d->gA && !d->B) return fail(GEV2_MISSING_INPUT, "gA requested but B is null");
  if (d->gB && !d->A) return fail(GEV2_MISSING_INPUT, "gB requested but A is null");
  const int64_t lda = dense_ld(d->lda, K), ldb = dense_ld(d->ldb, N);
  const int64_t ldgy = dense_ld(d->ldgy, N), ldz = dense_ld(d->ldz, N);
  const int64_t ldga = dense_ld(d->ldga, K), ldgb = dense_ld(d->ldgb, N), ldgc = dense_ld(d->ldgc, N);
  if (lda < K || ldb < N || ldgy < N || ldz < N || ldga < K || ldgb < N || ldgc < N)
    return fail(GEV2_STRIDE_MISMATCH, "leading dimension smaller than the row length");
  if (M == 0 || N == 0 || K == 0) {
    // the reference rejects empty problems in its backward (regemm_backward.cu:160)
    return fail(GEV2_INVALID_ARGUMENT, "invalid dims");
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int dt = d->dtype;
  const int64_t es = static_cast<int64_t>(elem_size(dt));
  const bool want_bias = d->gBias && d->bias_kind != GEV2_BIAS_NONE;
  const bool scalar_loads = env_int("GEV2_SCALAR_LOADS", 0) != 0;

  // dY' operand of the two GEMMs: gY with act'(Z) applied while the GEMM
  // kernels load it (piecewise-linear activations on small problems), or gZ
  // materialised once in a workspace.  Materialising costs one pass over
  // dY/Z (and yields dBias), but lets both GEMMs use the plain 256x256 kernels;
  // the transcendental activations always take it, so that their act' is
  // evaluated once per element rather than once per workgroup loading it.
  const bool linear = d->act == GEV2_ACT_NONE || d->act == GEV2_ACT_RELU || d->act == GEV2_ACT_LEAKY_RELU;
  const double work = static_cast<double>(M) * N * K * batch;
  const void* G = d->gY;
  int64_t ldG = ldgy, sG = d->stride_gy;
  bool fused = true;
  bool bias_done = false;
  const BwdScratch sc = bwd_scratch(d);
  if (sc.small_waves > 0) {
    // the whole backward in one launch: dX = alpha dY' B^T, dW = alpha A^T dY',
    // dBias = column sums of dY', with dY' = dY (.) act'(Z) formed on load
    gev2::SmallArgs a{};
    const auto* gy = static_cast<const float*>(d->gY);
    const auto* z = static_cast<const float*>(d->Z);
    if (d->gA) {
      gev2::SmallJob& J = a.job[a.njobs++];
      J.a = small_op(gy, ldgy, 1, z, ldz, 1);   // (m, n)
      J.b = small_op(d->B, ldb, 1);             // (k, n) of B [K,N]
      J.kind = 1;
      J.rows = static_cast<int>(M); J.cols = static_cast<int>(K); J.red = static_cast<int>(N);
      J.tiles_c = static_cast<int>((K + 15) / 16);
      J.tiles = static_cast<int>((M + 15) / 16) * J.tiles_c;
      J.own = N <= kSmallOwnRed;
      J.wgs = J.own ? (J.tiles + sc.small_waves - 1) / sc.small_waves : J.tiles;
      J.scale = d->alpha;
      J.out = static_cast<float*>(d->gA); J.ldo = ldga;
    }
    if (d->gB) {
      gev2::SmallJob& J = a.job[a.njobs++];
      J.a = small_op(d->A, 1, lda);             // (k, m) of A [M,K]
      J.b = small_op(gy, 1, ldgy, z, 1, ldz);   // (n, m)
      J.kind = 2;
      J.rows = static_cast<int>(K); J.cols = static_cast<int>(N); J.red = static_cast<int>(M);
      J.tiles_c = static_cast<int>((N + 15) / 16);
      J.tiles = static_cast<int>((K + 15) / 16) * J.tiles_c;
      J.own = M <= kSmallOwnRed;
      J.wgs = J.own ? (J.tiles + sc.small_waves - 1) / sc.small_waves : J.tiles;
      J.scale = d->alpha;
      J.out = static_cast<float*>(d->gB); J.ldo = ldgb;
    }
    a.fwd = 0;
    a.act = d->act; a.slope = d->leaky_slope;
    a.gY = gy; a.ldgy = ldgy; a.Zin = z; a.ldzin = ldz;
    a.gbias = want_bias ? d->gBias : nullptr;
    a.M = static_cast<int>(M); a.N = static_cast<int>(N);
    hipError_t e = gev2::launch_small(a, sc.small_waves, s);
    if (e != hipSuccess) return hip_fail(e, "small backward launch");
    t_last_path = "small";
    return GEV2_OK;
  }
  // Where dY' goes: the caller's workspace when it holds dY'; otherwise the
  // per-stream buffer.  Under graph capture without either (nothing is
  // allocated then) the GEMMs apply act' to dY on load instead for none /
  // ReLU / LeakyReLU, and the transcendental activations are refused.
  void* ws = nullptr;
  bool sums = sc.sums;
  const float* dw_part = nullptr;     // dBias partials the dW pass finishes
  int64_t dw_part_stride = 0;
  if (sc.materialise) {
    if (aligned256(d->workspace) && d->workspace_bytes >= sc.gz_bytes) {
      ws = d->workspace;
      // partials parked after dY' need the larger size; without it dBias
      // falls back to the column-sum kernel below
      if (sums && sc.part_home == kPartWorkspace && d->workspace_bytes < sc.need) sums = false;
    } else {
      st = acquire_stream_ws(s, static_cast<size_t>(sc.need), &ws);
      if (st != GEV2_OK) return st;
    }
    if (!ws && !linear) {
      // under capture with no scratch: act' is applied on load for the
      // piecewise-linear activations only
      return fail(GEV2_MISSING_INPUT, "the stream is being captured into a graph: a GELU / Sigmoid / Tanh backward "
                                      "needs a dY' workspace of " + std::to_string(sc.gz_bytes) +
                                      " bytes (nothing is allocated during capture)");
    }
  }
  if (ws) {
    const bool prep_vec = sc.prep_vec;
    const int row_blocks = sc.row_blocks;
    float* partial = nullptr;
    if (sums) {
      partial = sc.part_home == kPartDx   ? static_cast<float*>(d->gA)
                : sc.part_home == kPartDw ? static_cast<float*>(d->gB)
                                          : reinterpret_cast<float*>(static_cast<char*>(ws) + round256(sc.gz_bytes));
    }
    hipError_t e;
    if (prep_vec) {
      gev2::PrepArgs pa{};
      pa.gY = d->gY; pa.Z = d->Z; pa.out = ws; pa.partial = partial;
      pa.ldgy = ldgy; pa.ldz = ldz;
      pa.sgY = d->stride_gy; pa.sZ = d->stride_z; pa.sOut = M * N;
      pa.sPartial = static_cast<int64_t>(row_blocks) * N;
      pa.M = static_cast<int>(M); pa.N = static_cast<int>(N);
      pa.act = d->act; pa.slope = d->leaky_slope;
      if (want_bias && d->bias_kind == GEV2_BIAS_PER_M) {
        // row sums of dY' are the PerM bias gradient
        pa.rowsum = d->gBias; pa.sRowsum = d->stride_gbias;
        bias_done = true;
      }
      e = gev2::launch_grad_prep(dt, pa, batch, s);
      if (e != hipSuccess) return hip_fail(e, "gZ launch");
      if (sums && sc.sums_in_dw) {
        dw_part = partial;
        dw_part_stride = pa.sPartial;
      } else if (sums) {
        e = gev2::launch_finish_col_sums(partial, pa.sPartial, row_blocks, static_cast<int>(N), d->gBias,
                                         d->stride_gbias, batch, s);
        if (e != hipSuccess) return hip_fail(e, "dBias launch");
        bias_done = true;
      }
    } else {
      gev2::GradArgs g{};
      g.gY = d->gY; g.Z = d->Z; g.out = ws; g.gbias = nullptr;
      g.ldgy = ldgy; g.ldz = ldz; g.ldout = N;
      g.sgY = d->stride_gy; g.sZ = d->stride_z; g.sOut = M * N; g.sGbias = 0;
      g.M = static_cast<int>(M); g.N = static_cast<int>(N);
      g.act = d->act; g.slope = d->leaky_slope; g.beta = 1.0f; g.bias_kind = GEV2_BIAS_NONE;
      e = gev2::launch_grad_elementwise(dt, g, batch, s);
      if (e != hipSuccess) return hip_fail(e, "gZ launch");
    }
    G = ws; ldG = N; sG = M * N;
    fused = false;
  }
  const bool fuse_bias = fused && want_bias && d->bias_kind == GEV2_BIAS_PER_N && d->gB != nullptr;
  const bool gyz_vec = vec_ok(G, ldG, sG, N, M, batch, dt) &&
                       (!fused || vec_ok(d->Z, ldz, d->stride_z, N, M, batch, dt)) && !scalar_loads;

  // scratch of the fp32 dX split: the caller's workspace, else the stream's
  // buffer (none under capture without one: the unsplit launch then)
  // (a caller workspace too small for them means no split: a call that passes
  // scratch, like the reference's capture-safe backward with its M*N dZ,
  // never reaches the library's buffer)
  float* dx_part = nullptr;
  if (d->gA && fused && sc.dx_ks > 0) {
    if (aligned256(d->workspace) && d->workspace_bytes >= sc.dx_bytes) {
      dx_part = static_cast<float*>(d->workspace);
    } else if (!d->workspace) {
      void* w = nullptr;
      st = acquire_stream_ws(s, static_cast<size_t>(sc.dx_bytes), &w);
      if (st != GEV2_OK) return st;
      dx_part = static_cast<float*>(w);
    }
  }
  // gA[M,K] = alpha * dY' [M,N] * B^T : NT (prologue on A when fused)
  auto run_dx = [&]() -> int {
    if (!d->gA) return GEV2_OK;
    const bool vec = gyz_vec && vec_ok(d->B, ldb, d->stride_b, N, K, batch, dt);
    if (M <= gev2::kSkinnyMaxM && batch == 1 && vec && env_int("GEV2_NO_SKINNY", 0) == 0) {
      // one wave per output column, each reading one row of B
      gev2::SkinnyNtArgs n{};
      n.G = G; n.Z = fused ? d->Z : nullptr; n.B = d->B; n.D = d->gA;
      n.ldg = ldG; n.ldz = ldz; n.ldb = ldb; n.ldd = ldga;
      n.M = static_cast<int>(M); n.N = static_cast<int>(N); n.K = static_cast<int>(K);
      n.act = d->act; n.slope = d->leaky_slope; n.alpha = d->alpha;
      hipError_t e = gev2::launch_skinny_nt(dt, n, s);
      if (e != hipSuccess) return hip_fail(e, "dX skinny launch");
    } else if (float* part = dx_part) {
      // dX split over N: slices into fp32 partials, then an ordered sum (alpha)
      const int ks = sc.dx_ks;
      const int full = sc.dx_kc_last == sc.dx_kc ? ks : ks - 1;
      const int cfg = pick_cfg(dt, M, K, full, true);
      gev2::TileArgs a{};
      a.A = G; a.lda = ldG; a.sA = sc.dx_kc;
      a.Zi = d->Z; a.ldzi = ldz; a.sZi = sc.dx_kc;
      a.B = d->B; a.ldb = ldb; a.sB = sc.dx_kc;
      a.D = part; a.ldd = K; a.sD = M * K;
      a.M = static_cast<int>(M); a.N = static_cast<int>(K); a.K = static_cast<int>(sc.dx_kc);
      a.act = GEV2_ACT_NONE; a.bias_kind = GEV2_BIAS_NONE; a.alpha = 1.f;
      a.slope = d->leaky_slope; a.pro_act = d->act;
      const int bm = gev2::tile_bm(cfg, true), bn = gev2::tile_bn(cfg, true);
      a.tiles_m = static_cast<int>((M + bm - 1) / bm);
      a.tiles_n = static_cast<int>((K + bn - 1) / bn);
      a.store_vec = 1;
      hipError_t e = gev2::launch_tile(dt, cfg, false, true, 1, true, a, full, s);
      if (e != hipSuccess) return hip_fail(e, "dX split launch");
      if (full < ks) {
        gev2::TileArgs r = a;
        r.A = static_cast<const float*>(G) + (int64_t)full * sc.dx_kc;
        r.Zi = static_cast<const float*>(d->Z) + (int64_t)full * sc.dx_kc;
        r.B = static_cast<const float*>(d->B) + (int64_t)full * sc.dx_kc;
        r.D = part + (int64_t)full * M * K;
        r.K = static_cast<int>(sc.dx_kc_last);
        e = gev2::launch_tile(dt, cfg, false, true, 1, true, r, 1, s);
        if (e != hipSuccess) return hip_fail(e, "dX split launch");
      }
      gev2::SplitkReduceArgs ra{};
      ra.part = part; ra.ks = ks; ra.M = static_cast<int>(M); ra.N = static_cast<int>(K);
      ra.alpha = d->alpha; ra.bias = nullptr; ra.bias_kind = 0; ra.act = GEV2_ACT_NONE; ra.slope = 0.f;
      ra.Y = static_cast<float*>(d->gA); ra.ldy = ldga; ra.Z = nullptr; ra.ldz = 0;
      e = gev2::launch_splitk_reduce(ra, s);
      if (e != hipSuccess) return hip_fail(e, "dX split reduction launch");
    } else {
      const int cfg = pick_cfg(dt, M, K, batch, fused);
      gev2::TileArgs a{};
      a.A = G; a.lda = ldG; a.sA = sG;
      a.Zi = fused ? d->Z : nullptr; a.ldzi = ldz; a.sZi = d->stride_z;
      a.B = d->B; a.ldb = ldb; a.sB = d->stride_b;
      a.D = d->gA; a.ldd = ldga; a.sD = d->stride_ga;
      a.M = static_cast<int>(M); a.N = static_cast<int>(K); a.K = static_cast<int>(N);
      a.act = GEV2_ACT_NONE; a.bias_kind = GEV2_BIAS_NONE; a.alpha = d->alpha;
      a.slope = d->leaky_slope; a.pro_act = d->act;
      const int bm = gev2::tile_bm(cfg, vec), bn = gev2::tile_bn(cfg, vec);
      a.tiles_m = static_cast<int>((M + bm - 1) / bm);
      a.tiles_n = static_cast<int>((K + bn - 1) / bn);
      a.store_vec = out_level(d->gA, ldga, d->stride_ga, M, K, batch, dt);
      hipError_t e = gev2::launch_tile(dt, cfg, false, true, fused ? 1 : 0, vec, a, batch, s);
      if (e != hipSuccess) return hip_fail(e, "dX launch");
    }
    return GEV2_OK;
  };
  // gB[K,N] = alpha * A^T [K,M] * dY' [M,N] : TN (prologue on B + fused dBias
  // when fused; on a materialised dY' the direct-to-LDS kernel can finish
  // dBias from grad_prep's partials)
  auto run_dw = [&]() -> int {
    if (!d->gB) return GEV2_OK;
    const bool vec = gyz_vec && vec_ok(d->A, lda, d->stride_a, K, M, batch, dt);
    const int cfg = pick_cfg(dt, K, N, batch, fused);
    gev2::TileArgs a{};
    a.A = d->A; a.lda = lda; a.sA = d->stride_a;
    a.B = G; a.ldb = ldG; a.sB = sG;
    a.Zi = fused ? d->Z : nullptr; a.ldzi = ldz; a.sZi = d->stride_z;
    a.D = d->gB; a.ldd = ldgb; a.sD = d->stride_gb;
    a.dbias = fuse_bias ? d->gBias : nullptr; a.sDbias = d->stride_gbias;
    a.M = static_cast<int>(K); a.N = static_cast<int>(N); a.K = static_cast<int>(M);
    a.act = GEV2_ACT_NONE; a.bias_kind = GEV2_BIAS_NONE; a.alpha = d->alpha;
    a.slope = d->leaky_slope; a.pro_act = d->act;
    const int bm = gev2::tile_bm(cfg, vec), bn = gev2::tile_bn(cfg, vec);
    a.tiles_m = static_cast<int>((K + bm - 1) / bm);
    a.tiles_n = static_cast<int>((N + bn - 1) / bn);
    a.store_vec = out_level(d->gB, ldgb, d->stride_gb, K, N, batch, dt);
    if (dw_part) {
      if (gev2::dl_selected(dt, cfg, 0, vec, a)) {
        a.dbias = d->gBias; a.sDbias = d->stride_gbias;
        a.dbias_part = dw_part; a.sDbiasPart = dw_part_stride; a.dbias_rb = sc.row_blocks;
      } else {
        hipError_t e = gev2::launch_finish_col_sums(dw_part, dw_part_stride, sc.row_blocks, static_cast<int>(N),
                                                    d->gBias, d->stride_gbias, batch, s);
        if (e != hipSuccess) return hip_fail(e, "dBias launch");
      }
      bias_done = true;
    }
    hipError_t e = gev2::launch_tile(dt, cfg, true, false, fused ? 2 : 0, vec, a, batch, s);
    if (e != hipSuccess) return hip_fail(e, "dW launch");
    return GEV2_OK;
  };
  // dW first when it reads dBias partials parked in the dX output
  st = dw_part ? run_dw() : run_dx();
  if (st != GEV2_OK) return st;
  st = dw_part ? run_dx() : run_dw();
  if (st != GEV2_OK) return st;
  if (d->gC || (want_bias && !fuse_bias && !bias_done)) {
    gev2::GradArgs g{};
    g.gY = d->gY; g.Z = d->Z; g.out = d->gC; g.gbias = d->gBias;
    g.ldgy = ldgy; g.ldz = ldz; g.ldout = ldgc;
    g.sgY = d->stride_gy; g.sZ = d->stride_z; g.sOut = d->stride_gc; g.sGbias = d->stride_gbias;
    g.M = static_cast<int>(M); g.N = static_cast<int>(N);
    g.act = d->act; g.slope = d->leaky_slope; g.beta = d->beta; g.bias_kind = d->bias_kind;
    if (d->gC) {
      hipError_t e = gev2::launch_grad_elementwise(dt, g, batch, s);
      if (e != hipSuccess) return hip_fail(e, "gC launch");
    }
    if (want_bias && !fuse_bias && !bias_done) {
      hipError_t e = gev2::launch_bias_grad(dt, g, batch, s);
      if (e != hipSuccess) return hip_fail(e, "bias-grad launch");
    }
  }
  return GEV2_OK;
}

int gev2_gemm_fwd_repeat(const gev2_gemm_fwd_desc* descs, int n_descs, int reps, void* stream) {
  if (!descs || n_descs < 1 || reps < 0) return fail(GEV2_INVALID_ARGUMENT, "bad repeat arguments");
  for (int i = 0; i < reps; ++i) {
    const int st = gev2_gemm_fwd(descs + (i % n_descs), stream);
    if (st != GEV2_OK) return st;
  }
  return GEV2_OK;
}

int gev2_gemm_bwd_repeat(const gev2_gemm_bwd_desc* descs, int n_descs, int reps, void* stream) {
  if (!descs || n_descs < 1 || reps < 0) return fail(GEV2_INVALID_ARGUMENT, "bad repeat arguments");
  for (int i = 0; i < reps; ++i) {
    const int st = gev2_gemm_bwd(descs + (i % n_descs), stream);
    if (st != GEV2_OK) return st;
  }
  return GEV2_OK;
}

// ---------------------------------------------------------------------------
// Runtime helpers
// ---------------------------------------------------------------------------
#define GEV2_HIP_CALL(expr, where)                   \
  do {                                               \
    hipError_t e_ = (expr);                          \
    if (e_ != hipSuccess) return hip_fail(e_, where); \
  } while (0)

int gev2_device_count(int* count) {
  GEV2_HIP_CALL(hipGetDeviceCount(count), "hipGetDeviceCount");
  return GEV2_OK;
}
int gev2_set_device(int device) {
  GEV2_HIP_CALL(hipSetDevice(device), "hipSetDevice");
  return GEV2_OK;
}
int gev2_get_device(int* device) {
  GEV2_HIP_CALL(hipGetDevice(device), "hipGetDevice");
  return GEV2_OK;
}
int gev2_device_info(int device, char* name, size_t name_len, int* cu_count, int* clock_khz) {
  hipDeviceProp_t prop;
  GEV2_HIP_CALL(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (name && name_len) {
    std::snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  return GEV2_OK;
}
int gev2_malloc(void** ptr, size_t bytes) {
  GEV2_HIP_CALL(hipMalloc(ptr, bytes), "hipMalloc");
  return GEV2_OK;
}
int gev2_free(void* ptr) {
  if (t_captures > 0) {
    // hipFree is not allowed while this thread captures (it would invalidate
    // the graph): release the memory when the capture ends
    t_deferred_frees.push_back(ptr);
    return GEV2_OK;
  }
  GEV2_HIP_CALL(hipFree(ptr), "hipFree");
  return GEV2_OK;
}
int gev2_memcpy_htod(void* dst, const void* src, size_t bytes) {
  GEV2_HIP_CALL(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  return GEV2_OK;
}
int gev2_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  GEV2_HIP_CALL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return GEV2_OK;
}
int gev2_memcpy_dtod_async(void* dst, const void* src, size_t bytes, void* stream) {
  GEV2_HIP_CALL(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                               reinterpret_cast<hipStream_t>(stream)),
                "hipMemcpyAsync D2D");
  return GEV2_OK;
}
int gev2_memset(void* ptr, int value, size_t bytes) {
  GEV2_HIP_CALL(hipMemset(ptr, value, bytes), "hipMemset");
  return GEV2_OK;
}
int gev2_stream_create(void** stream) {
  hipStream_t s;
  GEV2_HIP_CALL(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = s;
  return GEV2_OK;
}
int gev2_stream_destroy(void* stream) {
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    for (auto it = g_stream_ws.begin(); it != g_stream_ws.end();) {
      if (it->first.second == reinterpret_cast<hipStream_t>(stream)) {
        (void)hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
        if (it->second.pinned) g_pinned_retired.push_back(it->second.ptr);
        else if (it->second.ptr) (void)hipFree(it->second.ptr);
        it = g_stream_ws.erase(it);
      } else {
        ++it;
      }
    }
  }
  GEV2_HIP_CALL(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)), "hipStreamDestroy");
  return GEV2_OK;
}
int gev2_stream_synchronize(void* stream) {
  GEV2_HIP_CALL(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)), "hipStreamSynchronize");
  return GEV2_OK;
}
int gev2_device_synchronize(void) {
  GEV2_HIP_CALL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return GEV2_OK;
}
int gev2_event_create(void** event) {
  hipEvent_t e;
  GEV2_HIP_CALL(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return GEV2_OK;
}
int gev2_event_destroy(void* event) {
  GEV2_HIP_CALL(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy");
  return GEV2_OK;
}
int gev2_event_record(void* event, void* stream) {
  GEV2_HIP_CALL(hipEventRecord(reinterpret_cast<hipEvent_t>(event), reinterpret_cast<hipStream_t>(stream)),
                "hipEventRecord");
  return GEV2_OK;
}
int gev2_event_synchronize(void* event) {
  GEV2_HIP_CALL(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "hipEventSynchronize");
  return GEV2_OK;
}
int gev2_event_elapsed_ms(float* ms, void* start, void* stop) {
  GEV2_HIP_CALL(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)),
                "hipEventElapsedTime");
  return GEV2_OK;
}

// HIP graph capture of a stream's work (thread-local capture mode: other
// threads' HIP calls are unaffected).  The operator calls allocate nothing
// while their stream is capturing (acquire_stream_ws; without scratch the
// forward and backward take their scratch-free paths).
int gev2_graph_begin(void* stream) {
  if (!stream) return fail(GEV2_INVALID_ARGUMENT, "capture needs a created stream, not the null stream");
  GEV2_HIP_CALL(hipStreamBeginCapture(reinterpret_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal),
                "hipStreamBeginCapture");
  ++t_captures;
  return GEV2_OK;
}
int gev2_graph_end(void* stream, void** exec) {
  if (!exec) return fail(GEV2_INVALID_ARGUMENT, "exec is null");
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(reinterpret_cast<hipStream_t>(stream), &g);
  if (t_captures > 0 && --t_captures == 0) {
    // the frees asked for during the capture
    for (void* p : t_deferred_frees) (void)hipFree(p);
    t_deferred_frees.clear();
  }
  if (ec != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return hip_fail(ec, "hipStreamEndCapture");
  }
  hipGraphExec_t e = nullptr;
  const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (err != hipSuccess) return hip_fail(err, "hipGraphInstantiate");
  *exec = e;
  return GEV2_OK;
}
int gev2_graph_launch(void* exec, void* stream) {
  GEV2_HIP_CALL(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), reinterpret_cast<hipStream_t>(stream)),
                "hipGraphLaunch");
  return GEV2_OK;
}
int gev2_graph_destroy(void* exec) {
  GEV2_HIP_CALL(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)), "hipGraphExecDestroy");
  return GEV2_OK;
}

}  // extern "C"
