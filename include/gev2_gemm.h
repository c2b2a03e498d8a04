/*
 * gev2_gemm.h -- C ABI of the MI355X (gfx950) GEMM + bias + activation
 * operator (libgev2.so).
 *
 * This is the thin C layer that the C++ host code behind the Python binding
 * (graph_executor_v2.ops._ops_gemm) calls.  It replaces, one for one:
 *   gev2_gemm_fwd  <- ai::cuda::shim::GemmCudaLaunch
 *                     (graph_executor_v2/backends/cuda/ops/gemm/api.hpp:124-134,
 *                      launcher.cu:147-274) and, with batch > 1 or a transpose,
 *                     the per-slice GEMM loops of conv2d/launcher.cu:180-227 and
 *                     sdpa/launcher.cu:185-270
 *   gev2_gemm_bwd  <- ai::cuda::shim::GemmCudaBackward / GemmCudaBackwardInto
 *                     (gemm/api.hpp:150-163, 166-188, launcher.cu:279-383,
 *                      kernels/regemm_backward.cu:151-301)
 * Its descriptor style (one POD of pointers, sizes and enums per call) follows
 * the reference's earlier C ABI, dev/backend/graph_executor_v2/include/
 * ge_v2_api_ex.h:37-134.
 *
 * Conventions
 *   - All matrices are row-major.  Leading dimensions (ld*) and batch strides
 *     (stride_*) are in elements.  ld* == 0 means "dense" (number of columns).
 *   - dtype applies to A, B, Y, Z, gY, gA, gB, gC; bias and gBias are float32.
 *   - Return values are the reference's Status codes (enums.hpp / ai_status.hpp):
 *     GEV2_HIP_ERROR (130) is the reference's CUDA_ERROR slot.  The functions
 *     never throw; gev2_last_error() gives a message for the calling thread.
 *   - Calls are asynchronous on `stream` (a hipStream_t; NULL = null stream).
 *   - Device memory is allocated only for scratch that the caller did not
 *     pass in `workspace`: the forward's split-K partial sums (skinny 16-bit
 *     problems, and fp32 problems of at most 32 64x64 tiles with K >= 256;
 *     gev2_gemm_fwd_workspace_size gives the size, 0 for all other problems)
 *     and the backward's materialised dY'.  Such a buffer is allocated once
 *     per (device, stream) and kept until gev2_stream_destroy.
 *   - Nothing is allocated while `stream` is being captured into a HIP graph.
 *     A per-stream buffer that an earlier eager call left large enough is
 *     used (the graph then holds the same kernels as the eager call) and is
 *     kept from then on until the process ends.  Without it, the forward uses
 *     its scratch-free kernels, and the backward applies act' to dY as its
 *     GEMMs load it (none / ReLU / LeakyReLU) or, for GELU / Sigmoid / Tanh,
 *     which need dY' in a workspace, returns GEV2_MISSING_INPUT.
 */
#ifndef GEV2_GEMM_H_
#define GEV2_GEMM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEV2_ABI_VERSION 4

/* Status (values of ai::cuda::shim::Status, ai_status.hpp:14-43) */
enum {
  GEV2_OK = 0,
  GEV2_INVALID = 1,
  GEV2_UNIMPLEMENTED = 2,
  GEV2_RUNTIME_ERROR = 3,
  GEV2_INVALID_ARGUMENT = 4,
  GEV2_MISSING_INPUT = 10,
  GEV2_MISSING_OUTPUT = 11,
  GEV2_DEVICE_MISMATCH = 100,
  GEV2_DTYPE_MISMATCH = 101,
  GEV2_LAYOUT_MISMATCH = 102,
  GEV2_SHAPE_MISMATCH = 103,
  GEV2_STRIDE_MISMATCH = 104,
  GEV2_TRANSPOSE_NOT_SUPPORTED = 105,
  GEV2_HIP_ERROR = 130,
  GEV2_UNKNOWN = 999
};

/* DType (ai_device.hpp:14-27), ActKind and BiasKind (enums.hpp:10-24) */
enum { GEV2_F32 = 0, GEV2_F16 = 1, GEV2_BF16 = 2 };
enum { GEV2_ACT_NONE = 0, GEV2_ACT_RELU = 1, GEV2_ACT_LEAKY_RELU = 2, GEV2_ACT_GELU = 3,
       GEV2_ACT_SIGMOID = 4, GEV2_ACT_TANH = 5 };
enum { GEV2_BIAS_NONE = 0, GEV2_BIAS_SCALAR = 1, GEV2_BIAS_PER_M = 2, GEV2_BIAS_PER_N = 3 };

/*
 * Forward, for each slice b < batch:
 *   Z_b = alpha * op(A_b) op(B_b) + bias_b          (op(A) is [M,K], op(B) is [K,N])
 *   Y_b = act(Z_b)
 * trans_a = 0: A is [M,K] (lda >= K);  1: A is stored [K,M] (lda >= M).
 * trans_b = 0: B is [K,N] (ldb >= N);  1: B is stored [N,K] (ldb >= K).
 * Z may be NULL (no pre-activation stash); Z == Y is allowed.
 * bias may be NULL or bias_kind NONE; PerN indexes bias[n], PerM bias[m].
 * Replaces GemmCudaLaunch (launcher.cu:147-274), which only has batch = 1,
 * alpha = 1 and no transposes (it returns TransposeNotSupported for them).
 * workspace: optional scratch (256-byte aligned) of at least
 * gev2_gemm_fwd_workspace_size(desc) bytes; NULL or too small makes the
 * library use its own per-(device, stream) buffer (outside graph capture).
 * Plays the role of the reference's GemmWorkspace (gemm/api.hpp:97-104,
 * GemmCudaLaunch's ws).
 */
typedef struct gev2_gemm_fwd_desc {
  int32_t dtype;
  int32_t act;
  int32_t bias_kind;
  int32_t trans_a;
  int32_t trans_b;
  float leaky_slope;
  float alpha;
  int32_t reserved0;
  int64_t M, N, K, batch;
  const void* A;     int64_t lda, stride_a;
  const void* B;     int64_t ldb, stride_b;
  const float* bias; int64_t stride_bias;
  void* Y;           int64_t ldy, stride_y;
  void* Z;           int64_t ldz, stride_z;
  void* workspace;   int64_t workspace_bytes;
} gev2_gemm_fwd_desc;

/*
 * Backward of the forward above (trans_a = trans_b = 0), for each slice:
 *   gZ = gY (.) act'(Z)                       (never written to memory)
 *   gA = alpha * gZ B^T        [M,K]   (optional)
 *   gB = alpha * A^T gZ        [K,N]   (optional)
 *   gC = beta * gZ             [M,N]   (optional)
 *   gBias = sum of gZ over rows (PER_N, [N]) / columns (PER_M, [M]) / all (SCALAR)
 * Replaces GemmCudaBackward (launcher.cu:279-383 + regemm_backward.cu:151-301).
 * gBias is overwritten (the reference zero-fills it first, :190-197).
 * gZ is either formed while the GEMM kernels load their operands (act none /
 * ReLU / LeakyReLU on problems below 2^30 multiply-adds, and every activation
 * in the one-launch fp32 backward of small problems: no gC, no PerM / Scalar
 * dBias, at most 2048 16x16 output tiles and 65536 gZ elements) or written
 * once to `workspace` by a pass that also sums dBias, after which the two GEMMs
 * read it.
 */
typedef struct gev2_gemm_bwd_desc {
  int32_t dtype;
  int32_t act;
  int32_t bias_kind;
  float leaky_slope;
  float alpha;
  float beta;
  int64_t M, N, K, batch;
  const void* A;  int64_t lda, stride_a;
  const void* B;  int64_t ldb, stride_b;
  const void* gY; int64_t ldgy, stride_gy;
  const void* Z;  int64_t ldz, stride_z;
  void* gA;       int64_t ldga, stride_ga;
  void* gB;       int64_t ldgb, stride_gb;
  void* gC;       int64_t ldgc, stride_gc;
  float* gBias;   int64_t stride_gbias;
  /* Optional scratch (256-byte aligned) for dY' = dY (.) act'(Z): batch*M*N
   * elements of dtype.  Used when gZ is materialised: always for GELU /
   * Sigmoid / Tanh, and for large problems (M*N*K*batch >= 2^30).  A PerN
   * dBias is summed by the same pass into batch*ceil(M/64)*N float partials,
   * parked in the gA output when gA is dense (ldga = K, slices back to back)
   * and large enough, else in a dense gB, else after dY' in this workspace
   * (then rounded up to 256 bytes; gev2_gemm_bwd_workspace_size includes
   * them).  So the reference's M*N fp32 dZ scratch always holds what is
   * needed.  NULL or too small for dY': the library uses a buffer it
   * allocates once per (device, stream) and keeps, or, while the stream is
   * being captured, forms dY' while loading instead (none / ReLU / LeakyReLU;
   * other activations return GEV2_MISSING_INPUT then).  The one-launch
   * backward of small fp32 problems needs no workspace for any activation.  Plays the role of the
   * reference's GemmWorkspace::scratch (gemm/api.hpp:97-104). */
  void* workspace; int64_t workspace_bytes;
} gev2_gemm_bwd_desc;

int gev2_gemm_fwd(const gev2_gemm_fwd_desc* desc, void* stream);
/* The forward above, allocating nothing, ever.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The only
 * scratch the forward uses, the split-K partial sums of skinny 16-bit
 * problems (gev2_gemm_fwd_workspace_size), is taken from a fixed 16 MiB device
 * array that each GPU holds until the process ends; desc->workspace is
 * ignored.  A problem needing more than 16 MiB of it returns
 * GEV2_INVALID_ARGUMENT (2 MiB at M = 8, N = K = 4096).  Every call on a GPU
 * shares that GPU's array and overwrites what it uses (nothing needs to start
 * at zero), so calls that overlap on one GPU (on different streams) race.
 * Results are bit-identical to gev2_gemm_fwd's. */
int gev2_gemm_fwd_noalloc(const gev2_gemm_fwd_desc* desc, void* stream);
/* Scratch bytes gev2_gemm_fwd uses for `desc` (0: none); -1 for an invalid
 * descriptor.  No counterpart in the reference (its forward needs none). */
int64_t gev2_gemm_fwd_workspace_size(const gev2_gemm_fwd_desc* desc);
int gev2_gemm_bwd(const gev2_gemm_bwd_desc* desc, void* stream);
/* Scratch bytes gev2_gemm_bwd uses for `desc` (0: none, dY' is formed while
 * loading); -1 for an invalid descriptor.  A `workspace` this large (256-byte
 * aligned) keeps the call off the per-stream buffer; one of batch*M*N
 * elements does too, with dBias then summed by a separate column pass when
 * its partials had no other home.  No counterpart in the reference (its
 * scratch is GemmWorkspace::scratch, sized by the caller). */
int64_t gev2_gemm_bwd_workspace_size(const gev2_gemm_bwd_desc* desc);

/*
 * 2-D convolution, NCHW, groups = 1, on the operator (replaces
 * Conv2DCudaLaunch / Conv2DCudaBackwardLaunch, conv2d/api.hpp:47-69,
 * conv2d/launcher.cu:106-459):
 *   Ho = (H + 2*pad_h - dil_h*(Kh-1) - 1) / stride_h + 1, likewise Wo;
 *   Z[n,co,ho,wo] = sum_{c,kh,kw} W[co,c,kh,kw] * X[n,c,ho*stride_h-pad_h+kh*dil_h,
 *                   wo*stride_w-pad_w+kw*dil_w] (zero outside) + bias[co];  Y = act(Z).
 * X [N,Cin,H,W], W [Cout,Cin,Kh,Kw], bias [Cout] fp32 (optional), Y / Z
 * [N,Cout,Ho,Wo], all contiguous.  K = Cin*Kh*Kw, HWo = Ho*Wo.
 * col: im2col workspace of at least K*HWo elements (one image); a larger one
 * lets one GEMM launch cover floor(col_bytes / (K*HWo*elem)) images.
 */
typedef struct gev2_conv2d_desc {
  int32_t dtype;
  int32_t act;
  float leaky_slope;
  int32_t save_z;                 /* 1: write Z (must be non-NULL) */
  int32_t N, Cin, H, W, Cout, Kh, Kw;
  int32_t stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, groups;
  const void* X;
  const void* Wt;
  const float* bias;
  void* Y;
  void* Z;
  void* col;  int64_t col_bytes;
} gev2_conv2d_desc;

/*
 * Backward: dW [Cout,Cin,Kh,Kw], dB [Cout] fp32, dX [N,Cin,H,W] (each optional),
 * from dY and the saved Z (both [N,Cout,Ho,Wo]); dW and dB are sums over all
 * images.  Workspaces, per image of a chunk (elements of dtype unless noted):
 *   col         K*HWo            im2col (always)
 *   dcol        K*HWo            gradient columns (when dX)
 *   gw          Cout*K           that image's dW (when dW)
 *   acc_b       Cout floats      that image's dB, after Cout floats of the sum (when dB)
 * and once:
 *   acc_w       Cout*K floats    fp32 sum of dW over images (when dW)
 *   dz          optional dY' scratch of the operator backward (see
 *               gev2_gemm_bwd_desc.workspace), dz_bytes its size
 * One batched operator backward covers as many images as every workspace in
 * use holds (*_bytes); the results do not depend on that chunk size.
 */
typedef struct gev2_conv2d_bwd_desc {
  int32_t dtype;
  int32_t act;
  float leaky_slope;
  int32_t reserved0;
  int32_t N, Cin, H, W, Cout, Kh, Kw;
  int32_t stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, groups;
  const void* X;
  const void* Wt;
  const void* dY;
  const void* Z;
  void* dW;
  float* dB;
  void* dX;
  void* col;    int64_t col_bytes;
  void* dcol;   int64_t dcol_bytes;
  void* gw;     int64_t gw_bytes;
  float* acc_b; int64_t acc_b_bytes;
  float* acc_w;
  void* dz;     int64_t dz_bytes;
} gev2_conv2d_bwd_desc;

int gev2_conv2d_fwd(const gev2_conv2d_desc* desc, void* stream);
int gev2_conv2d_bwd(const gev2_conv2d_bwd_desc* desc, void* stream);
/* Message for the last failing conv2d call on this thread ("" if none). */
const char* gev2_conv2d_last_error(void);

/*
 * Elman RNN on the operator (replaces RnnCudaLaunch / RnnCudaBackwardLaunch,
 * rnn/api.hpp:55-79, rnn/launcher.cu:129-383):
 *   h_t = act(X_t Wx + h_{t-1} Wh + b),  Y[:,t,:] = h_t,  Z[:,t,:] = pre-activation.
 * X [N,T,I], Wx [I,H], Wh [H,H], h0 [N,H], bias [H] fp32 (optional), Y / Z
 * [N,T,H], all contiguous, one dtype (F32 / F16 / BF16) except bias.
 * Workspaces (elements of dtype): xh N*(I+H), wcat (I+H)*H.  ws / ws_bytes:
 * optional scratch for the operator forward (gev2_gemm_fwd_desc.workspace).
 * One gather kernel and one operator forward per step; with F16 / BF16, N <= 16,
 * I a multiple of 256, H a multiple of 8, 16-byte aligned X, h0, Y and wcat,
 * and ws holding the step's split-K partials (gev2_gemm_fwd_workspace_size of
 * the step, 256-byte aligned), a step is instead the skinny split-K kernel
 * reading X_t and h_{t-1} in place (no gather) plus its K-block sum, with the
 * same results bit for bit (GEV2_RNN_GATHER=1 forces the gather form).  F32
 * steps within the one-launch small kernel's limits (I+H in 128..2048, at
 * most 512 16x16 output tiles, I a multiple of 4) read X_t and h_{t-1} in
 * place too, with or without ws.
 * On a created (non-null) stream, when ws covers every step's operator scratch
 * (gev2_gemm_fwd_workspace_size / gev2_gemm_bwd_workspace_size of one step),
 * the step loop of a descriptor seen before is recorded into a HIP graph on
 * its second call and replayed on later calls; the graph reads the buffers the
 * descriptor names as they are at launch.  GEV2_RNN_GRAPH=0 disables this.
 */
typedef struct gev2_rnn_desc {
  int32_t dtype;
  int32_t act;
  float leaky_slope;
  int32_t save_z;                 /* 1: write Z (must be non-NULL, not Y) */
  int32_t N, T, I, H;
  const void* X;
  const void* Wx;
  const void* Wh;
  const float* bias;
  const void* h0;
  void* Y;
  void* Z;
  void* xh;
  void* wcat;
  void* ws;  int64_t ws_bytes;
} gev2_rnn_desc;

/*
 * Backward through time from dY (= dL/dY, [N,T,H]) and the saved Z: dWx,
 * dWh, dB (fp32, sum over steps), dh0 and dX, each optional.  Workspaces
 * (elements of dtype unless noted): xh N*(I+H), g N*H, wcat (I+H)*H,
 * dxh N*(I+H), tmpw (I+H)*H, dwcat (I+H)*H floats, gb H floats.  ws / ws_bytes:
 * optional dY' scratch of the operator backward (gev2_gemm_bwd_desc.workspace).
 * With N <= 16, N*T <= I+H, H*elem a multiple of 16 bytes and 16-byte aligned
 * tmpw, wcat and dwcat, a step is one gather kernel (G' = (dY_t + dh_next) *
 * act'(Z_t) kept for all steps in tmpw as [N,T,H]) and one dXH product; dWx =
 * X^T G', dWh = Hprev^T G' (Hprev staged in dwcat) and dB are formed after the
 * loop (GEV2_RNN_STEP_DW=1 keeps one operator backward per step).  ws then
 * serves those two weight-gradient products.
 */
typedef struct gev2_rnn_bwd_desc {
  int32_t dtype;
  int32_t act;
  float leaky_slope;
  int32_t reserved0;
  int32_t N, T, I, H;
  const void* X;
  const void* Wx;
  const void* Wh;
  const void* h0;
  const void* dY;
  const void* Z;
  void* dWx;
  void* dWh;
  float* dB;
  void* dh0;
  void* dX;
  void* xh;
  void* g;
  void* wcat;
  void* dxh;
  float* dwcat;
  void* tmpw;
  float* gb;
  void* ws;  int64_t ws_bytes;
} gev2_rnn_bwd_desc;

int gev2_rnn_fwd(const gev2_rnn_desc* desc, void* stream);
int gev2_rnn_bwd(const gev2_rnn_bwd_desc* desc, void* stream);
/* Message for the last failing RNN call on this thread ("" if none). */
const char* gev2_rnn_last_error(void);

/*
 * Scaled dot-product attention (replaces SDPACudaLaunch /
 * SDPACudaBackwardLaunch, sdpa/api.hpp:8-33, sdpa/launcher.cu:129-747):
 *   S = scale * Q K^T (+ masks), P = softmax over keys, Y = P V.
 * Q [B,H,M,D], K / V [B,H,N,D], Y [B,H,M,D], contiguous, one dtype.
 * scale 0 means 1/sqrt(D).  causal adds -1e9 where key > query; mask
 * [B,1,M,N] (broadcast over H): I8 / I32 entries != 0 add -1e9, F32 entries
 * are added.  Dropout (dropout_p in [0, 1]) follows the reference's
 * stateless stream (dropout/kernels.cu:21-41, sdpa/launcher.cu:249-258,
 * 454-470): probability (b, h, q, key) is kept when the low 32 bits u of
 * splitmix64(seed ^ ((((b*H + h)*M + q)*N + key)) give float(u) * 2^-32 >= p,
 * and kept ones are scaled by 1/(1 - p) when scale_in_train (and p < 1); the
 * row sums of the softmax and the backward's regenerated mask use the same
 * stream, so one (seed, p) pair gives the same mask in both.
 * Forward, F16 / BF16 with D = 64 or 128: one fused kernel, no workspace;
 * `lse` (optional, fp32 [B,H,M]) receives each row's log-sum-exp.
 * Forward, F32: S / P in `workspace` (gev2_sdpa_workspace_size bytes).
 * Backward, F16 / BF16 with D = 64 or 128: fused kernels (P recomputed from
 * the forward's row log-sum-exp, O(N) workspace).  Otherwise the reference's
 * algorithm batched over all (b, h) slices in fp32, with P and dP in
 * `workspace`.
 */
enum { GEV2_MASK_NONE = 0, GEV2_MASK_I8 = 1, GEV2_MASK_I32 = 2, GEV2_MASK_F32 = 3 };

typedef struct gev2_sdpa_desc {
  int32_t dtype;
  int32_t B, H, M, N, D;
  float scale;
  int32_t causal;
  float dropout_p;
  int32_t mask_kind;               /* GEV2_MASK_* */
  const void* mask;
  const void* Q;
  const void* K;
  const void* V;
  void* Y;
  float* lse;
  void* workspace;  int64_t workspace_bytes;
  uint64_t seed;                    /* dropout stream seed */
  int32_t scale_in_train;           /* 1: kept probabilities scaled by 1/(1-p) */
  int32_t reserved1;
} gev2_sdpa_desc;

/* dQ / dK / dV (each optional, not all NULL) of the forward above for dY. */
typedef struct gev2_sdpa_bwd_desc {
  int32_t dtype;
  int32_t B, H, M, N, D;
  float scale;
  int32_t causal;
  float dropout_p;
  int32_t mask_kind;
  const void* mask;
  const void* Q;
  const void* K;
  const void* V;
  const void* dY;
  void* dQ;
  void* dK;
  void* dV;
  void* workspace;  int64_t workspace_bytes;
  uint64_t seed;
  int32_t scale_in_train;
  int32_t reserved1;
} gev2_sdpa_bwd_desc;

int gev2_sdpa_fwd(const gev2_sdpa_desc* desc, void* stream);
int gev2_sdpa_bwd(const gev2_sdpa_bwd_desc* desc, void* stream);
/* Workspace bytes of the forward (backward != 0: of the backward) for these
 * dimensions and dtype; -1 for an invalid descriptor.  No counterpart in the
 * reference, which allocates its S / P buffers on every call. */
int64_t gev2_sdpa_workspace_size(const gev2_sdpa_desc* desc, int backward);
/* Message for the last failing attention call on this thread ("" if none). */
const char* gev2_sdpa_last_error(void);

/*
 * Benchmark helpers (no counterpart in the reference): issue `reps` calls back
 * to back on `stream`, call i using descs[i % n_descs] (rotating buffer sets),
 * so that a timing of small problems measures the device, not the caller.
 */
int gev2_gemm_fwd_repeat(const gev2_gemm_fwd_desc* descs, int n_descs, int reps, void* stream);
int gev2_gemm_bwd_repeat(const gev2_gemm_bwd_desc* descs, int n_descs, int reps, void* stream);

/*
 * Measurement helper (no counterpart in the reference): launches one
 * 256-thread workgroup per compute unit (one wave per SIMD), each wave
 * issuing iters x 16 independent v_mfma_f32_32x32x16_bf16 on zero
 * (random_operands = 0) or random bf16 operands; total FLOP =
 * CUs * 4 * iters * 16 * 32768.  Time it with events on `stream` to get the
 * sustained MFMA rate for such data.
 */
int gev2_probe_mfma_bf16(int random_operands, int iters, void* stream);

/*
 * Measurement helper (no counterpart in the reference): `reps` back-to-back
 * launches, launch r reading the `bytes` at buf + (r % sets) * bytes (buf
 * 16-byte aligned, bytes a multiple of 4096 * unroll) with `workgroups`
 * 256-thread workgroups, each thread keeping `unroll` (8, 16 or 32) 16-byte
 * loads in flight; the data is discarded.  Timed with events on `stream`,
 * with sets * bytes larger than the 256 MB MALL, it gives the rate at which
 * this part streams a read of that size from HBM: the ceiling for the
 * bandwidth-bound forms (skinny M, the SDPA products).
 */
int gev2_probe_hbm_read(const void* buf, size_t bytes, int sets, int reps, int workgroups, int unroll,
                        void* stream);

/*
 * Measurement helper (no counterpart in the reference): as gev2_probe_hbm_read,
 * but each launch overwrites the `bytes` at buf + (r % sets) * bytes with
 * 16-byte stores (unroll 8 or 16 per thread): the rate at which this part
 * streams a write of that size to HBM, the ceiling for store-bound forms such
 * as the SDPA score product.
 */
int gev2_probe_hbm_write(void* buf, size_t bytes, int sets, int reps, int workgroups, int unroll, void* stream);

int gev2_abi_version(void);
const char* gev2_status_string(int status);
/* Message for the last failing call on this thread ("" if none). */
const char* gev2_last_error(void);
/* Name of the kernel family the last gev2_gemm_fwd on this thread used
 * ("dl:<cfg>", "tile:<cfg>", "tile:splitk", "skinny:split", "skinny",
 * "small"), or after a gev2_gemm_bwd "small" (the one-launch backward) or
 * "bwd" (any other), for tests and profiling. */
const char* gev2_last_path(void);

/*
 * Device, memory, stream and event helpers, so that hosts without a tensor
 * library (the C++ binding, ctypes tests, the benchmark) can stage buffers.
 * (The reference relies on CuPy for these.)
 */
int gev2_device_count(int* count);
int gev2_set_device(int device);
int gev2_get_device(int* device);
/* name (NUL-terminated, truncated to name_len), compute units, peak clock kHz */
int gev2_device_info(int device, char* name, size_t name_len, int* cu_count, int* clock_khz);
int gev2_malloc(void** ptr, size_t bytes);
/* A free requested while this thread has a capture open (gev2_graph_begin ..
 * gev2_graph_end) is carried out when the capture ends. */
int gev2_free(void* ptr);
int gev2_memcpy_htod(void* dst, const void* src, size_t bytes);
int gev2_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int gev2_memcpy_dtod_async(void* dst, const void* src, size_t bytes, void* stream);
int gev2_memset(void* ptr, int value, size_t bytes);
int gev2_stream_create(void** stream);
int gev2_stream_destroy(void* stream);
int gev2_stream_synchronize(void* stream);
int gev2_device_synchronize(void);
int gev2_event_create(void** event);
int gev2_event_destroy(void* event);
int gev2_event_record(void* event, void* stream);
int gev2_event_synchronize(void* event);
int gev2_event_elapsed_ms(float* ms, void* start, void* stop);

/*
 * HIP graph capture of a stream's work: begin, run the calls to record on
 * `stream`, end (instantiates; *exec receives the executable graph), then
 * launch it any number of times and destroy it.  Replaces the CuPy graph
 * capture of the reference's Python layer (graph/graph_exec.py:119-136).  The
 * GEMM calls allocate nothing under capture (see Conventions), so they may be
 * recorded without a warm-up call; with every workspace passed, the recorded
 * kernels are the same as the eager ones.
 */
int gev2_graph_begin(void* stream);
int gev2_graph_end(void* stream, void** exec);
int gev2_graph_launch(void* exec, void* stream);
int gev2_graph_destroy(void* exec);

#ifdef __cplusplus
}
#endif

#endif /* GEV2_GEMM_H_ */
