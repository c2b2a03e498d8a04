"""GPU parity at the benchmark workloads' own sizes, through the C ABI (and the conv2d
module for the operator form), against the float64 oracle on the same seeded inputs.
This follows the reference's own check of the op (tests/cuda_pyd_test/smoke_gemm_binding.py:84-123:
forward, then backward against NumPy), at the configurations the operator is measured on:

  C1  fp32 X[64,784] W[784,256] b[256], U(-1,1)/sqrt(784), ReLU; dY ~ N(0,1)
  C2  fp32 1024^3, GELU (tanh form), X, W ~ N(0,1/K), b ~ N(0,0.02), dY ~ N(0,1)
  C3  bf16 and fp16 4096^3, ReLU, Z saved: the forward on its default 256x256 direct-to-LDS
      tile, the backward on its materialised dY' path (M*N*K >= 2^30)
  C4  the SDPA batched form, B*H = 64 slices of 512x512x64: S = (Q K^T) * 1/8 (trans_b, alpha),
      then Y = P V with P = row-softmax of N(0,1) logits; slice strides 512*64 for Q, K, V, Y and
      512*512 for S / P (sdpa/launcher.cu:166-170,185-270); again with exact integers at full size
      so that index and stride handling is checked bit for bit
  C5a conv-as-GEMM, X NCHW [32,64,56,56] ~ U(0,1), 3x3 / stride 1 / pad 1, W ~ N(0,2/576),
      128 output channels: the stacked im2col GEMM 100352x576x128 (column order (c*3+kh)*3+kw,
      conv2d/kernels.cu:12-45), and the conv2d operator on all 32 images (forward and backward)
  (C5b, the skinny 8x4096x4096 bf16 shape, is test_gpu_parity.test_skinny_full_size.)

Tolerances, written per check below: fp32 accumulation over K terms, gamma_K (|A||B|), plus one
rounding of each stored result (u |x|, or half the subnormal spacing below the normal range); normwise relative error <= 1e-4 (fp32) or <= 1e-2 (bf16 / fp16);
ReLU masks bit-exact in both senses (Y == Z where Z > 0 else +0, and agreement with the float64
mask wherever |Z64| exceeds the error bound; dY' == dY where Z > 0 else 0).
"""
import numpy as np
import pytest

from oracle import gemm_oracle as O
from conv_helpers import _run as conv_run
from gemm_helpers import (BF16, F16, F32, DT_NAMES, TINY_OUT, U_ACC, U_OUT, Dev, act_lipschitz, assert_close,
                          fwd_bound, rounded)

pytestmark = pytest.mark.gpu


def _normal_inputs(seed, M, N, K, dtype):
    """X, W ~ N(0, 1/K), b ~ N(0, 0.02) (fp32), dY ~ N(0, 1); X, W, dY rounded to the dtype."""
    g = np.random.default_rng(seed)
    X = rounded(g.standard_normal((M, K)) / np.sqrt(K), dtype)
    W = rounded(g.standard_normal((K, N)) / np.sqrt(K), dtype)
    b = (0.02 * g.standard_normal(N)).astype(np.float32)
    gY = rounded(g.standard_normal((M, N)), dtype)
    return X, W, b, gY


def _fwd_bwd_on_device(capi, X, W, b, gY, act, dtype):
    """Forward with Z saved, then the backward (dX, dW, PerN dBias, and gC = dY' with beta = 1)
    reading the device's own Z stash. Returns host copies and the forward path."""
    M, K = X.shape
    N = W.shape[1]
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pX, pW = dev.put(capi.to_storage(X, dtype)), dev.put(capi.to_storage(W, dtype))
        pb, pgY = dev.put(b), dev.put(capi.to_storage(gY, dtype))
        pY, pZ = dev.empty(M * N * es), dev.empty(M * N * es)
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb,
                      bias_kind=O.BIAS_PERN, act=act)
        path = capi.last_path()
        pgA, pgB, pgC, pgb = dev.empty(M * K * es), dev.empty(K * N * es), dev.empty(M * N * es), dev.empty(N * 4)
        capi.gemm_bwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, gA=pgA, gB=pgB, gC=pgC,
                      gBias=pgb, bias_kind=O.BIAS_PERN, act=act, beta=1.0)
        capi.synchronize()
        out = dict(Y=dev.get(pY, (M, N), dtype), Z=dev.get(pZ, (M, N), dtype),
                   gA=dev.get(pgA, (M, K), dtype), gB=dev.get(pgB, (K, N), dtype),
                   gC=dev.get(pgC, (M, N), dtype), gBias=dev.get_f32(pgb, (N,)))
    finally:
        dev.close()
    return out, path


def _check_fwd_bwd(out, X, W, b, gY, act, dtype, tag):
    M, K = X.shape
    N = W.shape[1]
    u = U_OUT[dtype]
    rel = 1e-4 if dtype == F32 else 1e-2
    Y, Z = out["Y"], out["Z"]
    # forward: |Z - Z64| <= 1.01 K u32 (|X||W|)_mn + u32 |b_n| + u_out |Z64|
    Y64, Z64 = O.gemm_forward(X, W, b, O.BIAS_PERN, act)
    bz = fwd_bound(X, W, K, dtype, np.broadcast_to(b.astype(np.float64), (M, N)))
    assert_close(Z, Z64, bz + u * np.abs(Z64) + TINY_OUT[dtype], "Z " + tag, rel_norm=rel)
    ya = act_lipschitz(act) * bz + u * np.abs(Y64) + 8 * U_ACC * np.abs(Y64) + 2e-7 + TINY_OUT[dtype]
    assert_close(Y, Y64, ya, "Y " + tag, rel_norm=rel)
    if O.parse_act(act) == O.ACT_RELU:
        pos = Z > 0
        assert np.array_equal(Y[pos], Z[pos]), "Y != Z where Z > 0: " + tag
        assert np.all(Y[~pos] == 0) and not np.any(np.signbit(Y[~pos])), "Y != +0 where Z <= 0: " + tag
        sure = np.abs(Z64) > bz
        assert np.array_equal(pos[sure], (Z64 > 0)[sure]), "ReLU mask differs from float64: " + tag
    # backward against the device's Z (the backward's input)
    ref = O.gemm_backward(X, W, gY, Z, act, 0.01, O.BIAS_PERN, 1.0, 1.0)
    aG, aY = np.abs(ref["gZ"]), np.abs(gY.astype(np.float64))
    # 16-bit dY' for a non-piecewise-linear act' is rounded once before the GEMMs
    e16 = 0.0 if (dtype == F32 or O.parse_act(act) in (O.ACT_NONE, O.ACT_RELU)) else u
    # act' evaluated in fp32 on the device: |d act'| <= 1e-6 (GELU / sigmoid / tanh)
    dact = 0.0 if O.parse_act(act) in (O.ACT_NONE, O.ACT_RELU, O.ACT_LEAKY) else 1e-6
    Wt, Xt = np.abs(W.astype(np.float64)).T, np.abs(X.astype(np.float64)).T
    bnd = (1.01 * N * U_ACC + e16) * (aG @ Wt) + u * np.abs(ref["gA"]) + TINY_OUT[dtype]
    if dact:
        bnd = bnd + dact * (aY @ Wt)
    assert_close(out["gA"], ref["gA"], bnd, "dX " + tag, rel_norm=rel)
    bnd = (1.01 * M * U_ACC + e16) * (Xt @ aG) + u * np.abs(ref["gB"]) + TINY_OUT[dtype]
    if dact:
        bnd = bnd + dact * (Xt @ aY)
    assert_close(out["gB"], ref["gB"], bnd, "dW " + tag, rel_norm=rel)
    assert_close(out["gBias"], ref["gBias"], (1.01 * M * U_ACC + e16) * aG.sum(0) + dact * aY.sum(0) + TINY_OUT[dtype],
                 "dBias " + tag, rel_norm=rel)
    assert_close(out["gC"], ref["gZ"], u * aG + dact * aY + TINY_OUT[dtype], "dY' " + tag)
    if O.parse_act(act) == O.ACT_RELU:
        pos = Z > 0
        assert np.array_equal(out["gC"][pos], gY[pos]) and np.all(out["gC"][~pos] == 0), "dY' mask " + tag


def test_c1_mlp_dense_f32(gpu):
    """C1: the reference's Dense layer shape, fp32, uniform(-1,1)/sqrt(784) inputs, ReLU."""
    M, K, N = 64, 784, 256
    g = np.random.default_rng(101)
    X = (g.uniform(-1, 1, (M, K)) / np.sqrt(K)).astype(np.float32)
    W = (g.uniform(-1, 1, (K, N)) / np.sqrt(K)).astype(np.float32)
    b = (g.uniform(-1, 1, N) / np.sqrt(K)).astype(np.float32)
    gY = g.standard_normal((M, N)).astype(np.float32)
    out, path = _fwd_bwd_on_device(gpu, X, W, b, gY, "relu", F32)
    _check_fwd_bwd(out, X, W, b, gY, "relu", F32, f"C1 f32 64x256x784 path={path}")


def test_c2_square_gelu_f32(gpu):
    """C2: fp32 1024^3 with the GELU (tanh form) epilogue, forward + backward."""
    X, W, b, gY = _normal_inputs(102, 1024, 1024, 1024, F32)
    out, path = _fwd_bwd_on_device(gpu, X, W, b, gY, "gelu", F32)
    _check_fwd_bwd(out, X, W, b, gY, "gelu", F32, f"C2 f32 1024^3 path={path}")


@pytest.mark.parametrize("dtype", [BF16, F16], ids=lambda d: DT_NAMES[d])
def test_c3_headline_relu(gpu, dtype):
    """C3: 4096^3 with bias and ReLU, Z saved; the forward must run the 256x256 direct-to-LDS
    tile over the whole K = 4096 loop (the headline kernel), and the backward materialises dY'."""
    n = 4096
    X, W, b, gY = _normal_inputs(103 + dtype, n, n, n, dtype)
    out, path = _fwd_bwd_on_device(gpu, X, W, b, gY, "relu", dtype)
    assert path == "dl:256x256", path
    _check_fwd_bwd(out, X, W, b, gY, "relu", dtype, f"C3 {DT_NAMES[dtype]} 4096^3 path={path}")


C4_BH, C4_M, C4_N, C4_D = 64, 512, 512, 64


def _c4_run(capi, Q, Kt, V, P, dtype):
    """S = (Q K^T) / 8 over the 64 slices (trans_b, alpha), then Y = P V; returns S, Y."""
    BH, M, N, D = C4_BH, C4_M, C4_N, C4_D
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pQ, pK, pV, pP = (dev.put(capi.to_storage(a, dtype)) for a in (Q, Kt, V, P))
        pS, pY = dev.empty(BH * M * N * es), dev.empty(BH * M * D * es)
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=D, A=pQ, B=pK, Y=pS, trans_b=True, alpha=0.125,
                      batch=BH, stride_a=M * D, stride_b=N * D, stride_y=M * N)
        p1 = capi.last_path()
        capi.gemm_fwd(dtype=dtype, M=M, N=D, K=N, A=pP, B=pV, Y=pY, batch=BH,
                      stride_a=M * N, stride_b=N * D, stride_y=M * D)
        p2 = capi.last_path()
        capi.synchronize()
        return dev.get(pS, (BH, M, N), dtype), dev.get(pY, (BH, M, D), dtype), (p1, p2)
    finally:
        dev.close()


@pytest.mark.parametrize("dtype", [BF16, F16], ids=lambda d: DT_NAMES[d])
def test_c4_sdpa_batched_form(gpu, dtype):
    """C4 with the benchmark's distributions: Q, K, V ~ N(0,1); P = row-softmax(N(0,1) logits)."""
    BH, M, N, D = C4_BH, C4_M, C4_N, C4_D
    g = np.random.default_rng(104 + dtype)
    Q = rounded(g.standard_normal((BH, M, D)), dtype)
    Kt = rounded(g.standard_normal((BH, N, D)), dtype)
    V = rounded(g.standard_normal((BH, N, D)), dtype)
    logits = g.standard_normal((BH, M, N))
    e = np.exp(logits - logits.max(-1, keepdims=True))
    P = rounded(e / e.sum(-1, keepdims=True), dtype)
    S, Y, paths = _c4_run(gpu, Q, Kt, V, P, dtype)
    u = U_OUT[dtype]
    S64, _ = O.gemm_forward_batched(Q, Kt, BH, M, N, D, M * D, N * D, D, D, trans_b=True, alpha=0.125)
    aS, _ = O.gemm_forward_batched(np.abs(Q), np.abs(Kt), BH, M, N, D, M * D, N * D, D, D, trans_b=True,
                                   alpha=0.125)
    assert_close(S, S64, 1.01 * D * U_ACC * aS + u * np.abs(S64) + TINY_OUT[dtype],
                 f"S {DT_NAMES[dtype]} path={paths[0]}", rel_norm=1e-2)
    Y64, _ = O.gemm_forward_batched(P, V, BH, M, D, N, M * N, N * D, N, D)
    aY, _ = O.gemm_forward_batched(P, np.abs(V), BH, M, D, N, M * N, N * D, N, D)
    assert_close(Y, Y64, 1.01 * N * U_ACC * aY + u * np.abs(Y64) + TINY_OUT[dtype],
                 f"PV {DT_NAMES[dtype]} path={paths[1]}", rel_norm=1e-2)


@pytest.mark.parametrize("dtype", [BF16, F16], ids=lambda d: DT_NAMES[d])
def test_c4_sdpa_batched_form_exact(gpu, dtype):
    """C4 at full size with exact-integer inputs: every sum is exact, so S and Y must equal the
    float64 results after one rounding, bit for bit (slice offsets and strides)."""
    BH, M, N, D = C4_BH, C4_M, C4_N, C4_D
    g = np.random.default_rng(204 + dtype)
    Q = g.integers(-2, 3, (BH, M, D)).astype(np.float32)
    Kt = g.integers(-2, 3, (BH, N, D)).astype(np.float32)
    V = g.integers(-2, 3, (BH, N, D)).astype(np.float32)
    P = (g.random((BH, M, N)) < 0.05).astype(np.float32) * g.integers(1, 3, (BH, M, N)).astype(np.float32)
    S, Y, _ = _c4_run(gpu, Q, Kt, V, P, dtype)
    S64, _ = O.gemm_forward_batched(Q, Kt, BH, M, N, D, M * D, N * D, D, D, trans_b=True, alpha=0.125)
    Y64, _ = O.gemm_forward_batched(P, V, BH, M, D, N, M * N, N * D, N, D)
    assert np.array_equal(S, rounded(S64, dtype))
    assert np.array_equal(Y, rounded(Y64, dtype))


C5A = dict(N=32, Cin=64, H=56, W=56, Cout=128, Kh=3, Kw=3, stride=(1, 1), pad=(1, 1), dil=(1, 1))


def _c5a_inputs(seed, dtype):
    g = np.random.default_rng(seed)
    X = rounded(g.uniform(0, 1, (C5A["N"], C5A["Cin"], C5A["H"], C5A["W"])), dtype)
    Wc = rounded(g.standard_normal((C5A["Cout"], C5A["Cin"], 3, 3)) * np.sqrt(2 / 576), dtype)
    b = (0.02 * g.standard_normal(C5A["Cout"])).astype(np.float32)
    return X, Wc, b


def _im2col(X):
    """[N,C,H,W] -> [N*H*W, C*9] for a 3x3 / stride 1 / pad 1 window, column (c*3+kh)*3+kw."""
    n, c, h, w = X.shape
    Xp = np.pad(X, ((0, 0), (0, 0), (1, 1), (1, 1)))
    win = np.lib.stride_tricks.sliding_window_view(Xp, (3, 3), axis=(2, 3))   # [n,c,h,w,3,3]
    return np.ascontiguousarray(win.transpose(0, 2, 3, 1, 4, 5)).reshape(n * h * w, c * 9)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: DT_NAMES[d])
def test_c5a_conv_as_gemm(gpu, dtype):
    """C5a as one stacked GEMM: Col[100352,576] . W_KC[576,128] + b, ReLU, Z saved."""
    X, Wc, b = _c5a_inputs(105 + dtype, dtype)
    col = _im2col(X)
    w_kc = np.ascontiguousarray(Wc.reshape(C5A["Cout"], -1).T)
    M, K = col.shape
    N = w_kc.shape[1]
    assert (M, K, N) == (100352, 576, 128)
    capi = gpu
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pA, pB, pb = dev.put(capi.to_storage(col, dtype)), dev.put(capi.to_storage(w_kc, dtype)), dev.put(b)
        pY, pZ = dev.empty(M * N * es), dev.empty(M * N * es)
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=K, A=pA, B=pB, Y=pY, Z=pZ, bias=pb, bias_kind=O.BIAS_PERN,
                      act="relu")
        path = capi.last_path()
        capi.synchronize()
        Y, Z = dev.get(pY, (M, N), dtype), dev.get(pZ, (M, N), dtype)
    finally:
        dev.close()
    tag = f"C5a {DT_NAMES[dtype]} 100352x128x576 path={path}"
    Y64, Z64 = O.gemm_forward(col, w_kc, b, O.BIAS_PERN, "relu")
    bz = fwd_bound(col, w_kc, K, dtype, np.broadcast_to(b.astype(np.float64), (M, N)))
    u = U_OUT[dtype]
    rel = 1e-4 if dtype == F32 else 1e-2
    assert_close(Z, Z64, bz + u * np.abs(Z64) + TINY_OUT[dtype], "Z " + tag, rel_norm=rel)
    assert_close(Y, Y64, bz + u * np.abs(Y64) + TINY_OUT[dtype], "Y " + tag, rel_norm=rel)
    pos = Z > 0
    assert np.array_equal(Y[pos], Z[pos]) and np.all(Y[~pos] == 0) and not np.any(np.signbit(Y[~pos]))
    sure = np.abs(Z64) > bz
    assert np.array_equal(pos[sure], (Z64 > 0)[sure])


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: DT_NAMES[d])
def test_c5a_conv2d_operator(gpu, dtype):
    """C5a through the conv2d operator with one batched call over all 32 images: forward (bias,
    ReLU, Z) and backward (dW and dB summed over the images, dX).  Bounds per output element,
    with A the same sum taken over absolute values:
      Z:  1.01 K u32 A + u32 |b| + u |Z64|                     (K = 576 products)
      dW: (1.01 (HWo + N) u32 + u) A + u |dW64|                 (per-image GEMM over HWo = 3136
          terms, each image's dW rounded once to the dtype, then an fp32 sum over N = 32 images)
      dX: (1.01 (Cout + Kh Kw) u32 + u) A + u |dX64|            (column GEMM over Cout = 128
          terms, rounded once, then an fp32 gather of up to 9 columns)
      dB: 1.01 (N HWo) u32 A
    u is the unit roundoff of the storage type."""
    from graph_executor_v2.ops import _ops_conv2d as conv
    from graph_executor_v2.ops.device_array import DeviceArray
    g = C5A
    X, Wc, b = _c5a_inputs(205 + dtype, dtype)
    Ho, Wo = g["H"], g["W"]
    dY = rounded(np.random.default_rng(305 + dtype).standard_normal((g["N"], g["Cout"], Ho, Wo)), dtype)
    out = conv_run((conv, DeviceArray), g, X, Wc, b, "relu", dtype=dtype, all_images=True, dY=dY,
                   bwd_images=g["N"])
    u = U_OUT[dtype]
    K, HWo = g["Cin"] * 9, Ho * Wo
    Y64, Z64 = O.conv2d_forward(X, Wc, b, g["stride"], g["pad"], g["dil"], act="relu")
    absZ, _ = O.conv2d_forward(np.abs(X), np.abs(Wc), None, g["stride"], g["pad"], g["dil"])
    bz = 1.01 * K * U_ACC * absZ + U_ACC * np.abs(b).reshape(1, -1, 1, 1)
    assert_close(out["Z"], Z64, bz + u * np.abs(Z64) + TINY_OUT[dtype], "conv Z", rel_norm=1e-4 if dtype == F32 else 1e-2)
    pos = out["Z"] > 0
    assert np.array_equal(out["Y"][pos], out["Z"][pos]) and np.all(out["Y"][~pos] == 0)
    sure = np.abs(Z64) > bz
    assert np.array_equal(pos[sure], (Z64 > 0)[sure])
    ref = O.conv2d_backward(X, Wc, dY, out["Z"].astype(np.float64), g["stride"], g["pad"], g["dil"], act="relu")
    aref = O.conv2d_backward(np.abs(X), np.abs(Wc), np.abs(dY), np.ones_like(Z64), g["stride"], g["pad"],
                             g["dil"])
    rel = 1e-4 if dtype == F32 else 1e-2
    assert_close(out["dW"], ref["dW"], (1.01 * (HWo + g["N"]) * U_ACC + u) * aref["dW"] + u * np.abs(ref["dW"])
                 + TINY_OUT[dtype], "conv dW", rel_norm=rel)
    assert_close(out["dX"], ref["dX"], (1.01 * (g["Cout"] + 9) * U_ACC + u) * aref["dX"] + u * np.abs(ref["dX"])
                 + TINY_OUT[dtype], "conv dX", rel_norm=rel)
    assert_close(out["dB"], ref["dB"], 1.01 * g["N"] * HWo * U_ACC * aref["dB"] + TINY_OUT[dtype], "conv dB", rel_norm=rel)
