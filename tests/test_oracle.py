"""Pins for the CPU oracle (oracle/gemm_oracle.py, oracle/gemm_oracle.c).

Each check is chosen so that a plausible restatement mistake (a dropped term,
a wrong sign, a transposed operand, a wrong special case) fails it:
  * activations against special values, the erf form of GELU and central
    finite differences of the forward (pins every derivative formula);
  * GEMM forward/backward against exact integer arithmetic (Python ints);
  * backward against finite differences of a scalar loss (pins dX/dW/dBias
    including which operand is transposed);
  * bias-kind inference against the reference's rules (known answers read off
    bias.hpp:70-78 and gemm/launcher.cu:47-77);
  * the C fp32 restatement (the reference's small-kernel summation order)
    against the float64 one.
"""
import ctypes
import math
import os

import numpy as np
import pytest

from oracle import gemm_oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ACTS = ["none", "relu", "leakyrelu", "gelu", "sigmoid", "tanh"]


# ---------------------------------------------------------------------------
# activations
# ---------------------------------------------------------------------------
def test_act_special_values():
    f = O.act_forward
    assert f(0.0, "relu") == 0 and f(-1.0, "relu") == 0 and f(2.5, "relu") == 2.5
    assert f(-2.0, "leakyrelu", 0.1) == pytest.approx(-0.2) and f(0.0, "leakyrelu") == 0
    assert f(3.0, "leakyrelu", 0.1) == 3.0
    assert f(0.0, "gelu") == 0 and f(0.0, "sigmoid") == 0.5 and f(0.0, "tanh") == 0
    # branch-stable sigmoid: no overflow at the extremes
    with np.errstate(over="raise"):
        assert f(-1000.0, "sigmoid") == 0.0 and f(1000.0, "sigmoid") == 1.0
    d = O.act_deriv
    assert d(0.0, "relu") == 0 and d(1e-30, "relu") == 1
    assert d(0.0, "leakyrelu", 0.2) == 0.2          # slope at z == 0 (activations.hpp:47)
    assert d(0.0, "sigmoid") == 0.25 and d(0.0, "tanh") == 1.0
    assert d(0.0, "gelu") == pytest.approx(0.5)
    assert np.all(d(np.linspace(-5, 5, 11), "none") == 1.0)


def test_gelu_constants():
    """c is fixed by the mathematics (sqrt(2/pi), to the 10 digits activations.hpp:19 writes), and
    the whole tanh form, k1 = 0.044715 included, agrees with an independent implementation of the
    same approximation (torch's gelu(approximate='tanh'), float64) to 1e-12: a wrong digit in either
    constant moves it by more than 1e-6."""
    import torch
    assert abs(O.GELU_C - np.sqrt(2 / np.pi)) < 5e-11
    z = np.linspace(-8, 8, 20001)
    ref = torch.nn.functional.gelu(torch.from_numpy(z), approximate="tanh").numpy()
    assert np.max(np.abs(O.act_forward(z, "gelu") - ref)) < 1e-11


def test_gelu_tanh_form_tracks_erf_form():
    z = np.linspace(-8, 8, 4001)
    # the tanh approximation of GELU is within 1e-3 of the exact erf form
    assert np.max(np.abs(O.act_forward(z, "gelu") - O.gelu_erf(z))) < 1e-3
    # and it is *not* the erf form (the constants are the tanh ones)
    assert np.max(np.abs(O.act_forward(z, "gelu") - O.gelu_erf(z))) > 1e-5


@pytest.mark.parametrize("act", ACTS)
def test_act_deriv_matches_finite_difference(act):
    z = np.concatenate([np.linspace(-6, -0.05, 300), np.linspace(0.05, 6, 300)])
    h = 1e-6
    fd = (O.act_forward(z + h, act, 0.07) - O.act_forward(z - h, act, 0.07)) / (2 * h)
    an = O.act_deriv(z, act, 0.07)
    if act == "gelu":
        # where the derivative's tanh clamp (activations.hpp:55-56) engages, the
        # reference deliberately departs from d/dz of the forward; that region is
        # pinned by test_gelu_deriv_clamp_is_applied
        t = O.GELU_C * (z + O.GELU_K1 * z ** 3)
        keep = np.abs(np.tanh(t)) < O.GELU_TH_CLAMP
        assert keep.sum() > 300
        fd, an = fd[keep], an[keep]
    assert np.max(np.abs(fd - an)) < 2e-6


def test_gelu_deriv_clamp_is_applied():
    # for large |z| tanh(t) rounds to +-1; the clamp keeps sech^2 >= 1 - 0.999999^2
    z = np.array([12.0, -12.0])
    d = O.act_deriv(z, "gelu")
    th = 0.999999
    expect_pos = 0.5 * (1 + th) + 0.5 * 12.0 * (1 - th * th) * O.GELU_C * (1 + 3 * O.GELU_K1 * 144)
    assert d[0] == pytest.approx(expect_pos, rel=1e-12)
    assert d[0] != 1.0


# ---------------------------------------------------------------------------
# GEMM forward / backward
# ---------------------------------------------------------------------------
def _int_mat(g, r, c):
    return g.integers(-3, 4, size=(r, c))


def _py_matmul(A, B):
    return [[sum(int(A[i][k]) * int(B[k][j]) for k in range(len(B))) for j in range(len(B[0]))]
            for i in range(len(A))]


@pytest.mark.parametrize("bias_kind", [O.BIAS_NONE, O.BIAS_PERN, O.BIAS_PERM, O.BIAS_SCALAR])
def test_forward_exact_integers(bias_kind):
    g = np.random.default_rng(1)
    M, N, K = 5, 7, 6
    A, B = _int_mat(g, M, K), _int_mat(g, K, N)
    nb = {O.BIAS_NONE: 0, O.BIAS_PERN: N, O.BIAS_PERM: M, O.BIAS_SCALAR: 1}[bias_kind]
    bias = g.integers(-5, 6, size=nb) if nb else None
    Y, Z = O.gemm_forward(A, B, bias, bias_kind if nb else None, "relu", alpha=0.5)
    ref = _py_matmul(A.tolist(), B.tolist())
    for i in range(M):
        for j in range(N):
            pre = 0.5 * ref[i][j]
            if bias_kind == O.BIAS_PERN:
                pre += bias[j]
            elif bias_kind == O.BIAS_PERM:
                pre += bias[i]
            elif bias_kind == O.BIAS_SCALAR:
                pre += bias[0]
            assert Z[i, j] == pre
            assert Y[i, j] == max(pre, 0.0)


def test_forward_transposes():
    g = np.random.default_rng(2)
    A, B = _int_mat(g, 4, 3), _int_mat(g, 3, 5)
    Y0, _ = O.gemm_forward(A, B)
    Y1, _ = O.gemm_forward(A.T.copy(), B, trans_a=True)
    Y2, _ = O.gemm_forward(A, B.T.copy(), trans_b=True)
    assert np.array_equal(Y0, Y1) and np.array_equal(Y0, Y2)
    assert np.array_equal(Y0, np.array(_py_matmul(A.tolist(), B.tolist()), dtype=float))


def test_backward_exact_integers():
    g = np.random.default_rng(3)
    M, N, K = 6, 4, 5
    A, B = _int_mat(g, M, K), _int_mat(g, K, N)
    gY = _int_mat(g, M, N)
    _, Z = O.gemm_forward(A, B, None, None, "relu")
    r = O.gemm_backward(A, B, gY, Z, "relu", bias_kind=O.BIAS_PERN, beta=1.0)
    gZ = [[int(gY[i, j]) if Z[i, j] > 0 else 0 for j in range(N)] for i in range(M)]
    BT = [list(x) for x in zip(*B.tolist())]
    AT = [list(x) for x in zip(*A.tolist())]
    assert np.array_equal(r["gA"], np.array(_py_matmul(gZ, BT), dtype=float))
    assert np.array_equal(r["gB"], np.array(_py_matmul(AT, gZ), dtype=float))
    assert np.array_equal(r["gBias"], np.array([sum(gZ[i][j] for i in range(M)) for j in range(N)], dtype=float))
    assert np.array_equal(r["gC"], np.array(gZ, dtype=float))
    r2 = O.gemm_backward(A, B, gY, Z, "relu", bias_kind=O.BIAS_PERM)
    assert np.array_equal(r2["gBias"], np.array([sum(row) for row in gZ], dtype=float))
    r3 = O.gemm_backward(A, B, gY, Z, "relu", bias_kind=O.BIAS_SCALAR)
    assert r3["gBias"][0] == sum(map(sum, gZ))


@pytest.mark.parametrize("act", ["gelu", "sigmoid", "tanh", "none"])
def test_backward_matches_finite_difference(act):
    g = np.random.default_rng(4)
    M, N, K = 7, 5, 6
    X, W = g.standard_normal((M, K)), g.standard_normal((K, N)) / 2
    b = g.standard_normal(N) / 3
    G = g.standard_normal((M, N))

    def loss(X_, W_, b_):
        Y, _ = O.gemm_forward(X_, W_, b_, O.BIAS_PERN, act)
        return float(np.sum(G * Y))

    _, Z = O.gemm_forward(X, W, b, O.BIAS_PERN, act)
    r = O.gemm_backward(X, W, G, Z, act, bias_kind=O.BIAS_PERN)
    h = 1e-6
    for name, base, grad in (("X", X, r["gA"]), ("W", W, r["gB"]), ("b", b, r["gBias"])):
        D = g.standard_normal(base.shape)
        args_p = [X, W, b]
        args_m = [X, W, b]
        idx = {"X": 0, "W": 1, "b": 2}[name]
        args_p[idx] = base + h * D
        args_m[idx] = base - h * D
        fd = (loss(*args_p) - loss(*args_m)) / (2 * h)
        assert fd == pytest.approx(float(np.sum(grad * D)), rel=1e-6, abs=1e-8), name


def test_batched_slice_offsets():
    """Slice (b,h) of a [B,H,R,C] buffer starts at ((b*H+h)*R*C) (sdpa/launcher.cu:166-170)."""
    B, H, R, C = 2, 3, 4, 5
    flat = np.arange(B * H * R * C)
    t = flat.reshape(B, H, R, C)
    for b in range(B):
        for h in range(H):
            off = O.slice_offset(b, h, H, R, C)
            assert np.array_equal(flat[off:off + R * C].reshape(R, C), t[b, h])


def test_batched_forward_matches_loop():
    g = np.random.default_rng(5)
    batch, M, N, K = 3, 4, 6, 5
    lda, ldb = K + 2, K + 1
    sA, sB = M * lda + 3, N * ldb
    A = g.integers(-2, 3, batch * sA).astype(float)
    Bf = g.integers(-2, 3, batch * sB).astype(float)
    Y, _ = O.gemm_forward_batched(A, Bf, batch, M, N, K, sA, sB, lda, ldb, trans_b=True, alpha=0.25)
    for i in range(batch):
        a = A[i * sA:i * sA + M * lda].reshape(M, lda)[:, :K]
        bt = Bf[i * sB:i * sB + N * ldb].reshape(N, ldb)[:, :K]
        assert np.array_equal(Y[i], 0.25 * (a @ bt.T))


# ---------------------------------------------------------------------------
# bias-kind inference
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,M,N,expect", [
    ((8,), 4, 8, O.BIAS_PERN),
    ((4,), 4, 8, O.BIAS_PERM),
    ((1,), 4, 8, O.BIAS_SCALAR),
    ((8,), 8, 8, O.BIAS_PERN),        # PerN wins when M == N (bias.hpp:76-77)
    ((1,), 1, 1, O.BIAS_SCALAR),      # Scalar wins over everything
    ((1, 8), 4, 8, O.BIAS_PERN),      # 2-D forms via the fallback (launcher.cu:60-65)
    ((4, 1), 4, 8, O.BIAS_PERM),
    ((1, 1), 4, 8, O.BIAS_SCALAR),
    ((2, 4), 4, 8, O.BIAS_PERN),      # numel == N (launcher.cu:67)
    ((2, 2), 4, 8, O.BIAS_PERM),      # numel == M (launcher.cu:68)
    ((4, 8), 4, 8, O.BIAS_NONE),      # (M,N): silently no bias (launcher.cu:70)
    ((0,), 4, 8, O.BIAS_NONE),
    ((3,), 4, 8, O.BIAS_NONE),
    (None, 4, 8, O.BIAS_NONE),
])
def test_decide_bias_kind(shape, M, N, expect):
    assert O.decide_bias_kind(shape, M, N) == expect


# ---------------------------------------------------------------------------
# reduced precision emulation
# ---------------------------------------------------------------------------
def test_bf16_rounding_known_answers():
    one = 1.0
    x = np.array([one, one + 2 ** -8, one + 3 * 2 ** -8, -2.5, 3.0e38, 1e-40], np.float32)
    r = O.round_to(x, O.DT_BF16)
    assert r[0] == 1.0
    assert r[1] == 1.0                      # tie -> even
    assert r[2] == 1.0 + 2 ** -6            # tie -> even (odd neighbour rounds up)
    assert r[3] == -2.5
    assert np.isfinite(r[4])
    assert np.array_equal(O.round_to(np.float32(1.5), O.DT_F16), np.float32(1.5))
    assert O.round_to(np.float32(1 + 2 ** -11), O.DT_F16) == 1.0


# ---------------------------------------------------------------------------
# C restatement (fp32, reference small-kernel order)
# ---------------------------------------------------------------------------
def _load_c_oracle():
    # GEV2_ORACLE_LIB: the sanitizer build of the same source
    path = os.environ.get("GEV2_ORACLE_LIB") or os.path.join(REPO, "oracle", "libgemm_oracle.so")
    if not os.path.exists(path):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle")], check=True)
    L = ctypes.CDLL(path)
    f = ctypes.POINTER(ctypes.c_float)
    i64 = ctypes.c_int64
    L.gev2o_gemm_fwd_f32.argtypes = [i64, i64, i64, f, i64, f, i64, f, ctypes.c_int, ctypes.c_float,
                                     ctypes.c_int, ctypes.c_float, f, i64, f, i64]
    L.gev2o_act_array.argtypes = [f, f, i64, ctypes.c_int, ctypes.c_float]
    L.gev2o_act_deriv_array.argtypes = [f, f, i64, ctypes.c_int, ctypes.c_float]
    L.gev2o_gemm_bwd_f32.argtypes = [i64, i64, i64, f, i64, f, i64, f, i64, f, i64, ctypes.c_int,
                                     ctypes.c_float, ctypes.c_float, ctypes.c_float, f, i64, f, i64,
                                     f, i64, f, ctypes.c_int, f]
    return L


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


@pytest.mark.parametrize("act", ACTS)
def test_c_oracle_activations(act):
    L = _load_c_oracle()
    x = np.linspace(-7, 7, 1001).astype(np.float32)
    y = np.empty_like(x)
    d = np.empty_like(x)
    a = O.parse_act(act)
    L.gev2o_act_array(_fp(x), _fp(y), x.size, a, 0.05)
    L.gev2o_act_deriv_array(_fp(x), _fp(d), x.size, a, 0.05)
    assert np.max(np.abs(y - O.act_forward(x, act, 0.05))) < 4e-6
    assert np.max(np.abs(d - O.act_deriv(x, act, 0.05))) < 4e-6


def test_c_oracle_forward_and_backward():
    L = _load_c_oracle()
    g = np.random.default_rng(6)
    M, N, K = 33, 21, 47
    X = (g.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    W = g.standard_normal((K, N)).astype(np.float32)
    b = g.standard_normal(N).astype(np.float32)
    Y = np.empty((M, N), np.float32)
    Z = np.empty((M, N), np.float32)
    L.gev2o_gemm_fwd_f32(M, N, K, _fp(X), K, _fp(W), N, _fp(b), O.BIAS_PERN, 1.0, O.ACT_GELU, 0.01,
                         _fp(Y), N, _fp(Z), N)
    Y64, Z64 = O.gemm_forward(X, W, b, O.BIAS_PERN, "gelu")
    bound = 1.01 * K * 2.0 ** -24 * (np.abs(X.astype(float)) @ np.abs(W.astype(float))) + 1e-6
    assert np.all(np.abs(Z - Z64) <= bound)
    assert np.all(np.abs(Y - Y64) <= 1.2 * bound + 1e-6)
    gY = g.standard_normal((M, N)).astype(np.float32)
    gA = np.empty((M, K), np.float32)
    gB = np.empty((K, N), np.float32)
    gC = np.empty((M, N), np.float32)
    gb = np.empty(N, np.float32)
    tmp = np.empty((M, N), np.float32)
    L.gev2o_gemm_bwd_f32(M, N, K, _fp(X), K, _fp(W), N, _fp(gY), N, _fp(Z), N, O.ACT_GELU, 0.01,
                         1.0, 1.0, _fp(gA), K, _fp(gB), N, _fp(gC), N, _fp(gb), O.BIAS_PERN, _fp(tmp))
    r = O.gemm_backward(X, W, gY, Z, "gelu", bias_kind=O.BIAS_PERN, beta=1.0)
    for name, dev in (("gA", gA), ("gB", gB), ("gC", gC), ("gBias", gb)):
        ref = r[name]
        assert np.max(np.abs(dev - ref)) <= 1e-5 * (1 + np.max(np.abs(ref))), name


def test_numpy_baseline_matches_oracle():
    g = np.random.default_rng(8)
    X = g.standard_normal((16, 24)).astype(np.float32)
    W = g.standard_normal((24, 12)).astype(np.float32)
    b = g.standard_normal((1, 12)).astype(np.float32)
    gY = g.standard_normal((16, 12)).astype(np.float32)
    Y, Z, gA, gB, gb = O.numpy_fp32_step(X, W, b, gY, "relu")
    Y64, Z64 = O.gemm_forward(X, W, b[0], O.BIAS_PERN, "relu")
    r = O.gemm_backward(X, W, gY, Z, "relu", bias_kind=O.BIAS_PERN)
    assert np.allclose(Y, Y64, atol=1e-5) and np.allclose(gA, r["gA"], atol=1e-4)
    assert np.allclose(gB, r["gB"], atol=1e-4) and np.allclose(gb[0], r["gBias"], atol=1e-4)


# ---------------------------------------------------------------------------
# 2-D convolution
# ---------------------------------------------------------------------------
def _conv_brute(X, W, b, stride, pad, dil):
    """Pure-Python integer loops over every output and tap (conv2d/kernels.cu:12-45 semantics)."""
    N, C, H, Wd = X.shape
    Co, _, Kh, Kw = W.shape
    Ho, Wo = O.conv2d_out_size(H, Wd, Kh, Kw, stride, pad, dil)
    out = [[[[0] * Wo for _ in range(Ho)] for _ in range(Co)] for _ in range(N)]
    for n in range(N):
        for co in range(Co):
            for ho in range(Ho):
                for wo in range(Wo):
                    acc = int(b[co]) if b is not None else 0
                    for c in range(C):
                        for kh in range(Kh):
                            for kw in range(Kw):
                                hi = ho * stride[0] - pad[0] + kh * dil[0]
                                wi = wo * stride[1] - pad[1] + kw * dil[1]
                                if 0 <= hi < H and 0 <= wi < Wd:
                                    acc += int(W[co, c, kh, kw]) * int(X[n, c, hi, wi])
                    out[n][co][ho][wo] = acc
    return np.array(out, dtype=np.float64)


@pytest.mark.parametrize("geom", [((1, 1), (1, 1), (1, 1)), ((2, 1), (0, 2), (1, 1)), ((1, 2), (1, 0), (2, 1))],
                         ids=["s1p1", "s2-pad0x2", "dil2"])
def test_conv2d_forward_exact_integers(geom):
    stride, pad, dil = geom
    g = np.random.default_rng(31)
    X = g.integers(-3, 4, (2, 3, 7, 6)).astype(np.float64)
    W = g.integers(-2, 3, (4, 3, 3, 2)).astype(np.float64)
    b = g.integers(-5, 6, 4).astype(np.float64)
    Y, Z = O.conv2d_forward(X, W, b, stride, pad, dil, act="relu")
    ref = _conv_brute(X, W, b, stride, pad, dil)
    assert np.array_equal(Z, ref)
    assert np.array_equal(Y, np.maximum(ref, 0))
    assert O.conv2d_out_size(7, 6, 3, 2, stride, pad, dil) == Z.shape[2:]


@pytest.mark.parametrize("act", ["none", "relu", "tanh"])
def test_conv2d_backward_matches_finite_difference(act):
    """d/dX, d/dW, d/db of L = sum(dY * act(conv(X, W) + b)) by central differences."""
    g = np.random.default_rng(33)
    stride, pad, dil = (2, 1), (1, 1), (1, 2)
    X = g.standard_normal((2, 2, 6, 7))
    W = g.standard_normal((3, 2, 2, 3))
    b = g.standard_normal(3)
    _, Z = O.conv2d_forward(X, W, b, stride, pad, dil, act=act)
    dY = g.standard_normal(Z.shape)
    grads = O.conv2d_backward(X, W, dY, Z, stride, pad, dil, act=act)

    def loss(X_, W_, b_):
        Y_, _ = O.conv2d_forward(X_, W_, b_, stride, pad, dil, act=act)
        return float((dY * Y_).sum())

    h = 1e-6
    for name, arr, idxs in (("dX", X, [(0, 1, 2, 3), (1, 0, 5, 6), (0, 0, 0, 0)]),
                            ("dW", W, [(2, 1, 1, 2), (0, 0, 0, 0)]), ("dB", b, [(1,)])):
        for idx in idxs:
            p, m = arr.copy(), arr.copy()
            p[idx] += h
            m[idx] -= h
            args_p = [X, W, b]
            args_m = [X, W, b]
            k = {"dX": 0, "dW": 1, "dB": 2}[name]
            args_p[k], args_m[k] = p, m
            fd = (loss(*args_p) - loss(*args_m)) / (2 * h)
            assert abs(fd - grads[name][idx]) <= 1e-5 * max(1.0, abs(fd)), (name, idx, fd, grads[name][idx])


def test_conv2d_1x1_is_the_plain_gemm():
    """A 1x1 / stride 1 / pad 0 convolution is, per image, W[Cout,Cin] . X_n[Cin, H*W] + b."""
    g = np.random.default_rng(35)
    X = g.standard_normal((2, 5, 4, 3))
    W = g.standard_normal((6, 5, 1, 1))
    b = g.standard_normal(6)
    _, Z = O.conv2d_forward(X, W, b)
    for n in range(2):
        _, ref = O.gemm_forward(W[:, :, 0, 0], X[n].reshape(5, 12), b, O.BIAS_PERM)
        assert np.allclose(Z[n].reshape(6, 12), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("geom", [((1, 1), (1, 1), (1, 1)), ((2, 1), (0, 2), (1, 1)), ((1, 2), (1, 0), (2, 1))],
                         ids=["s1p1", "s2-pad0x2", "dil2"])
def test_conv2d_backward_exact_integers(geom):
    """dX / dW / dB against pure-Python integer loops over every output and tap (act none)."""
    stride, pad, dil = geom
    g = np.random.default_rng(37)
    X = g.integers(-3, 4, (2, 3, 7, 6)).astype(np.float64)
    W = g.integers(-2, 3, (4, 3, 3, 2)).astype(np.float64)
    N, C, H, Wd = X.shape
    Co, _, Kh, Kw = W.shape
    Ho, Wo = O.conv2d_out_size(H, Wd, Kh, Kw, stride, pad, dil)
    dY = g.integers(-3, 4, (N, Co, Ho, Wo)).astype(np.float64)
    r = O.conv2d_backward(X, W, dY, np.zeros_like(dY), stride, pad, dil)
    dX = [[[[0] * Wd for _ in range(H)] for _ in range(C)] for _ in range(N)]
    dW = [[[[0] * Kw for _ in range(Kh)] for _ in range(C)] for _ in range(Co)]
    dB = [0] * Co
    for n in range(N):
        for co in range(Co):
            for ho in range(Ho):
                for wo in range(Wo):
                    d = int(dY[n, co, ho, wo])
                    dB[co] += d
                    for c in range(C):
                        for kh in range(Kh):
                            for kw in range(Kw):
                                hi = ho * stride[0] - pad[0] + kh * dil[0]
                                wi = wo * stride[1] - pad[1] + kw * dil[1]
                                if 0 <= hi < H and 0 <= wi < Wd:
                                    dW[co][c][kh][kw] += d * int(X[n, c, hi, wi])
                                    dX[n][c][hi][wi] += d * int(W[co, c, kh, kw])
    assert np.array_equal(r["dX"], np.array(dX, dtype=np.float64))
    assert np.array_equal(r["dW"], np.array(dW, dtype=np.float64))
    assert np.array_equal(r["dB"], np.array(dB, dtype=np.float64))


# ---------------------------------------------------------------------------
# Elman RNN
# ---------------------------------------------------------------------------
def test_rnn_forward_exact_integers():
    """Pure-Python integer recurrence h_t = X_t Wx + h_{t-1} Wh + b (act none), step by step."""
    g = np.random.default_rng(41)
    N, T, I, H = 2, 4, 3, 5
    X = g.integers(-2, 3, (N, T, I))
    Wx = g.integers(-1, 2, (I, H))
    Wh = g.integers(-1, 2, (H, H))
    h0 = g.integers(-2, 3, (N, H))
    b = g.integers(-3, 4, H)
    Y, Z = O.rnn_forward(X, Wx, Wh, h0, b)
    h = [[int(v) for v in row] for row in h0]
    for t in range(T):
        new = [[int(b[j]) + sum(int(X[n, t, i]) * int(Wx[i, j]) for i in range(I))
                + sum(h[n][k] * int(Wh[k, j]) for k in range(H)) for j in range(H)] for n in range(N)]
        assert np.array_equal(Z[:, t], np.array(new, dtype=np.float64))
        h = new
    assert np.array_equal(Y, Z)


def test_rnn_one_step_is_the_concatenated_gemm():
    """T = 1: act([X_0, h0] [Wx; Wh] + b), the reference's per-step GEMM (launcher.cu:186-205)."""
    g = np.random.default_rng(43)
    X, Wx, Wh = g.standard_normal((3, 1, 4)), g.standard_normal((4, 6)), g.standard_normal((6, 6))
    h0, b = g.standard_normal((3, 6)), g.standard_normal(6)
    Y, Z = O.rnn_forward(X, Wx, Wh, h0, b, act="tanh")
    Yg, Zg = O.gemm_forward(np.concatenate([X[:, 0], h0], axis=1), np.concatenate([Wx, Wh]), b, O.BIAS_PERN,
                            "tanh")
    assert np.allclose(Z[:, 0], Zg, rtol=1e-12, atol=1e-12) and np.allclose(Y[:, 0], Yg, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("act", ["none", "tanh", "relu", "sigmoid"])
def test_rnn_backward_matches_finite_difference(act):
    """d/dX, d/dWx, d/dWh, d/dh0, d/db of L = sum(dY * Y) by central differences: a dropped
    dh_next term, a wrong h_{t-1} or a transposed weight gradient fails here."""
    g = np.random.default_rng(45)
    N, T, I, H = 2, 4, 3, 5
    X, Wx = g.standard_normal((N, T, I)), 0.5 * g.standard_normal((I, H))
    Wh, h0, b = 0.5 * g.standard_normal((H, H)), g.standard_normal((N, H)), g.standard_normal(H)
    _, Z = O.rnn_forward(X, Wx, Wh, h0, b, act=act)
    dY = g.standard_normal(Z.shape)
    r = O.rnn_backward(X, Wx, Wh, h0, dY, Z, act=act)

    def loss(X_, Wx_, Wh_, h0_, b_):
        Y_, _ = O.rnn_forward(X_, Wx_, Wh_, h0_, b_, act=act)
        return float((dY * Y_).sum())

    args = [X, Wx, Wh, h0, b]
    h = 1e-6
    for k, name, idxs in ((0, "dX", [(0, 0, 1), (1, 3, 2), (1, 1, 0)]), (1, "dWx", [(2, 4), (0, 1)]),
                          (2, "dWh", [(3, 1), (0, 0)]), (3, "dh0", [(1, 2), (0, 4)]), (4, "dB", [(3,)])):
        for idx in idxs:
            p, m = [a.copy() for a in args], [a.copy() for a in args]
            p[k][idx] += h
            m[k][idx] -= h
            fd = (loss(*p) - loss(*m)) / (2 * h)
            # (relu: no pre-activation at this seed lies within h of the kink at 0)
            assert abs(fd - r[name][idx]) <= 1e-5 * max(1.0, abs(fd)), (act, name, idx, fd, r[name][idx])


# ---------------------------------------------------------------------------
# Scaled dot-product attention
# ---------------------------------------------------------------------------
def _qkv(seed, B=2, H=2, M=5, N=7, D=4):
    g = np.random.default_rng(seed)
    return g.standard_normal((B, H, M, D)), g.standard_normal((B, H, N, D)), g.standard_normal((B, H, N, D))


def test_sdpa_special_cases():
    Q, K, V = _qkv(51)
    # one key: softmax of a single score is 1, so Y is that key's value row
    Y, _, lse = O.sdpa_forward(Q, K[:, :, :1], V[:, :, :1])
    assert np.allclose(Y, np.broadcast_to(V[:, :, :1], Y.shape), atol=1e-12)
    # Q = 0: every score equal, so Y is the mean of the value rows and lse = log N
    Y, _, lse = O.sdpa_forward(np.zeros_like(Q), K, V)
    assert np.allclose(Y, np.broadcast_to(V.mean(axis=2, keepdims=True), Y.shape), atol=1e-12)
    assert np.allclose(lse, math.log(7), atol=1e-12)
    # causal: query 0 sees key 0 only
    Y, _, _ = O.sdpa_forward(Q, K, V, causal=True)
    assert np.allclose(Y[:, :, 0], V[:, :, 0], atol=1e-9)
    # a very large scale turns the softmax into an argmax
    Y, _, _ = O.sdpa_forward(Q, K, V, scale=1e4)
    idx = np.argmax(np.einsum("bhmd,bhnd->bhmn", Q, K), axis=-1)
    assert np.allclose(Y, np.take_along_axis(V, idx[..., None].repeat(4, -1), axis=2), atol=1e-6)


def test_sdpa_key_permutation_and_masks():
    Q, K, V = _qkv(53)
    perm = np.random.default_rng(1).permutation(7)
    Y, _, _ = O.sdpa_forward(Q, K, V)
    Yp, _, _ = O.sdpa_forward(Q, K[:, :, perm], V[:, :, perm])
    assert np.allclose(Y, Yp, atol=1e-12)
    # an I8 mask that drops keys equals attention over the kept keys only
    keep = np.array([1, 0, 1, 1, 0, 1, 1], bool)
    mask = np.broadcast_to(~keep, (2, 1, 5, 7)).astype(np.int8)
    Ym, _, _ = O.sdpa_forward(Q, K, V, mask=mask, mask_kind=O.MASK_I8)
    Yk, _, _ = O.sdpa_forward(Q, K[:, :, keep], V[:, :, keep], scale=1 / math.sqrt(4))
    assert np.allclose(Ym, Yk, atol=1e-12)
    # a constant F32 mask shifts every score of a row equally, which the softmax ignores
    Yc, _, _ = O.sdpa_forward(Q, K, V, mask=np.full((2, 1, 5, 7), 3.0, np.float32), mask_kind=O.MASK_F32)
    assert np.allclose(Yc, Y, atol=1e-5)


@pytest.mark.parametrize("causal,mk", [(False, O.MASK_NONE), (True, O.MASK_NONE), (False, O.MASK_I8)])
def test_sdpa_backward_matches_finite_difference(causal, mk):
    Q, K, V = _qkv(55)
    mask = None
    if mk == O.MASK_I8:
        mask = (np.random.default_rng(2).random((2, 1, 5, 7)) < 0.3).astype(np.int8)
        mask[..., 0] = 0
    dY = np.random.default_rng(3).standard_normal(Q.shape)
    r = O.sdpa_backward(Q, K, V, dY, causal=causal, mask=mask, mask_kind=mk)

    def loss(Q_, K_, V_):
        return float((dY * O.sdpa_forward(Q_, K_, V_, causal=causal, mask=mask, mask_kind=mk)[0]).sum())

    args = [Q, K, V]
    h = 1e-6
    for k, name, idxs in ((0, "dQ", [(0, 1, 2, 3), (1, 0, 4, 0)]), (1, "dK", [(0, 0, 6, 1), (1, 1, 2, 2)]),
                          (2, "dV", [(1, 0, 3, 3), (0, 1, 0, 0)])):
        for idx in idxs:
            p, m = [a.copy() for a in args], [a.copy() for a in args]
            p[k][idx] += h
            m[k][idx] -= h
            fd = (loss(*p) - loss(*m)) / (2 * h)
            assert abs(fd - r[name][idx]) <= 1e-5 * max(1.0, abs(fd)), (name, idx, fd, r[name][idx])


# ---------------------------------------------------------------------------
# Attention dropout: the reference's stateless splitmix64 stream
# ---------------------------------------------------------------------------
def test_splitmix64_known_answers():
    """SplitMix64's published output sequences (Vigna's reference splitmix64.c): the n-th
    output of a generator seeded with s is the mixing function applied to s + (n-1)*gamma,
    i.e. splitmix64(s + (n-1)*gamma) here (the function adds gamma itself)."""
    gamma = 0x9E3779B97F4A7C15
    M64 = (1 << 64) - 1
    seq = {0: [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F],
           1234567: [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                     16408922859458223821]}
    for seed, outs in seq.items():
        x = np.array([(seed + i * gamma) & M64 for i in range(len(outs))], np.uint64)
        assert [int(v) for v in O.splitmix64(x)] == outs


def test_dropout_factors_stream():
    """Counter layout, keep rule and scaling: element (b,h,q,k) uses counter ((b*H+h)*M+q)*N+k;
    p = 0 keeps everything unscaled; the kept fraction matches 1 - p within 5 sigma; kept
    entries carry 1/(1-p) (or 1 without scale_in_train); p = 1 drops everything."""
    B, H, M, N, seed = 2, 3, 40, 50, 987654321
    f = O.dropout_factors(seed, B, H, M, N, 0.25)
    # one element recomputed with Python integers from the counter formula
    b, h, q, k = 1, 2, 17, 33
    ctr = ((b * H + h) * M + q) * N + k
    u = int(O.splitmix64(np.array([seed ^ ctr], np.uint64))[0]) & 0xFFFFFFFF
    kept = float(np.float32(u)) * 2.0 ** -32 >= 0.25
    assert f[b, h, q, k] == (np.float32(1) / np.float32(0.75) if kept else 0)
    n = f.size
    frac = float((f > 0).mean())
    assert abs(frac - 0.75) <= 5 * math.sqrt(0.75 * 0.25 / n)
    assert set(np.unique(f)) <= {0.0, float(np.float32(1) / np.float32(0.75))}
    assert np.all(O.dropout_factors(seed, B, H, M, N, 0.0) == 1)
    g = O.dropout_factors(seed, B, H, M, N, 0.25, scale_in_train=False)
    assert np.array_equal(g > 0, f > 0) and set(np.unique(g)) <= {0.0, 1.0}
    assert np.all(O.dropout_factors(seed, B, H, M, N, 1.0) == 0)
    # another seed gives another mask
    assert not np.array_equal(O.dropout_factors(seed + 1, B, H, M, N, 0.25) > 0, f > 0)


def test_sdpa_dropout_forward_and_backward():
    """With dropout, Y = (P . factors) V (so Q = K = 0 and V = I expose the factors directly),
    and the backward is the gradient of that function for the fixed mask (central finite
    differences of a scalar loss)."""
    B, H, M, N = 2, 2, 5, 7
    seed, p = 42, 0.3
    Y, _, _ = O.sdpa_forward(np.zeros((B, H, M, N)), np.zeros((B, H, N, N)), np.broadcast_to(np.eye(N), (B, H, N, N)),
                             dropout_p=p, seed=seed)
    assert np.allclose(Y, O.dropout_factors(seed, B, H, M, N, p) / N, atol=1e-15)
    Q, K, V = _qkv(56)
    dY = np.random.default_rng(4).standard_normal(Q.shape)
    r = O.sdpa_backward(Q, K, V, dY, dropout_p=p, seed=seed)

    def loss(Q_, K_, V_):
        return float((dY * O.sdpa_forward(Q_, K_, V_, dropout_p=p, seed=seed)[0]).sum())

    args = [Q, K, V]
    h = 1e-6
    for k, name, idxs in ((0, "dQ", [(0, 1, 2, 3), (1, 0, 4, 0)]), (1, "dK", [(0, 0, 6, 1), (1, 1, 2, 2)]),
                          (2, "dV", [(1, 0, 3, 3), (0, 1, 0, 0)])):
        for idx in idxs:
            a_, m_ = [a.copy() for a in args], [a.copy() for a in args]
            a_[k][idx] += h
            m_[k][idx] -= h
            fd = (loss(*a_) - loss(*m_)) / (2 * h)
            assert abs(fd - r[name][idx]) <= 1e-5 * max(1.0, abs(fd)), (name, idx, fd, r[name][idx])
    # p = 0 is the plain attention
    r0 = O.sdpa_backward(Q, K, V, dY)
    rz = O.sdpa_backward(Q, K, V, dY, dropout_p=0.0, seed=seed)
    assert all(np.array_equal(r0[k], rz[k]) for k in r0)
