"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Forward:  Y = act(alpha*X W + b), Z = pre-activation   (reference: launcher.cu:147-274,
          traits.hpp:43-71, activations.hpp:14-39)
Backward: gA = (gY . act'(Z)) W^T, gB = X^T (gY . act'(Z)), gBias, gC
          (reference: regemm_backward.cu:91-130,151-301)
Tolerances: fp32 accumulation bound gamma_K*(|X||W|) plus one rounding of the
stored output (see gemm_helpers.fwd_bound); ReLU masks bit-exact.
"""
import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import (BF16, F16, F32, DT_NAMES, U_ACC, U_OUT, Dev, act_lipschitz,
                          assert_close, fwd_bound, make_fwd_inputs, rounded, run_fwd)

pytestmark = pytest.mark.gpu

ACTS = ["none", "relu", "leakyrelu", "gelu", "sigmoid", "tanh"]
BIASES = [O.BIAS_PERN, O.BIAS_PERM, O.BIAS_SCALAR, O.BIAS_NONE]

# (M, N, K): covers the 64x64 / 128x128 / 128x256 tiles, ragged edges, the
# scalar-load variant (K not a multiple of 16 bytes) and the skinny kernel.
FWD_SHAPES = [
    (64, 256, 784),     # BASELINE config 1 (MLP dense layer)
    (33, 45, 70),       # ragged; K*elem not a multiple of 16 B -> scalar loads
    (200, 136, 96),     # ragged M/N on the vector path
    (520, 1040, 256),   # multi-tile
    (8, 512, 1024),     # skinny (M <= 16), split-K
    (13, 264, 320),     # skinny, M in (8, 16]
    (1, 64, 64),        # single row
]


def _check_fwd(capi, M, N, K, dtype, act, bias_kind, seed, alpha=1.0, slope=0.01):
    X, W, b = make_fwd_inputs(seed, M, N, K, dtype, bias_kind)
    dev = Dev(capi)
    try:
        Y, Z, path = run_fwd(capi, dev, X, W, b, bias_kind, act, dtype, alpha=alpha, slope=slope)
    finally:
        dev.close()
    Y64, Z64 = O.gemm_forward(X, W, b, bias_kind if b is not None else None, act, slope, alpha)
    bvals = None
    if b is not None:
        bvals = O.bias_add(np.zeros((M, N)), b, bias_kind)
    bz = abs(alpha) * fwd_bound(X, W, K, dtype, bvals)
    u = U_OUT[dtype]
    tag = f"{DT_NAMES[dtype]} {M}x{N}x{K} act={act} bias={bias_kind} path={path}"
    assert_close(Z, Z64, bz + u * np.abs(Z64) + 1e-30, "Z " + tag,
                 rel_norm=1e-4 if dtype == F32 else 1e-2)
    ya = act_lipschitz(act) * bz + u * np.abs(Y64) + 8 * U_ACC * np.abs(Y64) + 2e-7
    assert_close(Y, Y64, ya, "Y " + tag, rel_norm=1e-4 if dtype == F32 else 1e-2)
    if O.parse_act(act) == O.ACT_RELU:
        # (i) internal consistency: Y == Z where Z > 0, else +0, bit for bit
        pos = Z > 0
        assert np.array_equal(Y[pos], Z[pos]), tag
        assert np.all(Y[~pos] == 0) and not np.any(np.signbit(Y[~pos])), tag
        # (ii) agreement with the fp64 mask wherever |Z64| exceeds the error bound
        sure = np.abs(Z64) > bz
        assert np.array_equal(pos[sure], (Z64 > 0)[sure]), tag
    return path


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: DT_NAMES[d])
@pytest.mark.parametrize("shape", FWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_forward_shapes(gpu, dtype, shape):
    M, N, K = shape
    i = FWD_SHAPES.index(shape)
    act = ACTS[(i + dtype) % len(ACTS)]
    bias = BIASES[(i + 2 * dtype) % len(BIASES)]
    path = _check_fwd(gpu, M, N, K, dtype, act, bias, seed=1000 + 10 * i + dtype)
    if M <= 16 and K >= 64:
        # fp32 with K >= 128 takes the one-launch small kernel instead
        assert path.startswith("skinny") or (dtype == F32 and K >= 128 and path == "small"), path
    elif (K * (4 if dtype == F32 else 2)) % 16:
        assert path.endswith("scalar")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: DT_NAMES[d])
@pytest.mark.parametrize("act", ACTS)
def test_forward_activations(gpu, dtype, act):
    _check_fwd(gpu, 96, 160, 128, dtype, act, O.BIAS_PERN, seed=77, slope=0.05)


def test_forward_alpha(gpu):
    _check_fwd(gpu, 128, 128, 256, BF16, "relu", O.BIAS_PERN, seed=5, alpha=0.125)


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: DT_NAMES[d])
def test_forward_k_zero(gpu, dtype):
    """K = 0: Y = act(bias) (the accumulator is empty)."""
    capi = gpu
    M, N = 20, 24
    b = np.linspace(-1, 1, N).astype(np.float32)
    dev = Dev(capi)
    try:
        pb = dev.put(b)
        pY = dev.empty(M * N * capi.elem_bytes(dtype))
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=0, A=0, B=0, Y=pY, bias=pb,
                      bias_kind=O.BIAS_PERN, act="relu")
        capi.synchronize()
        Y = dev.get(pY, (M, N), dtype)
    finally:
        dev.close()
    ref = np.maximum(np.broadcast_to(rounded(b, dtype), (M, N)), 0)
    assert np.array_equal(Y, ref)


# ---------------------------------------------------------------------------
# Backward
# ---------------------------------------------------------------------------
BWD_CASES = [
    # (M, N, K, dtype, act, bias_kind, want_gA, want_gB, want_gC)
    (64, 256, 784, F32, "relu", O.BIAS_PERN, True, True, False),    # config 1 (fused dBias)
    (200, 136, 96, BF16, "gelu", O.BIAS_PERN, True, True, True),
    (33, 45, 70, F32, "leakyrelu", O.BIAS_PERM, True, True, False),  # scalar loads, PerM
    (33, 45, 70, BF16, "tanh", O.BIAS_SCALAR, True, True, False),
    (8, 512, 1024, BF16, "none", O.BIAS_PERN, True, True, False),    # skinny forward shape
    (300, 260, 520, F16, "sigmoid", O.BIAS_PERN, True, False, False),  # dBias w/o dW
    (256, 512, 384, BF16, "relu", O.BIAS_PERN, True, True, True),
    (130, 200, 64, F32, "gelu", O.BIAS_NONE, False, True, False),
    # M <= 16: gA on the skinny NT kernel (act' on the fly, or on a materialised dY')
    (5, 384, 200, F32, "relu", O.BIAS_PERN, True, True, False),
    (16, 1024, 1536, BF16, "tanh", O.BIAS_PERN, True, True, False),
    (1, 64, 96, F16, "leakyrelu", O.BIAS_SCALAR, True, False, False),
    (12, 520, 72, F32, "gelu", O.BIAS_PERM, True, True, True),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: f"{DT_NAMES[c[3]]}-{c[0]}x{c[1]}x{c[2]}-{c[4]}")
def test_backward(gpu, case):
    capi = gpu
    M, N, K, dtype, act, bias_kind, wA, wB, wC = case
    seed = 4000 + M + N + K
    X, W, b = make_fwd_inputs(seed, M, N, K, dtype, bias_kind)
    g = np.random.default_rng(seed + 1)
    gY = rounded(g.standard_normal((M, N)), dtype)
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        # forward first: the backward consumes the device's own Z stash
        Y, Z, _ = run_fwd(capi, dev, X, W, b, bias_kind, act, dtype)
        pX = dev.put(capi.to_storage(X, dtype))
        pW = dev.put(capi.to_storage(W, dtype))
        pgY = dev.put(capi.to_storage(gY, dtype))
        pZ = dev.put(capi.to_storage(Z, dtype))
        pgA = dev.empty(M * K * es) if wA else 0
        pgB = dev.empty(K * N * es) if wB else 0
        pgC = dev.empty(M * N * es) if wC else 0
        nb = {O.BIAS_NONE: 0, O.BIAS_SCALAR: 1, O.BIAS_PERM: M, O.BIAS_PERN: N}[bias_kind]
        pgb = dev.empty(max(nb, 1) * 4) if nb else 0
        capi.gemm_bwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, gA=pgA, gB=pgB,
                      gC=pgC, gBias=pgb, bias_kind=bias_kind, act=act, beta=1.0 if wC else 0.0)
        capi.synchronize()
        gA = dev.get(pgA, (M, K), dtype) if wA else None
        gB = dev.get(pgB, (K, N), dtype) if wB else None
        gC = dev.get(pgC, (M, N), dtype) if wC else None
        gb = dev.get_f32(pgb, (nb,)) if nb else None
    finally:
        dev.close()
    ref = O.gemm_backward(X, W, gY, Z, act, 0.01, bias_kind, 1.0, 1.0)
    gZ = ref["gZ"]
    u = U_OUT[dtype]
    e16 = 0.0 if (dtype == F32 or O.parse_act(act) in (O.ACT_NONE, O.ACT_RELU)) else U_OUT[dtype]
    aG, aY = np.abs(gZ), np.abs(gY.astype(np.float64))
    tag = f"{DT_NAMES[dtype]} {M}x{N}x{K} act={act}"
    if wA:
        Wt = np.abs(W.astype(np.float64)).T
        bnd = (1.01 * N * U_ACC + e16) * (aG @ Wt) + 1e-6 * (aY @ Wt) + u * np.abs(ref["gA"]) + 1e-30
        assert_close(gA, ref["gA"], bnd, "gA " + tag, rel_norm=1e-4 if dtype == F32 else 1e-2)
    if wB:
        Xt = np.abs(X.astype(np.float64)).T
        bnd = (1.01 * M * U_ACC + e16) * (Xt @ aG) + 1e-6 * (Xt @ aY) + u * np.abs(ref["gB"]) + 1e-30
        assert_close(gB, ref["gB"], bnd, "gB " + tag, rel_norm=1e-4 if dtype == F32 else 1e-2)
    if wC:
        assert_close(gC, gZ, u * aG + 1e-6 * aY + 1e-30, "gC " + tag)
    if gb is not None:
        if bias_kind == O.BIAS_PERN:
            s, sy = aG.sum(0), aY.sum(0)
        elif bias_kind == O.BIAS_PERM:
            s, sy = aG.sum(1), aY.sum(1)
        else:
            s, sy = np.array([aG.sum()]), np.array([aY.sum()])
        n_terms = {O.BIAS_PERN: M, O.BIAS_PERM: N, O.BIAS_SCALAR: M * N}[bias_kind]
        assert_close(gb, ref["gBias"], 1.01 * n_terms * U_ACC * s + 1e-6 * sy + 1e-30, "gBias " + tag)
    if O.parse_act(act) == O.ACT_RELU and wC:
        # dY' == dY where Z > 0 else 0, exactly
        pos = Z > 0
        assert np.array_equal(gC[pos], gY[pos]) and np.all(gC[~pos] == 0)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: DT_NAMES[d])
def test_backward_gc_beta_zero(gpu, dtype):
    """beta = 0 (no C in the forward): gC is zero-filled, as the reference's backward does
    (regemm_backward.cu:183-189), even where dY is inf or NaN."""
    capi = gpu
    M, N, K = 24, 40, 16
    g = np.random.default_rng(17)
    gY = rounded(g.standard_normal((M, N)), dtype)
    gY[0, :4] = [np.inf, -np.inf, np.nan, 1.0]
    Z = rounded(g.standard_normal((M, N)), dtype)
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pgY, pZ = dev.put(capi.to_storage(gY, dtype)), dev.put(capi.to_storage(Z, dtype))
        pgC = dev.empty(M * N * es)
        capi.gemm_bwd(dtype=dtype, M=M, N=N, K=K, A=0, B=0, gY=pgY, Z=pZ, gC=pgC, act="relu", beta=0.0)
        capi.synchronize()
        gC = dev.get(pgC, (M, N), dtype)
    finally:
        dev.close()
    assert np.all(gC == 0) and not np.any(np.signbit(gC))


# ---------------------------------------------------------------------------
# Batched / strided forms (exact-integer inputs: results must be bit-exact)
# ---------------------------------------------------------------------------
def _int_inputs(g, shape, lo=-2, hi=2):
    return g.integers(lo, hi + 1, size=shape).astype(np.float32)


@pytest.mark.parametrize("dtype", [BF16, F16, F32], ids=lambda d: DT_NAMES[d])
def test_batched_sdpa_form_exact(gpu, dtype):
    """S = (Q K^T) * 1/8 per (b,h) slice, then Y = P V; sdpa/launcher.cu:166-170,185-270.
    Layout: [B*H, rows, D] contiguous, slice stride rows*D (and M*N for S/P)."""
    capi = gpu
    BH, Mq, Nk, D = 16, 128, 96, 64
    g = np.random.default_rng(11)
    Q = _int_inputs(g, (BH, Mq, D))
    Kt = _int_inputs(g, (BH, Nk, D))
    V = _int_inputs(g, (BH, Nk, D))
    P = (g.random((BH, Mq, Nk)) < 0.05).astype(np.float32) * _int_inputs(g, (BH, Mq, Nk), 1, 2)
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pQ, pK, pV, pP = (dev.put(capi.to_storage(a, dtype)) for a in (Q, Kt, V, P))
        pS = dev.empty(BH * Mq * Nk * es)
        pY = dev.empty(BH * Mq * D * es)
        capi.gemm_fwd(dtype=dtype, M=Mq, N=Nk, K=D, A=pQ, B=pK, Y=pS, trans_b=True, alpha=0.125,
                      batch=BH, stride_a=Mq * D, stride_b=Nk * D, stride_y=Mq * Nk)
        capi.gemm_fwd(dtype=dtype, M=Mq, N=D, K=Nk, A=pP, B=pV, Y=pY, batch=BH,
                      stride_a=Mq * Nk, stride_b=Nk * D, stride_y=Mq * D)
        capi.synchronize()
        S = dev.get(pS, (BH, Mq, Nk), dtype)
        Y = dev.get(pY, (BH, Mq, D), dtype)
    finally:
        dev.close()
    S64, _ = O.gemm_forward_batched(Q, Kt, BH, Mq, Nk, D, Mq * D, Nk * D, D, D, trans_b=True,
                                    alpha=0.125)
    Y64, _ = O.gemm_forward_batched(P, V, BH, Mq, D, Nk, Mq * Nk, Nk * D, Nk, D)
    # exact integer sums (< 2^24) scaled by a power of two: one final rounding only
    assert np.array_equal(S, rounded(S64, dtype))
    assert np.array_equal(Y, rounded(Y64, dtype))


@pytest.mark.parametrize("dtype", [BF16, F32], ids=lambda d: DT_NAMES[d])
def test_batched_padded_strides_exact(gpu, dtype):
    """Slices with ld > cols and gaps between slices; untouched padding must stay untouched."""
    capi = gpu
    B, M, N, K = 3, 40, 48, 32
    lda, ldb, ldy = K + 8, N + 8, N + 16
    sA, sB, sY = M * lda + 64, K * ldb + 32, M * ldy + 128
    g = np.random.default_rng(3)
    A = _int_inputs(g, (B * sA,))
    Bm = _int_inputs(g, (B * sB,))
    bias = _int_inputs(g, (B * N,)).astype(np.float32)
    es = capi.elem_bytes(dtype)
    poison = np.full(B * sY, 7.0, np.float32)
    dev = Dev(capi)
    try:
        pA, pB = dev.put(capi.to_storage(A, dtype)), dev.put(capi.to_storage(Bm, dtype))
        pY = dev.put(capi.to_storage(poison, dtype))
        pb = dev.put(bias)
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=K, A=pA, B=pB, Y=pY, bias=pb,
                      bias_kind=O.BIAS_PERN, act="relu", batch=B, lda=lda, ldb=ldb, ldy=ldy,
                      stride_a=sA, stride_b=sB, stride_y=sY, stride_bias=N)
        capi.synchronize()
        Yflat = dev.get(pY, (B * sY,), dtype)
    finally:
        dev.close()
    Y64, _ = O.gemm_forward_batched(A, Bm, B, M, N, K, sA, sB, lda, ldb, bias=bias,
                                    bias_kind=O.BIAS_PERN, sBias=N, act="relu")
    expect = poison.copy()
    for i in range(B):
        for m in range(M):
            expect[i * sY + m * ldy: i * sY + m * ldy + N] = Y64[i, m]
    assert np.array_equal(Yflat, rounded(expect, dtype))


def test_conv_im2col_form(gpu):
    """conv2d lowered to one GEMM over stacked images (conv2d/launcher.cu:180-227,
    kernels.cu:12-45): Col[N*Ho*Wo, Cin*3*3] x W_KC[Cin*9, Cout] + b, ReLU."""
    capi = gpu
    n_img, cin, H, Wd, cout = 2, 8, 10, 12, 16
    g = np.random.default_rng(9)
    x = g.uniform(0, 1, (n_img, cin, H, Wd)).astype(np.float32)
    w = (g.standard_normal((cout, cin, 3, 3)) * np.sqrt(2 / (cin * 9))).astype(np.float32)
    b = (0.02 * g.standard_normal(cout)).astype(np.float32)
    xp = np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 1)))
    col = np.empty((n_img * H * Wd, cin * 9), np.float32)
    for n in range(n_img):
        for oh in range(H):
            for ow in range(Wd):
                row = (n * H + oh) * Wd + ow
                col[row] = xp[n, :, oh:oh + 3, ow:ow + 3].reshape(-1)   # k = (c*3+kh)*3+kw
    w_kc = w.reshape(cout, cin * 9).T.copy()
    _check = None
    dev = Dev(capi)
    try:
        Y, Z, _ = run_fwd(capi, dev, col, w_kc, b, O.BIAS_PERN, "relu", F32)
    finally:
        dev.close()
    ref = np.zeros((n_img, cout, H, Wd))
    for co in range(cout):
        for n in range(n_img):
            acc = np.zeros((H, Wd))
            for c in range(cin):
                for kh in range(3):
                    for kw in range(3):
                        acc += w[co, c, kh, kw].astype(np.float64) * xp[n, c, kh:kh + H, kw:kw + Wd]
            ref[n, co] = np.maximum(acc + b[co], 0)
    Ynchw = Y.reshape(n_img, H, Wd, cout).transpose(0, 3, 1, 2)
    assert np.max(np.abs(Ynchw - ref)) < 1e-5
    del _check


@pytest.mark.parametrize("fused", [False, True], ids=["materialised", "fused"])
def test_backward_both_dy_paths(gpu, fused, monkeypatch):
    """M*N*K = 2^30: the backward materialises dY' (vector pass + fixed-order dBias
    partials) unless GEV2_FUSED_BWD forces the act'-prologue GEMMs; both must agree
    with the oracle, and ReLU masks must agree bit for bit."""
    capi = gpu
    if fused:
        monkeypatch.setenv("GEV2_FUSED_BWD", "1")
    M = N = K = 1024
    dtype = BF16
    X, W, b = make_fwd_inputs(77, M, N, K, dtype, O.BIAS_PERN)
    gY = rounded(np.random.default_rng(78).standard_normal((M, N)), dtype)
    dev = Dev(capi)
    try:
        Y, Z, _ = run_fwd(capi, dev, X, W, b, O.BIAS_PERN, "relu", dtype)
        pX, pW = dev.put(capi.to_storage(X, dtype)), dev.put(capi.to_storage(W, dtype))
        pgY, pZ = dev.put(capi.to_storage(gY, dtype)), dev.put(capi.to_storage(Z, dtype))
        pgA, pgB, pgb = dev.empty(M * K * 2), dev.empty(K * N * 2), dev.empty(N * 4)
        capi.gemm_bwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, gA=pgA, gB=pgB,
                      gBias=pgb, bias_kind=O.BIAS_PERN, act="relu")
        capi.synchronize()
        gA, gB = dev.get(pgA, (M, K), dtype), dev.get(pgB, (K, N), dtype)
        gb = dev.get_f32(pgb, (N,))
    finally:
        dev.close()
    ref = O.gemm_backward(X, W, gY, Z, "relu", bias_kind=O.BIAS_PERN)
    aG, aY = np.abs(ref["gZ"]), np.abs(gY.astype(np.float64))
    u = U_OUT[dtype]
    Wt, Xt = np.abs(W.astype(np.float64)).T, np.abs(X.astype(np.float64)).T
    assert_close(gA, ref["gA"], 1.01 * N * U_ACC * (aG @ Wt) + u * np.abs(ref["gA"]) + 1e-30, "gA",
                 rel_norm=1e-2)
    assert_close(gB, ref["gB"], 1.01 * M * U_ACC * (Xt @ aG) + u * np.abs(ref["gB"]) + 1e-30, "gB",
                 rel_norm=1e-2)
    assert_close(gb, ref["gBias"], 1.01 * M * U_ACC * aG.sum(0) + 1e-30, "gBias")


SPLITK_CASES = [
    # (M, N, K, act, bias): fp32 problems of at most 32 64x64 tiles with K >= 256 split K
    (64, 256, 784, "relu", O.BIAS_PERN),      # C1
    (100, 132, 1000, "gelu", O.BIAS_PERM),    # ragged M / N, K tail slice
    (32, 64, 4096, "tanh", O.BIAS_SCALAR),    # one tile, many slices
    (256, 512, 256, "none", O.BIAS_NONE),     # 32 tiles, the limit
]


@pytest.mark.parametrize("case", SPLITK_CASES, ids=lambda c: "x".join(map(str, c[:3])))
def test_fp32_splitk(gpu, case, monkeypatch):
    """fp32 split-K: slices on the tile kernel into fp32 partials, then an ordered sum with
    alpha, bias, Z and act.  Within the fp32 bound of the oracle, bit-identical with or without
    a caller workspace (same slices, same order), and equal to the unsplit path within the bound."""
    capi = gpu
    M, N, K, act, bk = case
    monkeypatch.setenv("GEV2_NO_SMALL", "1")        # these shapes otherwise take the small kernel
    path = _check_fwd(capi, M, N, K, F32, act, bk, seed=700 + M, alpha=0.5)
    assert path == "tile:splitk", path
    X, W, b = make_fwd_inputs(701, M, N, K, F32, bk)
    dev = Dev(capi)
    try:
        pX, pW = dev.put(X), dev.put(W)
        pb = dev.put(b) if b is not None else 0
        kw = dict(dtype=F32, M=M, N=N, K=K, A=pX, B=pW, bias=pb, bias_kind=bk if b is not None else 0, act=act)
        need = capi.fwd_workspace_size(Y=1 << 20, **kw)
        assert need > 0
        outs = []
        for ws in (dev.empty(need), 0):
            pY, pZ = dev.empty(M * N * 4), dev.empty(M * N * 4)
            capi.gemm_fwd(Y=pY, Z=pZ, workspace=ws, workspace_bytes=need if ws else 0, **kw)
            capi.synchronize()
            outs.append((dev.get_f32(pY, (M, N)), dev.get_f32(pZ, (M, N))))
        monkeypatch.setenv("GEV2_NO_SPLITK", "1")
        pY, pZ = dev.empty(M * N * 4), dev.empty(M * N * 4)
        capi.gemm_fwd(Y=pY, Z=pZ, **kw)
        assert capi.last_path() != "tile:splitk"
        capi.synchronize()
        plain = dev.get_f32(pZ, (M, N))
    finally:
        dev.close()
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    bvals = O.bias_add(np.zeros((M, N)), b, bk) if b is not None else None
    bz = fwd_bound(X, W, K, F32, bvals)
    assert np.all(np.abs(plain - outs[0][1]) <= 2 * bz + 2 * U_OUT[F32] * np.abs(plain) + 1e-30)


@pytest.mark.parametrize("case", [(64, 256, 784, "relu"), (100, 520, 132, "leakyrelu"), (40, 1000, 64, "none")],
                         ids=lambda c: "x".join(map(str, c[:3])))
def test_fp32_backward_dx_splitk(gpu, case, monkeypatch):
    """Small fp32 backward with dY' formed while loading: dX (few 64x64 tiles, long reduction
    over N) is split over workgroups into fp32 partials and summed in order.  Same result with
    the caller's workspace as with the library's buffer, within the fp32 bound of the oracle,
    and within twice that bound of the unsplit launch."""
    capi = gpu
    M, N, K, act = case
    monkeypatch.setenv("GEV2_NO_SMALL", "1")        # these shapes otherwise take the small kernel
    X, W, b = make_fwd_inputs(810 + M, M, N, K, F32, O.BIAS_PERN)
    gY = np.random.default_rng(811 + M).standard_normal((M, N)).astype(np.float32)
    Z = np.random.default_rng(812 + M).standard_normal((M, N)).astype(np.float32)
    dev = Dev(capi)
    try:
        pX, pW, pgY, pZ = dev.put(X), dev.put(W), dev.put(gY), dev.put(Z)
        kw = dict(dtype=F32, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, act=act, alpha=0.75)
        import ctypes
        need = capi.lib().gev2_gemm_bwd_workspace_size(ctypes.byref(capi.bwd_desc(gA=1 << 20, **kw)))
        assert need > 0 and need % (M * K * 4) == 0 and need // (M * K * 4) >= 2   # >= 2 slices of [M,K] fp32
        outs = []
        for ws in (dev.empty(need), 0):
            pgA = dev.empty(M * K * 4)
            capi.gemm_bwd(gA=pgA, workspace=ws, workspace_bytes=need if ws else 0, **kw)
            capi.synchronize()
            outs.append(dev.get_f32(pgA, (M, K)))
        monkeypatch.setenv("GEV2_NO_SPLITK", "1")
        pgA = dev.empty(M * K * 4)
        capi.gemm_bwd(gA=pgA, **kw)
        capi.synchronize()
        plain = dev.get_f32(pgA, (M, K))
    finally:
        dev.close()
    assert np.array_equal(outs[0], outs[1])
    ref = O.gemm_backward(X, W, gY, Z, act, 0.01, O.BIAS_NONE, 0.75)
    aG = np.abs(gY.astype(np.float64) * O.act_deriv(Z, act))
    bnd = 0.75 * 1.01 * N * U_ACC * (aG @ np.abs(W.astype(np.float64)).T) + U_OUT[F32] * np.abs(ref["gA"]) + 1e-30
    assert_close(outs[0], ref["gA"], bnd, f"dX split {M}x{N}x{K}", rel_norm=1e-4)
    assert np.all(np.abs(outs[0] - plain) <= 2 * bnd)


def test_skinny_full_size(gpu):
    """BASELINE config 5b: M=8, N=K=4096, bf16, bias, through the skinny kernel."""
    path = _check_fwd(gpu, 8, 4096, 4096, BF16, "none", O.BIAS_PERN, seed=55)
    assert path == "skinny:split"


def test_skinny_repeat_calls(gpu):
    """Repeated skinny calls stay correct (the split-K partials in the per-stream
    workspace are rewritten by every call); K = 2048 + 640 also covers a partial
    last K block."""
    for i in range(3):
        _check_fwd(gpu, 4, 384, 2048, BF16, "relu", O.BIAS_PERN, seed=60 + i)
    _check_fwd(gpu, 16, 264, 2688, F32, "gelu", O.BIAS_PERM, seed=64)
    _check_fwd(gpu, 5, 136, 2688, F16, "none", O.BIAS_SCALAR, seed=65)
