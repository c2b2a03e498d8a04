"""GPU parity of the small fp32 kernel (one launch for the whole forward, one for the whole
backward) against the CPU oracle, through the C ABI.

The reference runs these layers on its general tile kernel and backward driver
(regemm_epilogue.cu, regemm_backward.cu:151-301, launcher.cu:147-383); the oracle restates
that arithmetic (oracle/gemm_oracle.py).  Checked here:
  - forward Z / Y within the fp32 accumulation bound, every activation and bias kind, both
    transposes, alpha, ragged edges; ReLU masks bit for bit;
  - backward dX, dW and the PerN dBias with dY' = dY (.) act'(Z) formed while loading, every
    activation, each output alone, no scratch;
  - exact-integer inputs (every sum exact in fp32): bit-identical to the oracle;
  - results repeat bit for bit, and agree with the multi-launch path (GEV2_NO_SMALL=1).
"""
import ctypes

import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import (F32, U_ACC, U_OUT, Dev, act_lipschitz, assert_close, fwd_bound,
                          make_fwd_inputs)

pytestmark = pytest.mark.gpu

ACTS = ["none", "relu", "leakyrelu", "gelu", "sigmoid", "tanh"]
NB = {O.BIAS_NONE: 0, O.BIAS_SCALAR: 1, O.BIAS_PERM: None, O.BIAS_PERN: None}


def _nbias(kind, M, N):
    return {O.BIAS_NONE: 0, O.BIAS_SCALAR: 1, O.BIAS_PERM: M, O.BIAS_PERN: N}[kind]


def _fwd(capi, X, W, b, bias_kind, act, alpha=1.0, slope=0.01, ta=False, tb=False):
    """Forward through the C ABI with X [M,K] and W [K,N] given logically; stored
    transposed when ta / tb.  Returns Y, Z and the path taken."""
    M, K = X.shape
    N = W.shape[1]
    dev = Dev(capi)
    try:
        pX = dev.put(np.ascontiguousarray(X.T if ta else X, np.float32))
        pW = dev.put(np.ascontiguousarray(W.T if tb else W, np.float32))
        pb = dev.put(b) if b is not None else 0
        pY, pZ = dev.empty(M * N * 4), dev.empty(M * N * 4)
        capi.gemm_fwd(dtype=F32, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb,
                      bias_kind=bias_kind if b is not None else 0, act=act, leaky_slope=slope,
                      alpha=alpha, trans_a=ta, trans_b=tb)
        path = capi.last_path()
        capi.synchronize()
        return dev.get_f32(pY, (M, N)), dev.get_f32(pZ, (M, N)), path
    finally:
        dev.close()


FWD_CASES = [
    # (M, N, K, act, bias_kind, alpha, trans_a, trans_b)
    (64, 256, 784, "relu", O.BIAS_PERN, 1.0, False, False),      # C1
    (100, 132, 1000, "gelu", O.BIAS_PERM, 0.5, False, False),    # ragged M / N
    (37, 90, 130, "tanh", O.BIAS_SCALAR, 1.0, True, False),      # A stored [K,M]
    (48, 70, 300, "sigmoid", O.BIAS_NONE, 2.0, False, True),     # B stored [N,K]
    (17, 33, 2048, "leakyrelu", O.BIAS_PERN, 1.0, True, True),   # longest reduction
    (256, 512, 256, "none", O.BIAS_PERN, 1.0, False, False),     # 512 tiles, the limit
]


@pytest.mark.parametrize("case", FWD_CASES, ids=lambda c: "x".join(map(str, c[:3])) + f"-{c[3]}")
def test_small_forward(gpu, case):
    capi = gpu
    M, N, K, act, bk, alpha, ta, tb = case
    X, W, b = make_fwd_inputs(900 + M + K, M, N, K, F32, bk)
    Y, Z, path = _fwd(capi, X, W, b, bk, act, alpha=alpha, ta=ta, tb=tb)
    assert path == "small", path
    Y64, Z64 = O.gemm_forward(X, W, b, bk if b is not None else None, act, 0.01, alpha)
    bvals = O.bias_add(np.zeros((M, N)), b, bk) if b is not None else None
    bz = abs(alpha) * fwd_bound(X, W, K, F32, bvals)
    u = U_OUT[F32]
    tag = f"{M}x{N}x{K} act={act} bias={bk} ta={ta} tb={tb}"
    assert_close(Z, Z64, bz + u * np.abs(Z64) + 1e-30, "Z " + tag, rel_norm=1e-4)
    ya = act_lipschitz(act) * bz + u * np.abs(Y64) + 8 * U_ACC * np.abs(Y64) + 2e-7
    assert_close(Y, Y64, ya, "Y " + tag, rel_norm=1e-4)
    if act == "relu":
        pos = Z > 0
        assert np.array_equal(Y[pos], Z[pos]) and np.all(Y[~pos] == 0) and not np.any(np.signbit(Y[~pos]))


def test_small_forward_exact_integers(gpu):
    """Integer inputs, every partial sum exact in fp32: Z and Y equal the oracle's bit for bit,
    whatever order the waves add in."""
    capi = gpu
    g = np.random.default_rng(11)
    M, N, K = 64, 256, 784
    X = g.integers(-2, 3, (M, K)).astype(np.float32)
    W = g.integers(-2, 3, (K, N)).astype(np.float32)
    b = g.integers(-4, 5, N).astype(np.float32)
    Y, Z, path = _fwd(capi, X, W, b, O.BIAS_PERN, "relu")
    assert path == "small"
    Y64, Z64 = O.gemm_forward(X, W, b, O.BIAS_PERN, "relu")
    assert np.array_equal(Z, Z64.astype(np.float32)) and np.array_equal(Y, Y64.astype(np.float32))


def test_small_forward_matches_tile_path(gpu, monkeypatch):
    """Same inputs through the small kernel and through the split-K tile path: within twice
    the fp32 bound of each other, and the small kernel repeats bit for bit."""
    capi = gpu
    M, N, K = 64, 256, 784
    X, W, b = make_fwd_inputs(31, M, N, K, F32, O.BIAS_PERN)
    Y1, Z1, p1 = _fwd(capi, X, W, b, O.BIAS_PERN, "gelu")
    Y2, Z2, _ = _fwd(capi, X, W, b, O.BIAS_PERN, "gelu")
    monkeypatch.setenv("GEV2_NO_SMALL", "1")
    Y3, Z3, p3 = _fwd(capi, X, W, b, O.BIAS_PERN, "gelu")
    assert p1 == "small" and p3 != "small", (p1, p3)
    assert np.array_equal(Z1, Z2) and np.array_equal(Y1, Y2)
    bz = fwd_bound(X, W, K, F32, O.bias_add(np.zeros((M, N)), b, O.BIAS_PERN))
    assert np.all(np.abs(Z1 - Z3) <= 2 * bz + 2 * U_OUT[F32] * np.abs(Z3))


def _bwd(capi, X, W, gY, Z, act, bias_kind, want=("gA", "gB", "gBias"), alpha=1.0, slope=0.01):
    M, K = X.shape
    N = W.shape[1]
    dev = Dev(capi)
    try:
        pX, pW = dev.put(X.astype(np.float32)), dev.put(W.astype(np.float32))
        pgY, pZ = dev.put(gY.astype(np.float32)), dev.put(Z.astype(np.float32))
        pgA = dev.empty(M * K * 4) if "gA" in want else 0
        pgB = dev.empty(K * N * 4) if "gB" in want else 0
        nb = _nbias(bias_kind, M, N)
        pgb = dev.empty(max(nb, 1) * 4) if ("gBias" in want and nb) else 0
        kw = dict(dtype=F32, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, gA=pgA, gB=pgB, gBias=pgb,
                  bias_kind=bias_kind, act=act, leaky_slope=slope, alpha=alpha)
        need = capi.lib().gev2_gemm_bwd_workspace_size(ctypes.byref(capi.bwd_desc(**kw)))
        capi.gemm_bwd(**kw)
        path = capi.last_path()
        capi.synchronize()
        out = {"path": path, "need": need}
        if pgA:
            out["gA"] = dev.get_f32(pgA, (M, K))
        if pgB:
            out["gB"] = dev.get_f32(pgB, (K, N))
        if pgb:
            out["gBias"] = dev.get_f32(pgb, (nb,))
        return out
    finally:
        dev.close()


BWD_CASES = [
    # (M, N, K, act, bias_kind, outputs, alpha)
    (64, 256, 784, "relu", O.BIAS_PERN, ("gA", "gB", "gBias"), 1.0),      # C1
    (64, 256, 784, "gelu", O.BIAS_PERN, ("gA", "gB", "gBias"), 1.0),
    (50, 70, 130, "sigmoid", O.BIAS_PERN, ("gA", "gB", "gBias"), 0.75),   # ragged everywhere
    (33, 600, 45, "tanh", O.BIAS_NONE, ("gA",), 1.0),                      # dX alone, 16 waves
    (130, 200, 64, "leakyrelu", O.BIAS_PERN, ("gB",), 1.0),                # dW alone
    (700, 90, 20, "none", O.BIAS_PERN, ("gA", "gB", "gBias"), 1.0),        # long dW reduction
    (5, 384, 200, "relu", O.BIAS_PERN, ("gBias",), 1.0),                   # dBias alone
    (8, 512, 600, "tanh", O.BIAS_PERN, ("gA", "gB", "gBias"), 1.0),       # rank-8 dW: a tile per wave
    (64, 40, 300, "gelu", O.BIAS_NONE, ("gA", "gB"), 1.0),                 # both reductions short
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: "x".join(map(str, c[:3])) + f"-{c[3]}-" + "+".join(c[5]))
def test_small_backward(gpu, case):
    capi = gpu
    M, N, K, act, bk, want, alpha = case
    seed = 950 + M + N + K
    X, W, _ = make_fwd_inputs(seed, M, N, K, F32, O.BIAS_NONE)
    g = np.random.default_rng(seed + 1)
    gY = g.standard_normal((M, N)).astype(np.float32)
    Z = g.standard_normal((M, N)).astype(np.float32)
    out = _bwd(capi, X, W, gY, Z, act, bk, want, alpha=alpha)
    assert out["path"] == "small" and out["need"] == 0, (out["path"], out["need"])
    ref = O.gemm_backward(X, W, gY, Z, act, 0.01, bk, alpha)
    aG, aY = np.abs(ref["gZ"]), np.abs(gY.astype(np.float64))
    u = U_OUT[F32]
    tag = f"{M}x{N}x{K} act={act}"
    if "gA" in want:
        Wt = np.abs(W.astype(np.float64)).T
        bnd = abs(alpha) * (1.01 * N * U_ACC * (aG @ Wt) + 1e-6 * (aY @ Wt)) + u * np.abs(ref["gA"]) + 1e-30
        assert_close(out["gA"], ref["gA"], bnd, "gA " + tag, rel_norm=1e-4)
    if "gB" in want:
        Xt = np.abs(X.astype(np.float64)).T
        bnd = abs(alpha) * (1.01 * M * U_ACC * (Xt @ aG) + 1e-6 * (Xt @ aY)) + u * np.abs(ref["gB"]) + 1e-30
        assert_close(out["gB"], ref["gB"], bnd, "gB " + tag, rel_norm=1e-4)
    if "gBias" in want and bk == O.BIAS_PERN:
        assert_close(out["gBias"], ref["gBias"], 1.01 * M * U_ACC * aG.sum(0) + 1e-6 * aY.sum(0) + 1e-30,
                     "gBias " + tag)


@pytest.mark.parametrize("act,slope", [("relu", 0.01), ("leakyrelu", 0.5), ("none", 0.01)])
def test_small_backward_exact_integers(gpu, act, slope):
    """Integer inputs and a power-of-two LeakyReLU slope: dY' and every sum are exact in fp32,
    so dX, dW and dBias equal the oracle bit for bit; ReLU masks included."""
    capi = gpu
    g = np.random.default_rng(12)
    M, N, K = 64, 256, 784
    X = g.integers(-2, 3, (M, K)).astype(np.float32)
    W = g.integers(-2, 3, (K, N)).astype(np.float32)
    gY = g.integers(-3, 4, (M, N)).astype(np.float32)
    Z = g.integers(-3, 4, (M, N)).astype(np.float32)
    out = _bwd(capi, X, W, gY, Z, act, O.BIAS_PERN, slope=slope)
    assert out["path"] == "small"
    ref = O.gemm_backward(X, W, gY, Z, act, slope, O.BIAS_PERN)
    for k in ("gA", "gB", "gBias"):
        assert np.array_equal(out[k], ref[k].astype(np.float32)), k


def test_small_backward_matches_multi_launch_path(gpu, monkeypatch):
    """C1's backward through the small kernel and through the multi-launch path: within twice
    the fp32 bound of each other; the small kernel repeats bit for bit."""
    capi = gpu
    M, N, K = 64, 256, 784
    X, W, _ = make_fwd_inputs(41, M, N, K, F32, O.BIAS_NONE)
    g = np.random.default_rng(42)
    gY = g.standard_normal((M, N)).astype(np.float32)
    Z = g.standard_normal((M, N)).astype(np.float32)
    a = _bwd(capi, X, W, gY, Z, "relu", O.BIAS_PERN)
    a2 = _bwd(capi, X, W, gY, Z, "relu", O.BIAS_PERN)
    monkeypatch.setenv("GEV2_NO_SMALL", "1")
    c = _bwd(capi, X, W, gY, Z, "relu", O.BIAS_PERN)
    assert a["path"] == "small" and c["path"] != "small"
    ref = O.gemm_backward(X, W, gY, Z, "relu", 0.01, O.BIAS_PERN)
    aG = np.abs(ref["gZ"])
    bounds = {"gA": 1.01 * N * U_ACC * (aG @ np.abs(W.astype(np.float64)).T),
              "gB": 1.01 * M * U_ACC * (np.abs(X.astype(np.float64)).T @ aG),
              "gBias": 1.01 * M * U_ACC * aG.sum(0)}
    for k, bnd in bounds.items():
        assert np.array_equal(a[k], a2[k]), k
        assert np.all(np.abs(a[k].astype(np.float64) - c[k]) <= 2 * bnd + 2 * U_OUT[F32] * np.abs(ref[k]) + 1e-30), k


def test_small_backward_not_taken_with_gc_or_perm(gpu):
    """gC, or a PerM / Scalar dBias, keep the multi-launch backward."""
    capi = gpu
    M, N, K = 40, 64, 96
    X, W, _ = make_fwd_inputs(51, M, N, K, F32, O.BIAS_NONE)
    g = np.random.default_rng(52)
    gY = g.standard_normal((M, N)).astype(np.float32)
    Z = g.standard_normal((M, N)).astype(np.float32)
    for bk in (O.BIAS_PERM, O.BIAS_SCALAR):
        out = _bwd(capi, X, W, gY, Z, "relu", bk)
        assert out["path"] != "small", bk
        ref = O.gemm_backward(X, W, gY, Z, "relu", 0.01, bk)
        aG = np.abs(ref["gZ"])
        n_terms = N if bk == O.BIAS_PERM else M * N
        s = aG.sum(1) if bk == O.BIAS_PERM else np.array([aG.sum()])
        assert_close(out["gBias"], ref["gBias"], 1.01 * n_terms * U_ACC * s + 1e-30, f"gBias {bk}")
