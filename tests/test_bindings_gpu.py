"""GPU parity through the Python binding surface (_ops_gemm), the way the
reference's own binding tests drive it (tests/cuda_pyd_test/smoke_gemm_binding.py:
forward_raw/backward_raw with save_z, m=32 k=64 n=16, default_rng(2025)), plus the
Tensor entry points, backward_into and the batched form, each against the
float64 oracle."""
import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, F32, U_ACC, Dev, assert_close, rounded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g(gpu):
    from graph_executor_v2.ops import _ops_gemm
    return _ops_gemm


def _bound_fwd(X, W, K):
    return 1.01 * K * U_ACC * (np.abs(X.astype(float)) @ np.abs(W.astype(float))) + 1e-6


@pytest.mark.parametrize("act", ["relu", "none", "gelu", "sigmoid", "tanh", "leaky_relu"])
def test_raw_smoke_like_reference(gpu, g, act):
    """smoke_gemm_binding.py:130-296: Y, Z, gA, gB, gBias at atol 1e-5 / rtol 1e-4, loosened
    for GELU to atol 5e-4 / rtol 1e-3 as that test does (:273-278): with |Z| up to ~25 the
    derivative's clamped tanh (activations.hpp:55-56) makes 1 - th^2 a cancellation in fp32."""
    capi = gpu
    m, k, n = 32, 64, 16
    rs = np.random.default_rng(2025)
    A = rs.standard_normal((m, k)).astype(np.float32)
    B = rs.standard_normal((k, n)).astype(np.float32)
    bias = rs.standard_normal((1, n)).astype(np.float32)
    gY = rs.standard_normal((m, n)).astype(np.float32)
    dev = Dev(capi)
    try:
        pA, pB, pb, pgY = dev.put(A), dev.put(B), dev.put(bias), dev.put(gY)
        pY, pZ = dev.empty(m * n * 4), dev.empty(m * n * 4)
        pgA, pgB, pgb = dev.empty(m * k * 4), dev.empty(k * n * 4), dev.empty(n * 4)
        g.forward_raw(pA, pB, pb, pY, m, k, n, act=act, with_bias=True, save_z=True, Z_ptr=pZ)
        g.backward_raw(pA, pB, 0, pgY, pZ, pgA, pgB, 0, pgb, m, k, n, act=act, with_bias=True)
        capi.synchronize()
        Y, Z = dev.get_f32(pY, (m, n)), dev.get_f32(pZ, (m, n))
        gA, gB, gb = dev.get_f32(pgA, (m, k)), dev.get_f32(pgB, (k, n)), dev.get_f32(pgb, (n,))
    finally:
        dev.close()
    Y64, Z64 = O.gemm_forward(A, B, bias[0], O.BIAS_PERN, act)
    r = O.gemm_backward(A, B, gY, Z, act, bias_kind=O.BIAS_PERN)
    for name, got, ref in (("Y", Y, Y64), ("Z", Z, Z64), ("gA", gA, r["gA"]), ("gB", gB, r["gB"]),
                           ("gBias", gb, r["gBias"])):
        atol, rtol = (5e-4, 1e-3) if act == "gelu" else (1e-5, 1e-4)
        assert np.allclose(got, ref, atol=atol, rtol=rtol), name


def test_tensor_api_bf16_and_backward_into(gpu, g):
    from graph_executor_v2.ops import _ops_common as c
    capi = gpu
    M, K, N = 96, 128, 80
    rs = np.random.default_rng(7)
    X = rounded(rs.standard_normal((M, K)) / np.sqrt(K), BF16)
    W = rounded(rs.standard_normal((K, N)), BF16)
    b = (0.1 * rs.standard_normal(N)).astype(np.float32)
    gY = rounded(rs.standard_normal((M, N)), BF16)
    dev = Dev(capi)
    dt = c.DType.BF16

    def t(ptr, r, cc, d=dt):
        return c.make_tensor_2d(ptr, [r, cc], d)
    try:
        pX, pW = dev.put(capi.to_storage(X, BF16)), dev.put(capi.to_storage(W, BF16))
        pb, pgY = dev.put(b), dev.put(capi.to_storage(gY, BF16))
        pY, pZ = dev.empty(M * N * 2), dev.empty(M * N * 2)
        pgA, pgB, pgb, pdZ = dev.empty(M * K * 2), dev.empty(K * N * 2), dev.empty(N * 4), dev.empty(M * N * 4)
        attrs = c.GemmAttrs()
        attrs.act = c.ActKind.ReLU
        attrs.with_bias = True
        g.forward(t(pX, M, K), t(pW, K, N), t(pb, 1, N, c.DType.F32), t(pY, M, N), attrs, t(pZ, M, N))
        g.backward_into(t(pX, M, K), t(pW, K, N), None, t(pgY, M, N), t(pZ, M, N), t(pgA, M, K),
                        t(pgB, K, N), None, t(pgb, 1, N, c.DType.F32), attrs, None, dZ_ptr=pdZ)
        capi.synchronize()
        Y, Z = dev.get(pY, (M, N), BF16), dev.get(pZ, (M, N), BF16)
        gA, gB, gb = dev.get(pgA, (M, K), BF16), dev.get(pgB, (K, N), BF16), dev.get_f32(pgb, (N,))
    finally:
        dev.close()
    Y64, Z64 = O.gemm_forward(X, W, b, O.BIAS_PERN, "relu")
    bz = _bound_fwd(X, W, K) + 2.0 ** -8 * np.abs(Z64)
    assert_close(Z, Z64, bz, "Z bf16")
    assert_close(Y, Y64, bz, "Y bf16")
    pos = Z > 0
    assert np.array_equal(Y[pos], Z[pos]) and np.all(Y[~pos] == 0)
    r = O.gemm_backward(X, W, gY, Z, "relu", bias_kind=O.BIAS_PERN)
    for name, got in (("gA", gA), ("gB", gB), ("gBias", gb)):
        ref = r[name]
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 1e-2, (name, rel)


def test_forward_batched_sdpa_exact(gpu, g):
    """QK^T * 1/8 over 8 (b,h) slices through forward_batched; exact-integer inputs."""
    from graph_executor_v2.ops import _ops_common as c
    capi = gpu
    BH, L, D = 8, 64, 32
    rs = np.random.default_rng(12)
    Q = rs.integers(-2, 3, (BH, L, D)).astype(np.float32)
    Kt = rs.integers(-2, 3, (BH, L, D)).astype(np.float32)
    dev = Dev(capi)
    try:
        pQ, pK = dev.put(capi.to_storage(Q, BF16)), dev.put(capi.to_storage(Kt, BF16))
        pS = dev.empty(BH * L * L * 2)
        attrs = c.GemmAttrs()
        attrs.trans_b = True
        attrs.alpha = 0.125
        g.forward_batched(c.make_tensor_2d(pQ, [L, D], c.DType.BF16), c.make_tensor_2d(pK, [L, D], c.DType.BF16),
                          None, c.make_tensor_2d(pS, [L, L], c.DType.BF16), attrs, batch=BH,
                          stride_a=L * D, stride_b=L * D, stride_y=L * L)
        capi.synchronize()
        S = dev.get(pS, (BH, L, L), BF16)
    finally:
        dev.close()
    S64, _ = O.gemm_forward_batched(Q, Kt, BH, L, L, D, L * D, L * D, D, D, trans_b=True, alpha=0.125)
    assert np.array_equal(S, rounded(S64, BF16))
