"""GPU tests of the Python glue (ops/gemm.py) and the Dense layer, through the native
modules on the device, against the float64 oracle.  They follow the reference's own
glue / layer tests (tests/cuda_pyd_test/glue_gemm.py, tests/layer_test/dense_gemm.py):
allocating and capture-safe forward/backward, the bias-shape and Z policies, and the
Dense layer at BASELINE config 1 (X[64,784] W[784,256] + b, ReLU)."""
import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, U_ACC, rounded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(gpu):
    from graph_executor_v2.ops import gemm
    from graph_executor_v2.ops.device_array import DeviceArray
    from graph_executor_v2.layers import Dense
    return gemm, DeviceArray, Dense


def _close(dev, ref, rtol=1e-4, atol=1e-5, what=""):
    np.testing.assert_allclose(np.asarray(dev, np.float64), np.asarray(ref, np.float64), rtol=rtol, atol=atol,
                               err_msg=what)


def _inputs(M=32, K=64, N=16, seed=2025):
    g = np.random.default_rng(seed)       # the reference tests' rng(2025) normal inputs
    return (g.standard_normal((M, K)).astype(np.float32), g.standard_normal((K, N)).astype(np.float32),
            g.standard_normal((1, N)).astype(np.float32), g.standard_normal((M, N)).astype(np.float32))


@pytest.mark.parametrize("act", ["none", "relu", "leakyrelu", "gelu", "sigmoid", "tanh"])
def test_forward_backward_allocating(mods, act):
    gemm, DA, _ = mods
    A, B, bias, gY = _inputs()
    dA, dB, db, dgY = (DA.from_numpy(x) for x in (A, B, bias, gY))
    Y, Z = gemm.forward(dA, dB, db, act=act, save_z=True, return_z=True)
    Y64, Z64 = O.gemm_forward(A, B, bias.reshape(-1), O.BIAS_PERN, act)
    tol = dict(rtol=1e-3, atol=5e-4) if act == "gelu" else {}
    _close(Z.get(), Z64, what="Z", **tol)
    _close(Y.get(), Y64, what="Y", **tol)
    if act == "none":
        assert Z is Y                               # Z aliases Y when act == none (gemm.py:158-172)
    outs = gemm.backward(dA, dB, dgY, Z, act=act, with_bias=True, want_gBias=True)
    assert set(outs) == {"gA", "gB", "gBias"}
    ref = O.gemm_backward(A, B, gY, Z.get().astype(np.float64), act=act, bias_kind=O.BIAS_PERN)
    _close(outs["gA"].get(), ref["gA"], rtol=1e-3, atol=1e-3, what="gA")
    _close(outs["gB"].get(), ref["gB"], rtol=1e-3, atol=1e-3, what="gB")
    _close(outs["gBias"].get().reshape(-1), ref["gBias"], rtol=1e-3, atol=1e-3, what="gBias")


def test_bias_forms(mods):
    """Scalar, (N,), (1,N), (M,1) and (M,N) biases (gemm.py:124-150); the operator's
    bias-kind rule drops an (M,N) bias (launcher.cu:47-77), exactly as in the reference."""
    gemm, DA, _ = mods
    A, B, bias, _ = _inputs(M=24, K=40, N=20, seed=7)
    dA, dB = DA.from_numpy(A), DA.from_numpy(B)
    plain = A.astype(np.float64) @ B
    y = gemm.forward(dA, dB, 0.75).get()
    _close(y, plain + 0.75, what="scalar")
    y = gemm.forward(dA, dB, DA.from_numpy(bias.reshape(-1))).get()
    _close(y, plain + bias, what="(N,)")
    y = gemm.forward(dA, dB, DA.from_numpy(bias)).get()
    _close(y, plain + bias, what="(1,N)")
    col = np.arange(24, dtype=np.float32).reshape(24, 1) / 8
    y = gemm.forward(dA, dB, DA.from_numpy(col)).get()
    _close(y, plain + col, what="(M,1)")
    y = gemm.forward(dA, dB, DA.from_numpy(np.ones((24, 20), np.float32))).get()
    _close(y, plain, what="(M,N) dropped")


def test_backward_output_selection(mods):
    gemm, DA, _ = mods
    A, B, bias, gY = _inputs(seed=3)
    dA, dB, dgY = DA.from_numpy(A), DA.from_numpy(B), DA.from_numpy(gY)
    _, Z = gemm.forward(dA, dB, DA.from_numpy(bias), act="relu", save_z=True, return_z=True)
    outs = gemm.backward(dA, dB, dgY, Z, act="relu", want_gA=False, want_gB=True)
    assert set(outs) == {"gB"}
    C = DA.from_numpy(np.zeros((32, 16), np.float32))
    outs = gemm.backward(dA, dB, dgY, Z, act="relu", C=C, want_gA=True, want_gB=False)
    assert set(outs) == {"gA", "gC"}
    ref = O.gemm_backward(A, B, gY, Z.get().astype(np.float64), act="relu", beta=1.0)
    _close(outs["gC"].get(), ref["gC"], what="gC")


def test_capture_safe_paths(mods):
    """forward_into / backward_into with every buffer preallocated (gemm.py:317-509)."""
    gemm, DA, _ = mods
    A, B, bias, gY = _inputs(M=48, K=96, N=32, seed=11)
    dA, dB, db, dgY = (DA.from_numpy(x) for x in (A, B, bias, gY))
    out, z = DA.empty((48, 32)), DA.empty((48, 32))
    gemm.forward_into(dA, dB, out=out, bias=db, act="leakyrelu", with_bias=True, leaky_slope=0.2, save_z=True,
                      z_out=z)
    Y64, Z64 = O.gemm_forward(A, B, bias.reshape(-1), O.BIAS_PERN, "leakyrelu", 0.2)
    _close(out.get(), Y64, what="Y")
    _close(z.get(), Z64, what="Z")
    ws = gemm.ensure_workspaces(48, 32)
    assert gemm.ensure_workspaces(48, 32) is ws
    gA, gB, gb = DA.empty((48, 96)), DA.empty((96, 32)), DA.empty((1, 32))
    gemm.backward_into(dA, dB, dgY, z, act="leakyrelu", with_bias=True, leaky_slope=0.2, gA_out=gA, gB_out=gB,
                       gBias_out=gb, work_dZ=ws.dZ)
    ref = O.gemm_backward(A, B, gY, Z64, act="leakyrelu", slope=0.2, bias_kind=O.BIAS_PERN)
    _close(gA.get(), ref["gA"], rtol=1e-3, atol=1e-3, what="gA")
    _close(gB.get(), ref["gB"], rtol=1e-3, atol=1e-3, what="gB")
    _close(gb.get().reshape(-1), ref["gBias"], rtol=1e-3, atol=1e-3, what="gBias")
    gemm.clear_ws_cache()


def test_dense_config1(mods):
    """Dense at BASELINE config 1: X[64,784] ~ U(-1,1)/sqrt(784), 256 units, ReLU; forward,
    native backward (dX, dW, dBias) against the oracle on the layer's own weights."""
    _, DA, Dense = mods
    g = np.random.default_rng(1)
    X = (g.uniform(-1, 1, (64, 784)) / np.sqrt(784)).astype(np.float32)
    dY = g.standard_normal((64, 256)).astype(np.float32)
    layer = Dense(256, activation="relu", use_native_bwd=True, seed=5)
    dX = DA.from_numpy(X)
    Y = layer(dX)
    assert layer.built and layer.output_shape == (None, 256)
    W, b = layer.W.get(), layer.b.get()
    Y64, Z64 = O.gemm_forward(X, W, b.reshape(-1), O.BIAS_PERN, "relu")
    _close(Y.get(), Y64, what="Y")
    _close(layer.last_linear.get(), Z64, what="Z")
    dx = layer.backward(DA.from_numpy(dY))
    ref = O.gemm_backward(X, W, dY, layer.last_linear.get().astype(np.float64), act="relu",
                          bias_kind=O.BIAS_PERN)
    _close(dx.get(), ref["gA"], what="dX")
    _close(layer.dW.get(), ref["gB"], what="dW")
    _close(layer.db.get().reshape(-1), ref["gBias"], what="db")
    assert [t for (_p, _g, t) in layer.parameters()] == ["Dense.W", "Dense.b"]
    layer.zero_grad()
    assert not layer.dW.get().any() and not layer.db.get().any()


def test_dense_eval_and_manual_mode(mods):
    """Inference mode keeps no Z; the backward then recomputes it (dense_gemm.py:218-228).
    The manual-mode flag gives the same gradients as the native one in this build."""
    _, DA, Dense = mods
    g = np.random.default_rng(9)
    X = g.standard_normal((16, 24)).astype(np.float32)
    dY = g.standard_normal((16, 8)).astype(np.float32)
    grads = []
    for native in (False, True):
        layer = Dense(8, activation="tanh", use_native_bwd=native, initializer="xavier", seed=3)
        layer.build((16, 24))
        layer.eval()
        layer(DA.from_numpy(X))
        assert layer.last_linear is None
        dx = layer.backward(DA.from_numpy(dY))
        grads.append((dx.get(), layer.dW.get(), layer.db.get()))
    for a, b in zip(*grads):
        np.testing.assert_array_equal(a, b)


def test_dense_capture_hooks(mods):
    _, DA, Dense = mods
    g = np.random.default_rng(4)
    X = g.standard_normal((32, 48)).astype(np.float32)
    dY = g.standard_normal((32, 16)).astype(np.float32)
    layer = Dense(16, activation="sigmoid", seed=8)
    layer.build((32, 48))
    work = {}
    out = DA.empty((32, 16))
    dX = DA.from_numpy(X)
    layer.forward_into(dX, out, work=work)
    W, b = layer.W.get(), layer.b.get()
    Y64, Z64 = O.gemm_forward(X, W, b.reshape(-1), O.BIAS_PERN, "sigmoid")
    _close(out.get(), Y64, rtol=1e-3, atol=1e-5, what="Y")
    gA, gW, gB = DA.empty((32, 48)), DA.empty((48, 16)), DA.empty((1, 16))
    layer.backward_into(DA.from_numpy(dY), gA, gW, gB, work_dZ=None, work=work)
    ref = O.gemm_backward(X, W, dY, Z64, act="sigmoid", bias_kind=O.BIAS_PERN)
    _close(gA.get(), ref["gA"], rtol=1e-3, atol=1e-4, what="dX")
    _close(gW.get(), ref["gB"], rtol=1e-3, atol=1e-4, what="dW")
    assert layer.dW is gW and layer.db is gB


def test_dense_bf16(mods):
    """bf16 weights and activations (additive): forward within one bf16 rounding of the
    fp32-accumulated result, gradients within the 4*K*eps bound of the contract."""
    _, DA, Dense = mods
    g = np.random.default_rng(12)
    M, K, N = 64, 256, 128
    X = rounded(g.standard_normal((M, K)) / np.sqrt(K), BF16).astype(np.float32)
    dY = rounded(g.standard_normal((M, N)), BF16).astype(np.float32)
    layer = Dense(N, activation="relu", dtype="bfloat16", seed=2)
    Y = layer(DA.from_numpy(X, "bfloat16"))
    W, b = layer.W.get(), layer.b.get()
    Y64, Z64 = O.gemm_forward(X, W, b.reshape(-1), O.BIAS_PERN, "relu")
    bound = 1.01 * K * U_ACC * (np.abs(X) @ np.abs(W)) + 2.0 ** -8 * np.abs(Y64) + 1e-6
    assert np.all(np.abs(Y.get() - Y64) <= bound)
    dx = layer.backward(DA.from_numpy(dY, "bfloat16"))
    ref = O.gemm_backward(X, W, dY, layer.last_linear.get().astype(np.float64), act="relu",
                          bias_kind=O.BIAS_PERN)
    eps = 2.0 ** -7
    gA_bound = 4 * N * eps * (np.abs(dY) @ np.abs(W).T) + 1e-6
    assert np.all(np.abs(dx.get() - ref["gA"]) <= gA_bound)
    gB_bound = 4 * M * eps * (np.abs(X).T @ np.abs(dY)) + 1e-6
    assert np.all(np.abs(layer.dW.get() - ref["gB"]) <= gB_bound)
    _close(layer.db.get().reshape(-1), ref["gBias"], rtol=1e-5, atol=1e-4, what="db")
