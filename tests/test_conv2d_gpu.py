"""GPU parity of conv2d on the operator (the _ops_conv2d module with the reference's
workspace contract, conv2d/launcher.cu:106-459) against the float64 direct-sum oracle:
forward with bias, activation and Z over stride / padding / dilation variants, the
multi-image launch (dCol_bytes), exact-integer inputs for bit-exact index handling, and
the backward's dW, dB (summed over every image) and dX."""
import numpy as np
import pytest

from oracle import gemm_oracle as O
from conv_helpers import GEOMS, WINDOW_GEOMS, _inputs, _run
from gemm_helpers import BF16, F32, rounded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env(gpu):
    from graph_executor_v2.ops import _ops_conv2d as conv
    from graph_executor_v2.ops.device_array import DeviceArray
    return conv, DeviceArray


@pytest.mark.parametrize("geom", list(GEOMS))
@pytest.mark.parametrize("all_images", [False, True], ids=["per-image", "one-launch"])
def test_conv2d_forward_f32(env, geom, all_images):
    g = GEOMS[geom]
    X, W, b = _inputs(g, 1)
    out = _run(env, g, X, W, b, "relu", all_images=all_images)
    Y64, Z64 = O.conv2d_forward(X, W, b, g["stride"], g["pad"], g["dil"], act="relu")
    np.testing.assert_allclose(out["Z"], Z64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(out["Y"], Y64, rtol=1e-4, atol=1e-5)
    pos = out["Z"] > 0
    assert np.array_equal(out["Y"][pos], out["Z"][pos]) and np.all(out["Y"][~pos] == 0)


@pytest.mark.parametrize("width", [1000, 999], ids=["aligned", "odd"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_conv2d_wide_planes(env, width, dtype):
    """Planes too wide for one LDS band of im2col (the band is split into row groups), with
    16-byte-aligned rows and with an odd width (element stores); exact-integer inputs, bit-exact."""
    g = dict(N=2, Cin=2, H=40, W=width, Cout=4, Kh=3, Kw=3, stride=(1, 1), pad=(1, 1), dil=(1, 1))
    X, W, b = _inputs(g, 8, integers=True)
    out = _run(env, g, X, W, b, "none", dtype=dtype, all_images=True)
    Y64, Z64 = O.conv2d_forward(X, W, b, g["stride"], g["pad"], g["dil"])
    assert np.array_equal(out["Z"], Z64) and np.array_equal(out["Y"], Y64)


@pytest.mark.parametrize("geom", list(GEOMS))
@pytest.mark.parametrize("bwd_images", [1, 2, 3])
def test_conv2d_exact_integers(env, geom, bwd_images):
    """Integer inputs make every sum exact: index, padding and stride handling bit-exact,
    for one image per backward call, for chunks that divide N, and for a ragged last chunk."""
    g = GEOMS[geom]
    X, W, b = _inputs(g, 2, integers=True)
    dY = np.random.default_rng(3).integers(-2, 3, (g["N"], g["Cout"]) + O.conv2d_out_size(
        g["H"], g["W"], g["Kh"], g["Kw"], g["stride"], g["pad"], g["dil"])).astype(np.float32)
    out = _run(env, g, X, W, b, "none", all_images=True, dY=dY, bwd_images=bwd_images)
    Y64, Z64 = O.conv2d_forward(X, W, b, g["stride"], g["pad"], g["dil"])
    assert np.array_equal(out["Z"], Z64) and np.array_equal(out["Y"], Y64)
    ref = O.conv2d_backward(X, W, dY, Z64, g["stride"], g["pad"], g["dil"])
    for k in ("dX", "dW", "dB"):                    # dB: summed over every image
        d = np.abs(out[k] - ref[k])
        assert np.array_equal(out[k], ref[k]), (k, int((d > 0).sum()), float(d.max()),
                                                np.unravel_index(int(np.argmax(d)), d.shape))


@pytest.mark.parametrize("geom", WINDOW_GEOMS)
def test_conv2d_exact_integers_bf16(env, geom):
    """bf16 with entries in {-1, 0, 1}: every sum (at most 120 terms) is an integer that bf16
    holds exactly, so the shifted-window reads of im2col and col2im are checked bit-exact for
    16-bit elements at odd and even element offsets."""
    g = GEOMS[geom]
    r = np.random.default_rng(11)
    X = r.integers(-1, 2, (g["N"], g["Cin"], g["H"], g["W"])).astype(np.float32)
    W = r.integers(-1, 2, (g["Cout"], g["Cin"], g["Kh"], g["Kw"])).astype(np.float32)
    b = r.integers(-4, 5, g["Cout"]).astype(np.float32)
    Ho, Wo = O.conv2d_out_size(g["H"], g["W"], g["Kh"], g["Kw"], g["stride"], g["pad"], g["dil"])
    dY = r.integers(-1, 2, (g["N"], g["Cout"], Ho, Wo)).astype(np.float32)
    out = _run(env, g, X, W, b, "none", dtype=BF16, all_images=True, dY=dY, bwd_images=2)
    Y64, Z64 = O.conv2d_forward(X, W, b, g["stride"], g["pad"], g["dil"])
    assert np.array_equal(out["Z"], Z64) and np.array_equal(out["Y"], Y64)
    ref = O.conv2d_backward(X, W, dY, Z64, g["stride"], g["pad"], g["dil"])
    for k in ("dX", "dW", "dB"):
        assert np.array_equal(out[k], ref[k]), k


@pytest.mark.parametrize("act", ["relu", "tanh", "leakyrelu"])
@pytest.mark.parametrize("bwd_images", [1, 3])
def test_conv2d_backward_f32(env, act, bwd_images):
    g = GEOMS["c5a-like"]
    X, W, b = _inputs(g, 4)
    Ho, Wo = O.conv2d_out_size(g["H"], g["W"], g["Kh"], g["Kw"], g["stride"], g["pad"], g["dil"])
    dY = np.random.default_rng(5).standard_normal((g["N"], g["Cout"], Ho, Wo)).astype(np.float32)
    out = _run(env, g, X, W, b, act, dY=dY, bwd_images=bwd_images)
    ref = O.conv2d_backward(X, W, dY, out["Z"].astype(np.float64), g["stride"], g["pad"], g["dil"], act=act)
    np.testing.assert_allclose(out["dX"], ref["dX"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(out["dW"], ref["dW"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(out["dB"], ref["dB"], rtol=1e-4, atol=1e-4)


def test_conv2d_bf16(env):
    """bf16 tensors (additive): forward within one bf16 rounding of the fp32-accumulated
    sum; gradients within 4*K*eps of their magnitude sums."""
    g = GEOMS["c5a-like"]
    X, W, b = _inputs(g, 6)
    X, W = rounded(X, BF16).astype(np.float32), rounded(W, BF16).astype(np.float32)
    Ho, Wo = O.conv2d_out_size(g["H"], g["W"], g["Kh"], g["Kw"], g["stride"], g["pad"], g["dil"])
    dY = rounded(np.random.default_rng(7).standard_normal((g["N"], g["Cout"], Ho, Wo)), BF16).astype(np.float32)
    out = _run(env, g, X, W, b, "relu", dtype=BF16, dY=dY, bwd_images=3)
    Y64, Z64 = O.conv2d_forward(X, W, b, g["stride"], g["pad"], g["dil"], act="relu")
    absZ, _ = O.conv2d_forward(np.abs(X), np.abs(W), np.abs(b), g["stride"], g["pad"], g["dil"])
    K = g["Cin"] * g["Kh"] * g["Kw"]
    assert np.all(np.abs(out["Z"] - Z64) <= 2.0 ** -8 * np.abs(Z64) + 1.01 * K * 2.0 ** -24 * absZ + 1e-7)
    ref = O.conv2d_backward(X, W, dY, out["Z"].astype(np.float64), g["stride"], g["pad"], g["dil"], act="relu")
    aref = O.conv2d_backward(np.abs(X), np.abs(W), np.abs(dY), np.ones_like(Z64), g["stride"], g["pad"], g["dil"])
    eps = 2.0 ** -7
    n_dx, n_dw = g["Cout"] * g["Kh"] * g["Kw"], g["N"] * Ho * Wo
    assert np.all(np.abs(out["dX"] - ref["dX"]) <= 4 * n_dx * eps * aref["dX"] + 1e-6)
    assert np.all(np.abs(out["dW"] - ref["dW"]) <= 4 * n_dw * eps * aref["dW"] + 1e-6)
    assert np.all(np.abs(out["dB"] - ref["dB"]) <= 1e-3 * aref["dB"] + 1e-5)
