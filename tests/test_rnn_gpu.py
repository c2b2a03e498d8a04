"""GPU parity of the Elman RNN on the operator (the _ops_rnn module with the reference's
workspace contract, rnn/launcher.cu:129-383) against the float64 oracle: forward Y / Z and
the backward through time (dWx, dWh, dB summed over steps, dh0, dX) for every activation,
batches on the skinny path (N <= 16) and the tile path, exact-integer inputs bit-exact, a
subset of requested gradients, and bf16 tensors."""
import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, F32, rounded

pytestmark = pytest.mark.gpu

ACTS = ["none", "relu", "leakyrelu", "gelu", "sigmoid", "tanh"]


@pytest.fixture(scope="module")
def env(gpu):
    from graph_executor_v2.ops import _ops_rnn as rnn
    from graph_executor_v2.ops.device_array import DeviceArray
    return rnn, DeviceArray


def _act(rnn, name):
    return {"none": rnn.ActKind.__members__["None"], "relu": rnn.ActKind.ReLU, "leakyrelu": rnn.ActKind.LeakyReLU,
            "gelu": rnn.ActKind.GELU, "sigmoid": rnn.ActKind.Sigmoid, "tanh": rnn.ActKind.Tanh}[name]


def _run(env, X, Wx, Wh, h0, b, act, dY=None, dtype=F32, want=("dWx", "dWh", "dB", "dh0", "dX")):
    rnn, DA = env
    dt = "float32" if dtype == F32 else "bfloat16"
    cdt = rnn.DType.F32 if dtype == F32 else rnn.DType.BF16
    N, T, I = X.shape
    H = Wx.shape[1]
    gX, gWx, gWh, gh0 = (DA.from_numpy(a, dt) for a in (X, Wx, Wh, h0))
    gb = DA.from_numpy(b, "float32") if b is not None else None
    Y, Z = DA.empty((N, T, H), dt), DA.empty((N, T, H), dt)
    a = rnn.RnnAttrs()
    a.act, a.with_bias, a.save_z = _act(rnn, act), b is not None, True
    # the reference's forward workspaces (rnn_pybind.cpp:84-87), kept alive for the call
    fws = dict(XH_cat_ptr=DA.empty((N, I + H)), Y_rows_ptr=DA.empty((N, H)), W_cat_ptr=DA.empty((I + H, H)),
               Z_rows_ptr=DA.empty((N, H)))
    rnn.forward(gX.ptr, list(X.shape), gWx.ptr, list(Wx.shape), gWh.ptr, list(Wh.shape), gh0.ptr, list(h0.shape),
                Y.ptr, [N, T, H], bias_ptr=gb.ptr if gb is not None else None, z_ptr=Z.ptr, attrs=a, dtype=cdt,
                **{k: v.ptr for k, v in fws.items()})
    out = {"Y": Y.get(), "Z": Z.get()}
    if dY is not None:
        gdY = DA.from_numpy(dY, dt)
        grads = {"dWx": DA.empty(Wx.shape, dt), "dWh": DA.empty(Wh.shape, dt), "dB": DA.empty((H,), "float32"),
                 "dh0": DA.empty(h0.shape, dt), "dX": DA.empty(X.shape, dt)}
        bws = dict(XH_cat_ptr=DA.empty((N, I + H)), G_rows_ptr=DA.empty((N, H)), Z_rows_ptr=DA.empty((N, H)),
                   W_cat_ptr=DA.empty((I + H, H)), dXH_cat_ptr=DA.empty((N, I + H)),
                   dWcat_ptr=DA.empty((I + H, H)), TmpW_ptr=DA.empty((I + H, H)))
        kw = {k.lower() + "_ptr": (grads[k].ptr if k in want else None) for k in grads}
        rnn.backward(gX.ptr, list(X.shape), gWx.ptr, list(Wx.shape), gWh.ptr, list(Wh.shape), gh0.ptr,
                     list(h0.shape), gdY.ptr, [N, T, H], Z.ptr, [N, T, H], attrs=a, dtype=cdt,
                     **kw, **{k: v.ptr for k, v in bws.items()})
        out.update({k: grads[k].get() for k in want})
    return out


def _inputs(seed, N, T, I, H):
    r = np.random.default_rng(seed)
    return (r.standard_normal((N, T, I)).astype(np.float32),
            (r.standard_normal((I, H)) / np.sqrt(I)).astype(np.float32),
            (0.5 * r.standard_normal((H, H)) / np.sqrt(H)).astype(np.float32),
            r.standard_normal((N, H)).astype(np.float32),
            (0.1 * r.standard_normal(H)).astype(np.float32),
            r.standard_normal((N, T, H)).astype(np.float32))


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("shape", [(4, 6, 24, 32), (40, 5, 48, 64), (3, 1, 16, 32)], ids=["skinny-N4", "tile-N40",
                                                                                     "one-step"])
def test_rnn_f32(env, act, shape):
    N, T, I, H = shape
    X, Wx, Wh, h0, b, dY = _inputs(11, N, T, I, H)
    out = _run(env, X, Wx, Wh, h0, b, act, dY=dY)
    Y64, Z64 = O.rnn_forward(X, Wx, Wh, h0, b, act)
    np.testing.assert_allclose(out["Z"], Z64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(out["Y"], Y64, rtol=1e-4, atol=1e-5)
    # gradients of the device's own forward (the recurrence re-reads Z)
    ref = O.rnn_backward(X, Wx, Wh, h0, dY, out["Z"].astype(np.float64), act)
    for k in ("dWx", "dWh", "dB", "dh0", "dX"):
        np.testing.assert_allclose(out[k], ref[k], rtol=1e-4, atol=1e-4, err_msg=k)


def test_rnn_exact_integers(env):
    """Integer inputs keep every sum exact in fp32: the step order, the h_{t-1} source, the
    dh_next chain and the per-step sums of dW / dB are checked bit-exact."""
    r = np.random.default_rng(12)
    N, T, I, H = 3, 4, 3, 5
    X = r.integers(-2, 3, (N, T, I)).astype(np.float32)
    Wx, Wh = (r.integers(-1, 2, s).astype(np.float32) for s in ((I, H), (H, H)))
    h0 = r.integers(-2, 3, (N, H)).astype(np.float32)
    b = r.integers(-3, 4, H).astype(np.float32)
    dY = r.integers(-2, 3, (N, T, H)).astype(np.float32)
    out = _run(env, X, Wx, Wh, h0, b, "none", dY=dY)
    Y64, Z64 = O.rnn_forward(X, Wx, Wh, h0, b)
    assert np.array_equal(out["Z"], Z64) and np.array_equal(out["Y"], Y64)
    ref = O.rnn_backward(X, Wx, Wh, h0, dY, Z64)
    for k in ("dWx", "dWh", "dB", "dh0", "dX"):
        assert np.array_equal(out[k], ref[k]), k


@pytest.mark.parametrize("form", ["gathered", "per-step"])
def test_rnn_exact_integers_both_backward_forms(env, monkeypatch, form):
    """H = 8 (32-byte fp32 rows) and N*T <= I+H: the backward forms G' into one [N, T, H]
    buffer and computes dWx, dWh (one GEMM of depth N*T each) and dB after the loop;
    GEV2_RNN_STEP_DW=1 keeps one operator backward and one accumulation per step.  Integer
    inputs keep every sum exact, so both forms must equal the oracle bit for bit."""
    if form == "per-step":
        monkeypatch.setenv("GEV2_RNN_STEP_DW", "1")
    r = np.random.default_rng(18)
    N, T, I, H = 3, 4, 8, 8
    X = r.integers(-2, 3, (N, T, I)).astype(np.float32)
    Wx, Wh = (r.integers(-1, 2, s).astype(np.float32) for s in ((I, H), (H, H)))
    h0 = r.integers(-2, 3, (N, H)).astype(np.float32)
    b = r.integers(-3, 4, H).astype(np.float32)
    dY = r.integers(-2, 3, (N, T, H)).astype(np.float32)
    out = _run(env, X, Wx, Wh, h0, b, "relu", dY=dY)
    Y64, Z64 = O.rnn_forward(X, Wx, Wh, h0, b, "relu")
    assert np.array_equal(out["Z"], Z64) and np.array_equal(out["Y"], Y64)
    ref = O.rnn_backward(X, Wx, Wh, h0, dY, Z64, "relu")
    for k in ("dWx", "dWh", "dB", "dh0", "dX"):
        assert np.array_equal(out[k], ref[k]), k


@pytest.mark.parametrize("shape", [(8, 4, 512, 1024), (13, 3, 256, 264)], ids=["N8-H1024", "N13-H264"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_rnn_backward_forms_agree(env, monkeypatch, dtype, shape):
    """The gathered-G' backward against the per-step one on the benchmark's shape class
    (N 8, I 512, H 1024, fewer steps; the step kernel for at most 8 rows) and on 13 rows with
    H = 264 (the 16-row step kernel, a ragged last pass of each dXH column): dh0 and dX are the
    same chain of dXH products (equal up to the per-step form's rounding of G before act'),
    dWx / dWh / dB differ only in summation order and rounding (one rounding of a depth-N*T
    sum against T roundings)."""
    N, T, I, H = shape
    X, Wx, Wh, h0, b, dY = _inputs(19, N, T, I, H)
    if dtype == BF16:
        X, Wx, Wh, h0, dY = (rounded(a, BF16).astype(np.float32) for a in (X, Wx, Wh, h0, dY))
    outs = []
    for form in ("gathered", "per-step"):
        if form == "per-step":
            monkeypatch.setenv("GEV2_RNN_STEP_DW", "1")
        outs.append(_run(env, X, Wx, Wh, h0, b, "tanh", dY=dY, dtype=dtype))
    assert np.array_equal(outs[0]["Z"], outs[1]["Z"])
    ref = O.rnn_backward(X, Wx, Wh, h0, dY, outs[0]["Z"].astype(np.float64), "tanh")
    tol = 1e-4 if dtype == F32 else 0.05
    for k in ("dWx", "dWh", "dB", "dh0", "dX"):
        for o in outs:
            rel = np.abs(o[k].astype(np.float64) - ref[k]).max() / max(1e-6, np.abs(ref[k]).max())
            assert rel <= tol, (k, rel)


def test_rnn_subset_of_gradients(env):
    """Only dWh and dB requested: the others stay untouched, the requested ones are unchanged."""
    N, T, I, H = 5, 3, 8, 16
    X, Wx, Wh, h0, b, dY = _inputs(13, N, T, I, H)
    full = _run(env, X, Wx, Wh, h0, b, "tanh", dY=dY)
    part = _run(env, X, Wx, Wh, h0, b, "tanh", dY=dY, want=("dWh", "dB"))
    assert np.array_equal(full["dWh"], part["dWh"]) and np.array_equal(full["dB"], part["dB"])


def test_rnn_without_bias(env):
    N, T, I, H = 4, 3, 8, 16
    X, Wx, Wh, h0, _, dY = _inputs(14, N, T, I, H)
    out = _run(env, X, Wx, Wh, h0, None, "relu", dY=dY, want=("dWx", "dWh", "dh0", "dX"))
    Y64, _ = O.rnn_forward(X, Wx, Wh, h0, None, "relu")
    np.testing.assert_allclose(out["Y"], Y64, rtol=1e-4, atol=1e-5)
    ref = O.rnn_backward(X, Wx, Wh, h0, dY, out["Z"].astype(np.float64), "relu")
    for k in ("dWx", "dWh", "dh0", "dX"):
        np.testing.assert_allclose(out[k], ref[k], rtol=1e-4, atol=1e-4, err_msg=k)


@pytest.mark.parametrize("shape", [(8, 6, 32, 64), (40, 4, 64, 128)], ids=["skinny-N8", "tile-N40"])
def test_rnn_bf16(env, shape):
    """bf16 tensors (additive): each step rounds h_t and Z_t to bf16, so the comparison is
    against the oracle fed the device's own Z (one step's error, not T steps compounded),
    within a few bf16 roundings of the step's magnitude sums."""
    N, T, I, H = shape
    X, Wx, Wh, h0, b, dY = _inputs(15, N, T, I, H)
    X, Wx, Wh, h0, dY = (rounded(a, BF16).astype(np.float32) for a in (X, Wx, Wh, h0, dY))
    out = _run(env, X, Wx, Wh, h0, b, "tanh", dY=dY, dtype=BF16)
    Z = out["Z"].astype(np.float64)
    eps = 2.0 ** -8
    for t in range(T):
        hprev = h0 if t == 0 else out["Y"][:, t - 1]
        zt = X[:, t] @ Wx + hprev @ Wh + b
        mag = np.abs(X[:, t]) @ np.abs(Wx) + np.abs(hprev) @ np.abs(Wh) + np.abs(b)
        assert np.all(np.abs(Z[:, t] - zt) <= 2 * eps * mag + 1e-6), t
        assert np.all(np.abs(out["Y"][:, t] - np.tanh(Z[:, t])) <= 2 * eps * np.abs(np.tanh(Z[:, t])) + 1e-6), t
    ref = O.rnn_backward(X, Wx, Wh, h0, dY, Z, "tanh")
    for k in ("dWx", "dWh", "dB", "dh0", "dX"):
        rel = np.abs(out[k] - ref[k]).max() / max(1e-6, np.abs(ref[k]).max())
        assert rel <= 0.05, (k, rel)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_rnn_graph_replays(env, dtype):
    """On a created stream with the scratch in the descriptor, the step loops are recorded into
    a HIP graph on the second call and replayed after: every call (eager, recording, replays),
    each with new inputs and eager work between, equals an eager run bit for bit."""
    import ctypes
    from graph_executor_v2.ops import capi
    N, T, I, H = 8, 6, 256, 256
    es = capi.elem_bytes(dtype)
    r = np.random.default_rng(16)
    L = capi.lib()
    bufs = []

    def buf(nbytes):
        b = capi.DeviceBuffer(max(nbytes, 16))
        bufs.append(b)
        return b.ptr

    def put(a):
        b = capi.DeviceBuffer.from_numpy(capi.to_storage(a, dtype))
        bufs.append(b)
        return b

    X0, Wx, Wh, h0, b, dY0 = _inputs(17, N, T, I, H)
    gX, gWx, gWh, gh0, gdY = (put(a) for a in (X0, Wx, Wh, h0, dY0))
    gb = capi.DeviceBuffer.from_numpy(b)
    bufs.append(gb)
    IH = I + H
    ws_bytes = 4 << 20

    def descs():
        Y, Z = buf(N * T * H * es), buf(N * T * H * es)
        ws = buf(ws_bytes)
        fd = capi.RnnDesc(dtype=dtype, act=capi.ACT["tanh"], save_z=1, N=N, T=T, I=I, H=H, X=gX.ptr, Wx=gWx.ptr,
                          Wh=gWh.ptr, bias=gb.ptr, h0=gh0.ptr, Y=Y, Z=Z, xh=buf(N * IH * es), wcat=buf(IH * H * es),
                          ws=ws, ws_bytes=ws_bytes)
        out = {k: buf(n) for k, n in (("dWx", I * H * es), ("dWh", H * H * es), ("dB", H * 4), ("dh0", N * H * es),
                                      ("dX", N * T * I * es))}
        bd = capi.RnnBwdDesc(dtype=dtype, act=capi.ACT["tanh"], N=N, T=T, I=I, H=H, X=gX.ptr, Wx=gWx.ptr, Wh=gWh.ptr,
                             h0=gh0.ptr, dY=gdY.ptr, Z=Z, xh=buf(N * IH * es), g=buf(N * H * es),
                             wcat=buf(IH * H * es), dxh=buf(N * IH * es), dwcat=buf(IH * H * 4),
                             tmpw=buf(IH * H * es), gb=buf(H * 4), ws=ws, ws_bytes=ws_bytes, **out)
        return fd, bd, dict(Y=(Y, (N, T, H)), Z=(Z, (N, T, H)), **{k: (v, None) for k, v in out.items()})

    st = capi.to_storage(np.zeros(1, np.float32), dtype).dtype

    def read(ptrs):
        capi.synchronize()
        shapes = dict(Y=(N, T, H), Z=(N, T, H), dWx=(I, H), dWh=(H, H), dB=(H,), dh0=(N, H), dX=(N, T, I))
        out = {}
        for k, (p, _) in ptrs.items():
            a = np.empty(shapes[k], np.float32 if k == "dB" else st)
            capi.check(L.gev2_memcpy_dtoh(a.ctypes.data, p, a.nbytes), "dtoh")
            out[k] = a
        return out

    stream = capi.Stream()
    gfd, gbd, gptr = descs()          # graph-mode descriptors (created stream)
    efd, ebd, eptr = descs()          # eager reference (null stream)
    try:
        for call in range(4):
            X = r.standard_normal((N, T, I)).astype(np.float32)
            dY = r.standard_normal((N, T, H)).astype(np.float32)
            gX.upload(capi.to_storage(X, dtype))
            gdY.upload(capi.to_storage(dY, dtype))
            capi.check_rnn(L.gev2_rnn_fwd(ctypes.byref(gfd), stream.ptr), "fwd graph")
            capi.check_rnn(L.gev2_rnn_bwd(ctypes.byref(gbd), stream.ptr), "bwd graph")
            stream.synchronize()
            capi.check_rnn(L.gev2_rnn_fwd(ctypes.byref(efd), None), "fwd eager")
            capi.check_rnn(L.gev2_rnn_bwd(ctypes.byref(ebd), None), "bwd eager")
            got, ref = read(gptr), read(eptr)
            for k in got:
                assert np.array_equal(got[k], ref[k]), (call, k)
    finally:
        stream.destroy()


@pytest.mark.parametrize("dtype", [BF16, F32], ids=["bf16", "f32"])
@pytest.mark.parametrize("shape", [(8, 4, 512, 1024), (13, 3, 256, 264), (1, 2, 768, 128)],
                         ids=["N8-I512-H1024", "N13-H264", "N1-K896"])
def test_rnn_fwd_two_part_matches_gather(gpu, monkeypatch, shape, dtype):
    """The forward step reads X_t and h_{t-1} where they lie, with no gather launch: 16-bit
    (N <= 16, I a multiple of 256, operator scratch in the descriptor) through the skinny
    split kernel, fp32 through the one-launch small kernel.  Its Y and Z equal, bit for bit,
    those of the gather + operator path (GEV2_RNN_GATHER=1: the same kernel over the gathered
    rows, same reduction order), and each step is within the storage type's roundings of the
    float64 step fed the device's own h_{t-1}.  Shapes: the benchmark's step; 13 rows and 264
    columns (a ragged column slab / tile); K = 896 (the last 256-row K block half empty)."""
    import ctypes
    from graph_executor_v2.ops import capi
    N, T, I, H = shape
    es = capi.elem_bytes(dtype)
    L = capi.lib()
    X, Wx, Wh, h0, b, _ = _inputs(41, N, T, I, H)
    if dtype == BF16:
        X, Wx, Wh, h0 = (rounded(a, BF16).astype(np.float32) for a in (X, Wx, Wh, h0))
    IH = I + H
    bufs = []

    def buf(nbytes):
        d = capi.DeviceBuffer(max(nbytes, 16))
        bufs.append(d)
        return d.ptr

    def put(a):
        d = capi.DeviceBuffer.from_numpy(capi.to_storage(a, dtype))
        bufs.append(d)
        return d.ptr

    try:
        gX, gWx, gWh, gh0 = (put(a) for a in (X, Wx, Wh, h0))
        gb = capi.DeviceBuffer.from_numpy(b)
        bufs.append(gb)
        st = capi.to_storage(np.zeros(1, np.float32), dtype).dtype
        outs = []
        for gather in ("0", "1"):
            if gather == "1":
                monkeypatch.setenv("GEV2_RNN_GATHER", "1")
            Y, Z = buf(N * T * H * es), buf(N * T * H * es)
            ws_bytes = 4 << 20
            fd = capi.RnnDesc(dtype=dtype, act=capi.ACT["tanh"], save_z=1, N=N, T=T, I=I, H=H, X=gX, Wx=gWx,
                              Wh=gWh, bias=gb.ptr, h0=gh0, Y=Y, Z=Z, xh=buf(N * IH * es), wcat=buf(IH * H * es),
                              ws=buf(ws_bytes), ws_bytes=ws_bytes)
            capi.check_rnn(L.gev2_rnn_fwd(ctypes.byref(fd), None), f"fwd gather={gather}")
            capi.synchronize()
            got = {}
            for k, p in (("Y", Y), ("Z", Z)):
                a = np.empty((N, T, H), st)
                capi.check(L.gev2_memcpy_dtoh(a.ctypes.data, p, a.nbytes), "dtoh")
                got[k] = capi.from_storage(a, dtype).astype(np.float64)
            outs.append(got)
        monkeypatch.delenv("GEV2_RNN_GATHER")
    finally:
        for d in bufs:
            d.free()
    assert np.array_equal(outs[0]["Z"], outs[1]["Z"])
    assert np.array_equal(outs[0]["Y"], outs[1]["Y"])
    Z, Yd = outs[0]["Z"], outs[0]["Y"]
    # bf16: two roundings of the step's magnitude sum; fp32: the accumulation bound over I+H terms
    eps = 2.0 ** -8 if dtype == BF16 else 1.01 * (I + H) * 2.0 ** -24
    for t in range(T):
        hprev = h0 if t == 0 else Yd[:, t - 1]
        zt = X[:, t].astype(np.float64) @ Wx + hprev @ Wh + b
        mag = np.abs(X[:, t]).astype(np.float64) @ np.abs(Wx) + np.abs(hprev) @ np.abs(Wh) + np.abs(b)
        assert np.all(np.abs(Z[:, t] - zt) <= 2 * eps * mag + 1e-6), t
