"""HIP graph capture of the capture-safe Dense paths (forward_into / backward_into, the
reference's graph/graph_exec.py:119-136 recorder with CuPy graphs): the graph is replayed
several times with new inputs, eager work and synchronisations in between, and every replay
must equal the eager result bit for bit (the same kernels on the same data).  The operator
allocates nothing under capture, so no eager warm-up call is needed; a call recorded without
the workspace it would use eagerly takes its scratch-free path, and a later eager call that
grows the library's own buffer cannot affect the graph."""
import numpy as np
import pytest

from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(gpu):
    from graph_executor_v2.graph import capture_stream
    from graph_executor_v2.layers import Dense
    from graph_executor_v2.ops import capi
    from graph_executor_v2.ops.device_array import DeviceArray
    return capture_stream, Dense, capi, DeviceArray


@pytest.mark.parametrize("warmup", [True, False], ids=["warmup", "no-warmup"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("act", ["relu", "gelu"])
def test_dense_step_graph_replays(mods, dtype, act, warmup):
    capture_stream, Dense, capi, DA = mods
    M, K, N = 64, 256, 128
    layer = Dense(N, activation=act, dtype=dtype, seed=31)
    layer.build((M, K))
    stream = capi.Stream()
    g = np.random.default_rng(32)

    def buffers():
        return dict(out=DA.empty((M, N), dtype), z=DA.empty((M, N), dtype), gA=DA.empty((M, K), dtype),
                    gW=DA.empty((K, N), dtype), gB=DA.empty((1, N), "float32"), dz=DA.empty((M, N), "float32"))

    def step(x, gy, b):
        layer.forward_into(x, b["out"], b["z"], stream=stream.ptr)
        layer.backward_into(gy, b["gA"], b["gW"], b["gB"], work_dZ=b["dz"], stream=stream.ptr)

    x, gy = DA.empty((M, K), dtype), DA.empty((M, N), dtype)
    cap_bufs, eager_bufs = buffers(), buffers()
    x.set(g.standard_normal((M, K)).astype(np.float32))
    gy.set(g.standard_normal((M, N)).astype(np.float32))
    if warmup:
        step(x, gy, cap_bufs)                   # eager warm-up on the capture stream
        stream.synchronize()
    # The graph holds the eager call's kernels: the 16-bit paths here need no scratch, and the
    # fp32 layer is small enough for the one-launch kernels, which need none either.
    exact = True
    with capture_stream(stream) as cap:
        step(x, gy, cap_bufs)
    gexec = cap.graph.instantiate()
    try:
        for rep in range(3):
            X = g.standard_normal((M, K)).astype(np.float32)
            GY = g.standard_normal((M, N)).astype(np.float32)
            x.set(X)
            gy.set(GY)
            gexec.launch(stream)
            stream.synchronize()
            got = {k: cap_bufs[k].get() for k in ("out", "z", "gA", "gW", "gB")}
            step(x, gy, eager_bufs)             # eager work between replays
            stream.synchronize()
            for k, v in got.items():
                if exact:
                    np.testing.assert_array_equal(v, eager_bufs[k].get(), err_msg=f"replay {rep}: {k}")
                elif k in ("out", "z"):
                    # recorded without scratch: the plain tile kernel instead of the eager split-K;
                    # both within the fp32 accumulation bound of the exact product
                    absprod = np.abs(X.astype(np.float64)) @ np.abs(layer.W.get().astype(np.float64))
                    bound = 2 * 1.01 * K * 2.0 ** -24 * absprod + 2.0 ** -23 * np.abs(v) + 1e-30
                    assert np.all(np.abs(v - eager_bufs[k].get()) <= bound), f"replay {rep}: {k}"
            if rep == 0 and dtype == "float32":
                W, b = layer.W.get(), layer.b.get()
                Y64, Z64 = O.gemm_forward(X, W, b.reshape(-1), O.BIAS_PERN, act)
                np.testing.assert_allclose(got["out"], Y64, rtol=1e-3, atol=1e-4)
                ref = O.gemm_backward(X, W, GY, Z64, act=act, bias_kind=O.BIAS_PERN)
                np.testing.assert_allclose(got["gW"], ref["gB"], rtol=1e-3, atol=1e-3)
    finally:
        gexec.close()
        stream.destroy()


def test_capture_rejects_null_stream(mods):
    capture_stream, _, _, _ = mods
    with pytest.raises(ValueError):
        with capture_stream(0):
            pass


def _fwd_bwd_descs(capi, dev, dtype, M, N, K, act, seed):
    """Device inputs and descriptors (no workspace in either) of a forward with Z saved and
    the backward that reads that Z."""
    from gemm_helpers import make_fwd_inputs, rounded
    X, W, b = make_fwd_inputs(seed, M, N, K, dtype, O.BIAS_PERN)
    gY = rounded(np.random.default_rng(seed + 1).standard_normal((M, N)), dtype)
    es = capi.elem_bytes(dtype)
    p = dict(X=dev.put(capi.to_storage(X, dtype)), W=dev.put(capi.to_storage(W, dtype)), b=dev.put(b),
             gY=dev.put(capi.to_storage(gY, dtype)), Y=dev.empty(M * N * es), Z=dev.empty(M * N * es),
             gA=dev.empty(M * K * es), gB=dev.empty(K * N * es), gb=dev.empty(N * 4))
    fwd = capi.fwd_desc(dtype=dtype, M=M, N=N, K=K, A=p["X"], B=p["W"], Y=p["Y"], Z=p["Z"], bias=p["b"],
                        bias_kind=O.BIAS_PERN, act=act)
    bwd = capi.bwd_desc(dtype=dtype, M=M, N=N, K=K, A=p["X"], B=p["W"], gY=p["gY"], Z=p["Z"], gA=p["gA"],
                        gB=p["gB"], gBias=p["gb"], bias_kind=O.BIAS_PERN, act=act)
    return (X, W, b, gY), p, fwd, bwd


def test_capture_without_workspace_then_larger_eager_call(mods):
    """Recorded with no workspace and no warm-up: a skinny forward (eagerly split-K with the
    library's per-stream buffer) and a ReLU backward large enough to materialise dY' eagerly
    (M*N*K = 2^30).  The graph holds their scratch-free kernels instead.  Larger eager calls
    on the same stream then grow the per-stream buffer (freeing the old one), and the replays
    must still match the oracle, and each other bit for bit."""
    import ctypes
    from gemm_helpers import BF16, Dev, U_ACC, U_OUT
    capture_stream, _, capi, _ = mods
    L = capi.lib()
    stream = capi.Stream()
    dev = Dev(capi)
    try:
        shapes = {"fwd": (8, 512, 2048), "bwd": (256, 2048, 2048)}
        host, p, fwd, _ = _fwd_bwd_descs(capi, dev, BF16, *shapes["fwd"], "gelu", 71)
        hb, pb, fwd_b, bwd = _fwd_bwd_descs(capi, dev, BF16, *shapes["bwd"], "relu", 73)
        assert capi.fwd_workspace_size(dtype=BF16, M=8, N=512, K=2048, A=p["X"], B=p["W"], Y=p["Y"]) > 0
        assert L.gev2_gemm_bwd_workspace_size(ctypes.byref(bwd)) > 0
        capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd_b), stream.ptr), "eager forward for the backward's Z")
        stream.synchronize()
        with capture_stream(stream) as cap:
            capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd), stream.ptr), "captured fwd")
            capi.check(L.gev2_gemm_bwd(ctypes.byref(bwd), stream.ptr), "captured bwd")
        gexec = cap.graph.instantiate()
        # larger eager calls on the same stream: the per-stream buffer grows
        _, _, fwd2, bwd2 = _fwd_bwd_descs(capi, dev, BF16, 16, 4096, 4096, "gelu", 72)
        capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd2), stream.ptr), "eager fwd")
        capi.check(L.gev2_gemm_bwd(ctypes.byref(bwd2), stream.ptr), "eager bwd")
        stream.synchronize()
        outs = []
        try:
            for _ in range(3):
                for q, keys in ((p, ("Y", "Z")), (pb, ("gA", "gB", "gb"))):
                    for k in keys:
                        next(x for x in dev.bufs if x.ptr == q[k]).fill_bytes(0x7f)
                gexec.launch(stream)
                stream.synchronize()
                capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd2), stream.ptr), "eager fwd between replays")
                stream.synchronize()
                Mb, Nb, Kb = shapes["bwd"]
                outs.append(dict(Y=dev.get(p["Y"], (8, 512), BF16), Z=dev.get(p["Z"], (8, 512), BF16),
                                 gA=dev.get(pb["gA"], (Mb, Kb), BF16), gB=dev.get(pb["gB"], (Kb, Nb), BF16),
                                 gb=dev.get_f32(pb["gb"], (Nb,)), Zb=dev.get(pb["Z"], (Mb, Nb), BF16)))
        finally:
            gexec.close()
    finally:
        dev.close()
        stream.destroy()
    for o in outs[1:]:
        for k in o:
            np.testing.assert_array_equal(o[k], outs[0][k], err_msg=k)
    o = outs[0]
    u = U_OUT[BF16]
    X, W, b, _ = host
    K = shapes["fwd"][2]
    Y64, Z64 = O.gemm_forward(X, W, b, O.BIAS_PERN, "gelu")
    absZ = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64))
    assert np.all(np.abs(o["Z"] - Z64) <= 1.01 * K * U_ACC * absZ + U_ACC * np.abs(b) + u * np.abs(Z64) + 1e-7)
    assert np.all(np.abs(o["Y"] - Y64) <= 1.13 * 1.01 * K * U_ACC * absZ + 2 * u * np.abs(Y64) + 1e-6)
    X, W, _, gY = hb
    M, N, _ = shapes["bwd"]
    ref = O.gemm_backward(X, W, gY, o["Zb"], "relu", bias_kind=O.BIAS_PERN)
    aG = np.abs(ref["gZ"])
    Wt, Xt = np.abs(W.astype(np.float64)).T, np.abs(X.astype(np.float64)).T
    assert np.all(np.abs(o["gA"] - ref["gA"]) <= 1.01 * N * U_ACC * (aG @ Wt) + u * np.abs(ref["gA"]) + 1e-7)
    assert np.all(np.abs(o["gB"] - ref["gB"]) <= 1.01 * M * U_ACC * (Xt @ aG) + u * np.abs(ref["gB"]) + 1e-7)
    assert np.all(np.abs(o["gb"] - ref["gBias"]) <= 1.01 * M * U_ACC * aG.sum(0) + 1e-7)


def test_capture_small_fp32_gelu_without_workspace(mods):
    """A small fp32 GELU forward + backward (C1's shape) recorded with no workspace and no
    warm-up: the one-launch kernels form act' while loading and need no scratch, so nothing is
    refused or allocated, and every replay equals the eager calls bit for bit."""
    import ctypes
    from gemm_helpers import F32, Dev
    capture_stream, _, capi, _ = mods
    L = capi.lib()
    stream = capi.Stream()
    dev = Dev(capi)
    try:
        M, N, K = 64, 256, 784
        _, p, fwd, bwd = _fwd_bwd_descs(capi, dev, F32, M, N, K, "gelu", 75)
        assert capi.fwd_workspace_size(dtype=F32, M=M, N=N, K=K, A=p["X"], B=p["W"], Y=p["Y"]) == 0
        assert L.gev2_gemm_bwd_workspace_size(ctypes.byref(bwd)) == 0
        with capture_stream(stream) as cap:
            capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd), stream.ptr), "captured fwd")
            capi.check(L.gev2_gemm_bwd(ctypes.byref(bwd), stream.ptr), "captured bwd")
        gexec = cap.graph.instantiate()
        keys = (("Y", (M, N)), ("Z", (M, N)), ("gA", (M, K)), ("gB", (K, N)), ("gb", (N,)))
        try:
            replays = []
            for _ in range(3):
                for k, _shape in keys:
                    next(x for x in dev.bufs if x.ptr == p[k]).fill_bytes(0x7f)
                gexec.launch(stream)
                stream.synchronize()
                replays.append({k: dev.get_f32(p[k], shape) for k, shape in keys})
        finally:
            gexec.close()
        capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd), stream.ptr), "eager fwd")
        capi.check(L.gev2_gemm_bwd(ctypes.byref(bwd), stream.ptr), "eager bwd")
        stream.synchronize()
        eager = {k: dev.get_f32(p[k], shape) for k, shape in keys}
    finally:
        dev.close()
        stream.destroy()
    for r in replays:
        for k, _shape in keys:
            np.testing.assert_array_equal(r[k], eager[k], err_msg=k)


def test_capture_refuses_transcendental_backward_without_workspace(mods):
    """Under capture, a GELU backward needs dY' in a workspace: without one the call returns
    MissingInput before recording anything (the capture itself stays valid); with one it is
    recorded and replays equal the eager call bit for bit."""
    import ctypes
    from gemm_helpers import BF16, Dev
    capture_stream, _, capi, _ = mods
    L = capi.lib()
    stream = capi.Stream()
    dev = Dev(capi)
    try:
        M, N, K = 96, 160, 128
        _, p, fwd, bwd = _fwd_bwd_descs(capi, dev, BF16, M, N, K, "gelu", 74)
        capi.check(L.gev2_gemm_fwd(ctypes.byref(fwd), stream.ptr), "eager fwd")
        need = L.gev2_gemm_bwd_workspace_size(ctypes.byref(bwd))
        assert need == M * N * 2
        ws = dev.empty(need)                     # allocated before the capture
        with capture_stream(stream) as cap:
            assert L.gev2_gemm_bwd(ctypes.byref(bwd), stream.ptr) == 10      # MissingInput
            bwd.workspace, bwd.workspace_bytes = ws, need
            capi.check(L.gev2_gemm_bwd(ctypes.byref(bwd), stream.ptr), "captured bwd with workspace")
        gexec = cap.graph.instantiate()
        try:
            gexec.launch(stream)
            stream.synchronize()
            got = [dev.get(p["gA"], (M, K), BF16), dev.get(p["gB"], (K, N), BF16), dev.get_f32(p["gb"], (N,))]
        finally:
            gexec.close()
        capi.check(L.gev2_gemm_bwd(ctypes.byref(bwd), stream.ptr), "eager bwd")
        stream.synchronize()
        eager = [dev.get(p["gA"], (M, K), BF16), dev.get(p["gB"], (K, N), BF16), dev.get_f32(p["gb"], (N,))]
    finally:
        dev.close()
        stream.destroy()
    for a, e in zip(got, eager):
        np.testing.assert_array_equal(a, e)
