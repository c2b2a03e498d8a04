"""HIP graph capture of the capture-safe Dense paths (forward_into / backward_into, the
reference's graph/graph_exec.py:119-136 recorder with CuPy graphs): the graph is replayed
several times with new inputs, eager work and synchronisations in between, and every replay
must equal the eager result bit for bit (the same kernels on the same data)."""
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


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("act", ["relu", "gelu"])
def test_dense_step_graph_replays(mods, dtype, act):
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
    step(x, gy, cap_bufs)                       # eager warm-up on the capture stream
    stream.synchronize()
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
                np.testing.assert_array_equal(v, eager_bufs[k].get(), err_msg=f"replay {rep}: {k}")
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
