"""CPU checks of the Python binding surface (graph_executor_v2.ops._ops_common /
_ops_gemm), mirroring the reference's src/bindings/ops_common_pybind.cpp and
gemm_pybind.cpp: names, enum values, defaults, and every validation path that
fails before device work (Status -> exception mapping, binding-level checks).
No GPU is touched: each call below is rejected during validation."""
import ctypes

import pytest


@pytest.fixture(scope="module")
def mods():
    from graph_executor_v2.ops import _ops_common as c
    from graph_executor_v2.ops import _ops_gemm as g
    return c, g


FAKE = 1 << 20   # an address that is never dereferenced (validation fails first)


def T(c, shape, dtype=None, device=None, stride=None):
    t = c.make_tensor_2d(FAKE, list(shape), dtype if dtype is not None else c.DType.F32,
                         device if device is not None else c.Device.CUDA, 0)
    if stride is not None:
        d = t.desc
        d.stride = list(stride)
        t.desc = d
    return t


def test_module_surface(mods):
    c, g = mods
    assert set(c.__all__) == {"ActKind", "GemmAttrs", "Device", "DType", "Layout", "TensorDesc",
                              "Tensor", "make_tensor_2d"}
    ref_fns = {"forward", "backward", "forward_ex", "backward_ex", "backward_into",
               "forward_ex_attrs", "backward_ex_attrs", "forward_raw", "backward_raw"}
    assert ref_fns <= set(g.__all__)
    for n in ref_fns | {"forward_batched", "backward_batched"}:
        assert callable(getattr(g, n))
    assert g.Tensor is c.Tensor and g.GemmAttrs is c.GemmAttrs


def test_enum_values(mods):
    c, _ = mods
    # ABI anchors: enums.hpp:10-24, ai_device.hpp:14-27
    assert [int(c.ActKind.__members__[n]) for n in
            ("None", "ReLU", "LeakyReLU", "GELU", "Sigmoid", "Tanh")] == [0, 1, 2, 3, 4, 5]
    assert int(c.Device.CPU) == 0 and int(c.Device.CUDA) == 1
    assert [int(c.DType.F32), int(c.DType.F16), int(c.DType.BF16), int(c.DType.I32),
            int(c.DType.I8)] == [0, 1, 2, 3, 4]
    assert int(c.Layout.RowMajor) == 0 and int(c.Layout.ColMajor) == 1


def test_attrs_defaults_and_tensor(mods):
    c, _ = mods
    a = c.GemmAttrs()
    assert (a.trans_a, a.trans_b, a.with_bias, a.save_z) == (False, False, False, False)
    assert int(a.act) == 0 and abs(a.leaky_slope - 0.01) < 1e-9 and a.alpha == 1.0
    t = c.make_tensor_2d(1234, [3, 5])
    assert t.data_u64 == 1234 and t.is_cuda() and t.is_contiguous_rowmajor_2d()
    assert list(t.desc.shape) == [3, 5] and list(t.desc.stride) == [5, 1] and t.desc.dim(1) == 5
    assert t.desc.dtype == c.DType.F32 and t.device_index == 0
    t.data_u64 = 99
    assert t.data_u64 == 99
    with pytest.raises(ValueError):
        c.make_tensor_2d(0, [1, 2, 3])


def _fwd(c, g, A, B, Y, bias=None, **kw):
    a = c.GemmAttrs()
    for k, v in kw.items():
        setattr(a, k, v)
    g.forward(A, B, bias, Y, a)


def _status_msg(excinfo):
    return str(excinfo.value)


def test_forward_status_paths(mods):
    c, g = mods
    A, B, Y = T(c, (4, 8)), T(c, (8, 6)), T(c, (4, 6))
    # DeviceMismatch: a CPU tensor, an integer dtype, mixed dtypes (gemm/launcher.cu:158-159)
    for bad in (T(c, (4, 8), device=c.Device.CPU), T(c, (4, 8), dtype=c.DType.I32),
                T(c, (4, 8), dtype=c.DType.BF16)):
        with pytest.raises(RuntimeError, match=r"\[_ops_gemm::forward\] DeviceMismatch"):
            _fwd(c, g, bad, B, Y)
    with pytest.raises(RuntimeError, match="TransposeNotSupported"):
        _fwd(c, g, A, B, Y, trans_b=True)
    with pytest.raises(RuntimeError, match="ShapeMismatch"):
        _fwd(c, g, A, T(c, (7, 6)), Y)
    with pytest.raises(RuntimeError, match="ShapeMismatch"):
        _fwd(c, g, A, B, T(c, (4, 5)))
    with pytest.raises(RuntimeError, match="StrideMismatch"):
        _fwd(c, g, T(c, (4, 8), stride=(7, 1)), B, Y)
    with pytest.raises(RuntimeError, match="Invalid"):
        _fwd(c, g, T(c, (4, 1 << 31)), T(c, (1 << 31, 6)), Y)
    # bias must be F32 (validate_bias_buffer, gemm/launcher.cu:80-81)
    with pytest.raises(RuntimeError, match="Invalid"):
        _fwd(c, g, A, B, Y, bias=T(c, (1, 6), dtype=c.DType.F16))
    # binding-level: save_z without Z (gemm_pybind.cpp:143-146)
    with pytest.raises(ValueError, match="save_z"):
        _fwd(c, g, A, B, Y, save_z=True)
    # Z must match Y
    with pytest.raises(RuntimeError, match="ShapeMismatch"):
        g.forward(A, B, None, Y, c.GemmAttrs(), T(c, (4, 5)))


def test_forward_ex_and_raw_checks(mods):
    c, g = mods
    A, B, Y = T(c, (4, 8)), T(c, (8, 6)), T(c, (4, 6))
    with pytest.raises(ValueError, match="with_bias=True but bias is None"):
        g.forward_ex(A, B, None, Y, with_bias=True)
    with pytest.raises(ValueError, match="unknown act"):
        g.forward_ex(A, B, None, Y, act="swish")
    with pytest.raises(ValueError, match="Bias_ptr==0"):
        g.forward_raw(FAKE, FAKE, 0, FAKE, 4, 8, 6, with_bias=True)
    with pytest.raises(ValueError, match="Z_ptr==0"):
        g.forward_raw(FAKE, FAKE, 0, FAKE, 4, 8, 6, save_z=True)
    with pytest.raises(RuntimeError, match="forward_raw.*TransposeNotSupported"):
        g.forward_raw(FAKE, FAKE, 0, FAKE, 4, 8, 6, trans_a=True)
    # empty problems are a no-op (no device work)
    g.forward_raw(FAKE, FAKE, 0, FAKE, 0, 8, 6)
    # case-insensitive activation names (gemm_pybind.cpp:57-69)
    for name in ("ReLU", "LEAKY_RELU", "lrelu", "Gelu", "SIGMOID", "tanh", "None"):
        g.forward_raw(FAKE, FAKE, 0, FAKE, 0, 8, 6, act=name)


def test_backward_status_paths(mods):
    c, g = mods
    M, K, N = 4, 8, 6
    A, B, gY, Z = T(c, (M, K)), T(c, (K, N)), T(c, (M, N)), T(c, (M, N))
    attrs = c.GemmAttrs()
    # gBias shaped like a PerM reduction is refused for Dense (gemm_pybind.cpp:190-203)
    for sh in ((M,), (M, 1)):
        gb = c.make_tensor_2d(FAKE, [1, N])
        d = gb.desc
        d.shape = list(sh)
        gb.desc = d
        with pytest.raises(ValueError, match="PerN"):
            g.backward(A, B, None, gY, Z, None, None, None, gb, attrs)
    with pytest.raises(RuntimeError, match="MissingInput"):
        g.backward(A, B, None, gY, Z, gC=T(c, (M, N)), attrs=attrs)
    with pytest.raises(RuntimeError, match="ShapeMismatch"):
        g.backward(A, B, None, gY, Z, gA=T(c, (M, N)), attrs=attrs)
    with pytest.raises(RuntimeError, match="StrideMismatch"):
        g.backward(A, B, None, T(c, (M, N), stride=(3, 1)), Z, attrs=attrs)
    with pytest.raises(RuntimeError, match="TransposeNotSupported"):
        g.backward_ex(A, B, None, gY, Z, trans_a=True)
    # empty reduction: the reference's backward throws invalid_argument("invalid dims")
    with pytest.raises(ValueError, match="InvalidArgument"):
        g.backward(T(c, (M, 0)), T(c, (0, N)), None, gY, Z, attrs=attrs)
    # capture-safe variant argument rules (gemm_pybind.cpp:403-411)
    with pytest.raises(ValueError, match="dZ_ptr is required"):
        g.backward_into(A, B, None, gY, Z, attrs=attrs, dZ_ptr=0)
    with pytest.raises(ValueError, match="both zero or both non-zero"):
        g.backward_into(A, B, None, gY, Z, attrs=attrs, dZ_ptr=FAKE, lt_ws_ptr=FAKE)
    # lt workspace must be 256-byte aligned (gemm/launcher.cu:87-91)
    with pytest.raises(RuntimeError, match="Invalid"):
        g.backward_into(A, B, None, gY, Z, attrs=attrs, dZ_ptr=FAKE, lt_ws_ptr=FAKE + 4, lt_ws_bytes=64)


def test_batched_checks(mods):
    c, g = mods
    a = c.GemmAttrs()
    a.trans_b = True
    Q, Kt, S = T(c, (16, 8)), T(c, (12, 8)), T(c, (16, 12))
    with pytest.raises(RuntimeError, match="forward_batched.*ShapeMismatch"):
        g.forward_batched(Q, T(c, (12, 7)), None, S, a, batch=2, stride_a=128, stride_b=96, stride_y=192)
    with pytest.raises(RuntimeError, match="Invalid"):
        g.forward_batched(Q, Kt, None, S, a, batch=0, stride_a=128, stride_b=96, stride_y=192)


def test_stream_argument_forms(mods):
    c, g = mods
    # None, an int and a PyCapsule are accepted; anything else is a TypeError
    mk = ctypes.pythonapi.PyCapsule_New
    mk.restype = ctypes.py_object
    mk.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
    cap = mk(ctypes.c_void_p(0x10), None, None)
    for s in (None, 0, cap):
        g.forward_raw(FAKE, FAKE, 0, FAKE, 0, 8, 6, stream=s)
    with pytest.raises(TypeError):
        g.forward_raw(FAKE, FAKE, 0, FAKE, 0, 8, 6, stream="default")
