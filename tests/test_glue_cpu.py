"""CPU checks of the Python glue (ops/gemm.py, ops/common.py) and the Dense layer: every
policy that rejects a call does so before any device work (reference policies:
python/graph_executor_v2/ops/gemm.py:99-509, layers/dense_gemm.py:112-196).  The
arrays here are stand-ins that only describe device memory; none is dereferenced."""
import numpy as np
import pytest


class FakeDev:
    """Describes a device array through __cuda_array_interface__ (never dereferenced)."""

    def __init__(self, shape, typestr="<f4", ptr=0x10000, strides=None):
        self.shape = tuple(shape)
        self.__cuda_array_interface__ = {"shape": self.shape, "typestr": typestr, "data": (ptr, False),
                                         "strides": strides, "version": 3}


@pytest.fixture(scope="module")
def ops():
    from graph_executor_v2.ops import gemm, common
    return gemm, common


def test_array_info_and_contiguity(ops):
    _, common = ops
    a = FakeDev((3, 5))
    assert common.array_info(a) == (0x10000, (3, 5), "float32", True)
    assert common.array_info(FakeDev((3, 5), "<f2"))[2] == "float16"
    assert common.is_c_contiguous(FakeDev((3, 5), strides=(20, 4)))
    assert not common.is_c_contiguous(FakeDev((3, 5), strides=(4, 12)))   # column-major
    with pytest.raises(TypeError):
        common.array_info(np.zeros((2, 2), np.float32))                   # host array
    with pytest.raises(TypeError):
        common.assert_2d(FakeDev((3, 5), "<i4"), "A")                      # dtype (reference: float32 only)
    with pytest.raises(ValueError):
        common.assert_2d(FakeDev((3, 5, 2)), "A")
    with pytest.raises(TypeError):
        common.assert_f32_2d(FakeDev((3, 5), "<f2"), "A")


def test_act_parser(ops):
    gemm, _ = ops
    g = gemm.g
    assert gemm._parse_act_to_kind("Leaky_ReLU") == g.ActKind.LeakyReLU
    assert gemm._parse_act_to_kind("lrelu") == g.ActKind.LeakyReLU
    assert gemm._parse_act_to_kind(None) == getattr(g.ActKind, "None")
    assert gemm._parse_act_to_kind("GELU") == g.ActKind.GELU
    with pytest.raises(ValueError):
        gemm._parse_act_to_kind("swish")


def test_forward_rejections(ops):
    gemm, _ = ops
    A, B = FakeDev((4, 8)), FakeDev((8, 6))
    with pytest.raises(ValueError, match="K mismatch"):
        gemm.forward(A, FakeDev((7, 6)))
    with pytest.raises(TypeError):
        gemm.forward(A, FakeDev((8, 6), "<f2"))                 # mixed dtypes
    with pytest.raises(ValueError, match="with_bias=True but bias is None"):
        gemm.forward(A, B, with_bias=True)
    with pytest.raises(ValueError, match="1D length"):
        gemm.forward(A, B, FakeDev((5,)))
    with pytest.raises(ValueError, match="unsupported bias shape"):
        gemm.forward(A, B, FakeDev((2, 6)))
    with pytest.raises(ValueError, match="unsupported bias ndim"):
        gemm.forward(A, B, FakeDev((1, 1, 6)))
    with pytest.raises(ValueError, match="out must be"):
        gemm.forward(A, B, out=FakeDev((4, 5)))
    with pytest.raises(ValueError, match="z_out must be"):
        gemm.forward(A, B, out=FakeDev((4, 6)), z_out=FakeDev((4, 6), "<f2"))


def test_backward_rejections(ops):
    gemm, _ = ops
    A, B, gY, Z = FakeDev((4, 8)), FakeDev((8, 6)), FakeDev((4, 6)), FakeDev((4, 6))
    with pytest.raises(ValueError, match="Shape mismatch"):
        gemm.backward(A, B, FakeDev((4, 5)), Z)
    with pytest.raises(ValueError, match="want_gBias=True requires with_bias=True"):
        gemm.backward(A, B, gY, Z, want_gBias=True)


def test_capture_rejections(ops):
    gemm, _ = ops
    A, B, out = FakeDev((4, 8)), FakeDev((8, 6)), FakeDev((4, 6))
    with pytest.raises(ValueError, match="out must be C-contiguous"):
        gemm.forward_into(A, B, out=FakeDev((4, 6), strides=(4, 16)))
    with pytest.raises(ValueError, match="inputs must be C-contiguous"):
        gemm.forward_into(FakeDev((4, 8), strides=(4, 16)), B, out=out)
    with pytest.raises(ValueError, match="bias provided but with_bias=False"):
        gemm.forward_into(A, B, out=out, bias=FakeDev((1, 6)))
    with pytest.raises(ValueError, match=r"bias must be C-contiguous float32\[1,N\]"):
        gemm.forward_into(A, B, out=out, bias=FakeDev((6,)), with_bias=True)
    with pytest.raises(ValueError, match="save_z=True requires z_out"):
        gemm.forward_into(A, B, out=out, act="relu", save_z=True)
    gY, Z = FakeDev((4, 6)), FakeDev((4, 6))
    with pytest.raises(ValueError, match="work_dZ must be"):
        gemm.backward_into(A, B, gY, Z)
    with pytest.raises(ValueError, match="work_dZ must be"):
        gemm.backward_into(A, B, gY, Z, work_dZ=FakeDev((4, 5)))
    with pytest.raises(ValueError, match="gC_out must be None when C is None"):
        gemm.backward_into(A, B, gY, Z, gC_out=FakeDev((4, 6)), work_dZ=FakeDev((4, 6)))
    with pytest.raises(ValueError, match="gBias_out must be None when with_bias=False"):
        gemm.backward_into(A, B, gY, Z, gBias_out=FakeDev((1, 6)), work_dZ=FakeDev((4, 6)))
    with pytest.raises(ValueError, match="gA_out must be"):
        gemm.backward_into(A, B, gY, Z, gA_out=FakeDev((4, 7)), work_dZ=FakeDev((4, 6)))
    with pytest.raises(ValueError, match="lt_workspace must be"):
        gemm.backward_into(A, B, gY, Z, work_dZ=FakeDev((4, 6)), lt_workspace=FakeDev((16,), "<f4"))


def test_dense_shape_rules():
    from graph_executor_v2.layers import Dense
    d = Dense(16, activation="relu")
    assert d.compute_output_shape((None, 8)) == (None, 16)
    assert d.compute_output_shape((4, 8)) == (4, 16)
    with pytest.raises(ValueError):
        d.compute_output_shape((4, 8, 2))
    with pytest.raises(RuntimeError):
        d.call(FakeDev((4, 8)))                       # before build
    with pytest.raises(RuntimeError):
        d.backward(FakeDev((4, 16)))
    with pytest.raises(ValueError):
        Dense(4, initializer="bogus")._init_weights(3)
    assert d.train(False).training is False and d.train().training is True
