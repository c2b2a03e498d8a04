"""CPU checks of the RNN boundary: the _ops_rnn module surface (the reference's
src/bindings/rnn_pybind.cpp:74-283), its binding-level workspace checks, the host
validation codes (rnn/launcher.cu:39-127) and the C ABI's, all of which fail before any
device work (nothing here is dereferenced)."""
import ctypes

import pytest


@pytest.fixture(scope="module")
def rnn():
    from graph_executor_v2.ops import _ops_rnn as r
    return r


X, WX, WH, H0, Y = [2, 5, 3], [3, 4], [4, 4], [2, 4], [2, 5, 4]


def test_module_surface(rnn):
    a = rnn.RnnAttrs()
    assert a.act == rnn.ActKind.__members__["None"] and a.leaky_slope == pytest.approx(0.01)
    assert not a.with_bias and a.save_z            # the reference's defaults (api.hpp:10-15)
    for f in ("forward", "backward"):
        assert callable(getattr(rnn, f))


def test_binding_workspace_checks(rnn):
    a = rnn.RnnAttrs()
    a.save_z = False
    with pytest.raises(ValueError, match="XH_cat, Y_rows, W_cat"):
        rnn.forward(16, X, 32, WX, 48, WH, 64, H0, 80, Y, attrs=a)
    a.save_z = True
    with pytest.raises(ValueError, match="requires z_ptr"):
        rnn.forward(16, X, 32, WX, 48, WH, 64, H0, 80, Y, attrs=a, XH_cat_ptr=96, Y_rows_ptr=112, W_cat_ptr=128)
    with pytest.raises(ValueError, match="Z_rows workspace"):
        rnn.forward(16, X, 32, WX, 48, WH, 64, H0, 80, Y, z_ptr=144, attrs=a, XH_cat_ptr=96, Y_rows_ptr=112,
                    W_cat_ptr=128)
    with pytest.raises(ValueError, match="all workspace pointers"):
        rnn.backward(16, X, 32, WX, 48, WH, 64, H0, 80, Y, 96, Y, XH_cat_ptr=112)
    with pytest.raises(ValueError, match="3D"):
        rnn.forward(16, [2, 5], 32, WX, 48, WH, 64, H0, 80, Y)


def test_host_validation(rnn):
    """Shape errors surface as the reference's Status (ShapeMismatch = 103) before any launch."""
    a = rnn.RnnAttrs()
    a.save_z = False
    ws = dict(XH_cat_ptr=96, Y_rows_ptr=112, W_cat_ptr=128)
    with pytest.raises(RuntimeError, match="Status=103"):
        rnn.forward(16, X, 32, [2, 4], 48, WH, 64, H0, 80, Y, attrs=a, **ws)      # Wx rows != I
    with pytest.raises(RuntimeError, match="Status=103"):
        rnn.forward(16, X, 32, WX, 48, WH, 64, H0, 80, [2, 5, 3], attrs=a, **ws)  # Y last dim != H
    a.with_bias = True
    with pytest.raises(RuntimeError, match="Status=10:"):
        rnn.forward(16, X, 32, WX, 48, WH, 64, H0, 80, Y, attrs=a, **ws)          # with_bias, no B
    bws = dict(XH_cat_ptr=96, G_rows_ptr=100, Z_rows_ptr=104, W_cat_ptr=108, dXH_cat_ptr=112, dWcat_ptr=116,
               TmpW_ptr=120)
    with pytest.raises(RuntimeError, match="Status=103"):
        rnn.backward(16, X, 32, WX, 48, WH, 64, H0, 80, Y, 96, [2, 4, 4], **bws)  # Z shape


def test_c_abi_validation(rnn):
    from graph_executor_v2.ops import capi
    L = capi.lib()

    def fwd(**kw):
        d = capi.RnnDesc(dtype=0, N=2, T=5, I=3, H=4, X=16, Wx=32, Wh=48, h0=64, Y=80, xh=96, wcat=112)
        for k, v in kw.items():
            setattr(d, k, v)
        return L.gev2_rnn_fwd(ctypes.byref(d), None)

    assert fwd(dtype=7) == 101                     # DtypeMismatch
    assert fwd(act=9) == 4                         # InvalidArgument
    assert fwd(H=0) == 1                           # Invalid
    assert fwd(Wh=None) == 10                      # MissingInput
    assert fwd(xh=None) == 10                      # workspace
    assert fwd(Y=None) == 11                       # MissingOutput
    assert fwd(save_z=1) == 11                     # save_z without Z
    assert fwd(save_z=1, Z=80) == 1                # Z aliases Y
    assert L.gev2_rnn_last_error() == b"Z must not alias Y"
    b = capi.RnnBwdDesc(dtype=0, N=2, T=5, I=3, H=4, X=16, Wx=32, Wh=48, h0=64, dY=80, Z=96)
    assert L.gev2_rnn_bwd(ctypes.byref(b), None) == 10   # workspaces missing
