"""CPU checks of the conv2d boundary: the _ops_conv2d module surface (the reference's
src/bindings/conv2d_pybind.cpp:60-258), its binding-level workspace checks, and the C ABI's
validation codes, all of which fail before any device work (nothing here is dereferenced)."""
import ctypes

import pytest


@pytest.fixture(scope="module")
def conv():
    from graph_executor_v2.ops import _ops_conv2d as c
    return c


def test_module_surface(conv):
    a = conv.Conv2DAttrs()
    assert (a.stride_h, a.stride_w, a.pad_h, a.pad_w, a.dil_h, a.dil_w, a.groups) == (1, 1, 0, 0, 1, 1, 1)
    assert a.act == conv.ActKind.__members__["None"] and a.leaky_slope == pytest.approx(0.01)
    assert not a.with_bias and not a.save_z
    for f in ("forward", "backward"):
        assert callable(getattr(conv, f))


def test_binding_workspace_checks(conv):
    x, w, y = [2, 3, 8, 8], [4, 3, 3, 3], [2, 4, 6, 6]
    with pytest.raises(ValueError, match="dCol, W_KC, Y_tmp"):
        conv.forward(16, x, 32, w, 48, y)
    a = conv.Conv2DAttrs()
    a.save_z = True
    with pytest.raises(ValueError, match="requires z_ptr"):
        conv.forward(16, x, 32, w, 48, y, attrs=a, dCol_ptr=64, W_KC_ptr=80, Y_tmp_ptr=96)
    with pytest.raises(ValueError, match="Z_rows workspace"):
        conv.forward(16, x, 32, w, 48, y, z_ptr=112, attrs=a, dCol_ptr=64, W_KC_ptr=80, Y_tmp_ptr=96)
    with pytest.raises(ValueError, match="dCol_ptr and dTmp_ptr"):
        conv.backward(16, x, 32, w, 48, y, 64, y)
    with pytest.raises(ValueError, match="gy_rows_ptr and Z_rows_ptr"):
        conv.backward(16, x, 32, w, 48, y, 64, y, dCol_ptr=80, dTmp_ptr=96)
    with pytest.raises(ValueError, match="gX path"):
        conv.backward(16, x, 32, w, 48, y, 64, y, dx_ptr=128, dCol_ptr=80, dTmp_ptr=96, gy_rows_ptr=100,
                      Z_rows_ptr=104)
    with pytest.raises(ValueError, match="gW path"):
        conv.backward(16, x, 32, w, 48, y, 64, y, dw_ptr=128, dCol_ptr=80, dTmp_ptr=96, gy_rows_ptr=100,
                      Z_rows_ptr=104)
    with pytest.raises(ValueError, match="4D"):
        conv.forward(16, [2, 3, 8], 32, w, 48, y)


def _fwd_desc(capi, **kw):
    d = capi.Conv2dDesc()
    d.dtype, d.N, d.Cin, d.H, d.W, d.Cout, d.Kh, d.Kw = 0, 2, 3, 8, 8, 4, 3, 3
    d.stride_h = d.stride_w = d.dil_h = d.dil_w = d.groups = 1
    d.X, d.Wt, d.Y, d.col, d.col_bytes = 16, 32, 48, 64, 10 ** 6
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_c_abi_validation(conv):
    from graph_executor_v2.ops import capi
    L = capi.lib()

    def st(**kw):
        return L.gev2_conv2d_fwd(ctypes.byref(_fwd_desc(capi, **kw)), None)

    assert st(dtype=7) == 101                      # DtypeMismatch
    assert st(act=9) == 4                          # InvalidArgument
    assert st(groups=2) == 2                       # Unimplemented (launcher.cu:117)
    assert st(Kh=11) == 1                          # empty output -> Invalid
    assert st(stride_h=0) == 1
    assert st(col=None) == 10                      # MissingInput (workspace)
    assert st(col_bytes=100) == 10                 # smaller than one image
    assert st(Y=None) == 11                        # MissingOutput
    assert st(save_z=1) == 11                      # save_z without Z
    assert b"col" in L.gev2_conv2d_last_error() or True
    b = capi.Conv2dBwdDesc()
    b.dtype, b.N, b.Cin, b.H, b.W, b.Cout, b.Kh, b.Kw = 0, 2, 3, 8, 8, 4, 3, 3
    b.stride_h = b.stride_w = b.dil_h = b.dil_w = b.groups = 1
    b.X, b.Wt, b.dY, b.Z, b.col, b.dX = 16, 32, 48, 64, 80, 96
    assert L.gev2_conv2d_bwd(ctypes.byref(b), None) == 10   # dX without the dcol workspace
