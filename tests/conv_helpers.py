"""Shared helpers for the conv2d operator tests: geometries, seeded inputs, and one
forward (+ backward) call through _ops_conv2d with the reference's workspace contract
(conv2d_pybind.cpp:163-166; conv2d/launcher.cu:106-459)."""
import numpy as np

from oracle import gemm_oracle as O
from gemm_helpers import F32


GEOMS = {
    "c5a-like": dict(N=3, Cin=8, H=10, W=12, Cout=16, Kh=3, Kw=3, stride=(1, 1), pad=(1, 1), dil=(1, 1)),
    "stride2": dict(N=2, Cin=5, H=11, W=9, Cout=12, Kh=3, Kw=2, stride=(2, 1), pad=(0, 2), dil=(1, 1)),
    "dilated": dict(N=2, Cin=4, H=9, W=10, Cout=8, Kh=2, Kw=3, stride=(1, 2), pad=(1, 0), dil=(2, 1)),
    "pointwise": dict(N=2, Cin=6, H=5, W=7, Cout=4, Kh=1, Kw=1, stride=(1, 1), pad=(0, 0), dil=(1, 1)),
    # kernel the size of the input: a 1x1 output, so the reference-sized gy_rows workspace
    # (Cout*Ho*Wo floats) holds only the dB sum
    "1x1-output": dict(N=3, Cin=4, H=3, W=5, Cout=6, Kh=3, Kw=5, stride=(1, 1), pad=(0, 0), dil=(1, 1)),
    # unit horizontal stride with 16-byte input rows and Wo a multiple of 8: im2col and col2im
    # read each run as shifted 16-byte windows (even shifts here, both parities below)
    "window-dilated": dict(N=2, Cin=3, H=9, W=24, Cout=8, Kh=3, Kw=3, stride=(2, 1), pad=(2, 2), dil=(2, 2)),
    "window-odd-pad": dict(N=2, Cin=3, H=6, W=16, Cout=5, Kh=3, Kw=5, stride=(1, 1), pad=(1, 2), dil=(1, 1)),
}
WINDOW_GEOMS = ("window-dilated", "window-odd-pad")


def _attrs(conv, g, act, with_bias, save_z):
    a = conv.Conv2DAttrs()
    a.stride_h, a.stride_w = g["stride"]
    a.pad_h, a.pad_w = g["pad"]
    a.dil_h, a.dil_w = g["dil"]
    a.act = {"none": conv.ActKind.__members__["None"], "relu": conv.ActKind.ReLU, "tanh": conv.ActKind.Tanh,
             "leakyrelu": conv.ActKind.LeakyReLU}[act]
    a.with_bias = with_bias
    a.save_z = save_z
    return a


def _run(env, g, X, W, b, act, dtype=F32, all_images=False, dY=None, bwd_images=1):
    conv, DA = env
    dt = "float32" if dtype == F32 else "bfloat16"
    cdt = conv.DType.F32 if dtype == F32 else conv.DType.BF16
    N, Cout = g["N"], g["Cout"]
    Ho, Wo = O.conv2d_out_size(g["H"], g["W"], g["Kh"], g["Kw"], g["stride"], g["pad"], g["dil"])
    K, HWo = g["Cin"] * g["Kh"] * g["Kw"], Ho * Wo
    dX_, dW_, db_ = DA.from_numpy(X, dt), DA.from_numpy(W, dt), DA.from_numpy(b, "float32")
    Y, Z = DA.empty((N, Cout, Ho, Wo), dt), DA.empty((N, Cout, Ho, Wo), dt)
    col = DA.empty((N if all_images else 1, K * HWo), dt)
    wkc, ytmp, zrows = DA.empty((K * Cout,)), DA.empty((HWo * Cout,)), DA.empty((HWo * Cout,))
    a = _attrs(conv, g, act, True, True)
    conv.forward(dX_.ptr, list(X.shape), dW_.ptr, list(W.shape), Y.ptr, list(Y.shape), bias_ptr=db_.ptr,
                 z_ptr=Z.ptr, attrs=a, dCol_ptr=col.ptr, W_KC_ptr=wkc.ptr, Y_tmp_ptr=ytmp.ptr, Z_rows_ptr=zrows.ptr,
                 dtype=cdt, dCol_bytes=col.nbytes if all_images else 0)
    out = {"Y": Y.get(), "Z": Z.get()}
    if dY is not None:
        gdY = DA.from_numpy(dY, dt)
        gW, gb, gX = DA.empty(W.shape, dt), DA.empty((Cout,), "float32"), DA.empty(X.shape, dt)
        # the reference's backward workspaces (conv2d_pybind.cpp:163-166), kept alive for the call
        # (bwd_images > 1: larger dCol / dTmp / W_CK, so that one batched call covers that many images)
        c = bwd_images
        bufs = dict(dCol_ptr=DA.empty((c, K * HWo), dt), dTmp_ptr=DA.empty((c, max(Cout * K, HWo * K))),
                    W_CK_ptr=DA.empty((c, Cout * K)), dWpack_ptr=DA.empty((Cout * K,)),
                    dY_HT_ptr=DA.empty((HWo * Cout,)), gy_rows_ptr=DA.empty((Cout * HWo,)),
                    Z_rows_ptr=DA.empty((Cout * HWo,)))
        sizes = {} if c == 1 else dict(dCol_bytes=bufs["dCol_ptr"].nbytes, dTmp_bytes=bufs["dTmp_ptr"].nbytes,
                                       W_CK_bytes=bufs["W_CK_ptr"].nbytes)
        conv.backward(dX_.ptr, list(X.shape), dW_.ptr, list(W.shape), gdY.ptr, list(dY.shape), Z.ptr, list(dY.shape),
                      dw_ptr=gW.ptr, db_ptr=gb.ptr, dx_ptr=gX.ptr, attrs=a, dtype=cdt,
                      **{k: v.ptr for k, v in bufs.items()}, **sizes)
        out.update(dW=gW.get(), dB=gb.get(), dX=gX.get())
    return out


def _inputs(g, seed, integers=False):
    r = np.random.default_rng(seed)
    shapeX = (g["N"], g["Cin"], g["H"], g["W"])
    shapeW = (g["Cout"], g["Cin"], g["Kh"], g["Kw"])
    if integers:
        return (r.integers(-3, 4, shapeX).astype(np.float32), r.integers(-2, 3, shapeW).astype(np.float32),
                r.integers(-4, 5, g["Cout"]).astype(np.float32))
    K = g["Cin"] * g["Kh"] * g["Kw"]
    return (r.uniform(0, 1, shapeX).astype(np.float32),
            (r.standard_normal(shapeW) * np.sqrt(2 / K)).astype(np.float32),
            (0.02 * r.standard_normal(g["Cout"])).astype(np.float32))


