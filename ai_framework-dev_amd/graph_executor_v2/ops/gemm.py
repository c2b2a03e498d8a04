"""Python glue of the GEMM operator (reference: python/graph_executor_v2/ops/gemm.py:99-509).

Same functions, keywords, defaults and policies as the reference, over the
native ``_ops_gemm`` module:

  forward / backward            allocating; bias given as a scalar, (N,), (1,N),
                                (M,1) or (M,N); Z aliases Y when act == "none";
                                returns (Y, Z) when save_z / return_z
  forward_into / backward_into  capture-safe: every buffer preallocated and
                                C-contiguous, bias exactly (1,N), work_dZ required
  ensure_workspaces / clear_ws_cache / GemmWorkspaces

Arrays are device arrays of any kind (see ops.common); float32 as in the
reference, plus float16 / bfloat16 operands with float32 bias and gBias.  An
(M,N) bias is accepted here and dropped by the operator's bias-kind rule
(launcher.cu:47-77), as in the reference.  There is no host fallback: a missing
native module raises at import.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import numpy as np

from . import _ops_gemm as g
from .common import (array_info, as_tensor_2d, assert_2d, astype, dtype_of, empty, empty_2d, empty_like_2d,
                     get_stream_ptr, is_c_contiguous, reshape, to_voidp_capsule)

# -------------------------------
# Workspace helpers (gemm.py:22-58)
# -------------------------------
class GemmWorkspaces:
    def __init__(self):
        self.dZ = None
        self.lt_ws = None

    def ensure_backward(self, M: int, N: int):
        if self.dZ is None or dtype_of(self.dZ) != "float32" or tuple(array_info(self.dZ)[1]) != (M, N):
            raise ValueError(f"[capture] work.dZ must be preallocated float32[{M},{N}]")
        if self.lt_ws is not None and dtype_of(self.lt_ws) != "uint8":
            raise ValueError("[capture] work.lt_ws must be uint8 or None")


_WS_CACHE: Dict[Tuple[int, int, int], GemmWorkspaces] = {}


def _device() -> int:
    from . import capi
    import ctypes
    d = ctypes.c_int()
    capi.check(capi.lib().gev2_get_device(ctypes.byref(d)), "gev2_get_device")
    return int(d.value)


def ensure_workspaces(M: int, N: int, *, lt_bytes: int = 0, like=None) -> GemmWorkspaces:
    """Cached float32 dZ[M,N] (and uint8 lt workspace) per (M, N, device)."""
    key = (int(M), int(N), _device())
    ws = _WS_CACHE.get(key)
    ref = like
    if ws is None:
        ws = GemmWorkspaces()
        ws.dZ = empty((M, N), "float32", ref)
        ws.lt_ws = empty((lt_bytes,), "uint8", ref) if lt_bytes > 0 else None
        _WS_CACHE[key] = ws
    else:
        if ws.dZ is None or tuple(array_info(ws.dZ)[1]) != (M, N) or dtype_of(ws.dZ) != "float32":
            ws.dZ = empty((M, N), "float32", ref)
        if lt_bytes > 0 and (ws.lt_ws is None or array_info(ws.lt_ws)[1][0] < lt_bytes
                             or dtype_of(ws.lt_ws) != "uint8"):
            ws.lt_ws = empty((lt_bytes,), "uint8", ref)
    return ws


def clear_ws_cache() -> None:
    _WS_CACHE.clear()


# -------------------------------
# Attr helpers (gemm.py:64-94)
# -------------------------------
def _parse_act_to_kind(act: str):
    s = (act or "none").strip().lower().replace(" ", "").replace("-", "").replace("_", "")
    if s == "none":
        return getattr(g.ActKind, "None")
    if s == "relu":
        return g.ActKind.ReLU
    if s in ("leakyrelu", "lrelu"):
        return g.ActKind.LeakyReLU
    if s == "gelu":
        return g.ActKind.GELU
    if s == "sigmoid":
        return g.ActKind.Sigmoid
    if s == "tanh":
        return g.ActKind.Tanh
    raise ValueError(f"unknown act: {act}")


def _mk_attrs(act: str, with_bias: bool, leaky_slope: float):
    a = g.GemmAttrs()
    a.trans_a = False
    a.trans_b = False
    a.act = _parse_act_to_kind(act)
    a.with_bias = bool(with_bias)
    a.leaky_slope = float(leaky_slope)
    return a


def _act_is_none(act) -> bool:
    return (act or "none").strip().lower() in ("none",)


def _check_operands(A, B) -> Tuple[int, int, int, str]:
    M, K = assert_2d(A, "A")
    K2, N = assert_2d(B, "B")
    if K != K2:
        raise ValueError(f"K mismatch: A(K={K}) vs B(K={K2})")
    dt = dtype_of(A)
    if dtype_of(B) != dt:
        raise TypeError(f"A and B must have the same dtype, got {dt} and {dtype_of(B)}")
    return M, K, N, dt


def _scalar_bias(value, like):
    """(1,1) float32 device array holding `value` (gemm.py:131-132)."""
    out = empty((1, 1), "float32", like)
    if hasattr(out, "fill_"):   # torch
        out.fill_(float(value))
    else:
        out.fill(float(value))
    return out


# ============================================================
# Forward (allocating), gemm.py:99-218
# ============================================================
def forward(
    A,
    B,
    bias=None,
    *,
    act: str = "none",
    with_bias: bool = False,
    leaky_slope: float = 0.01,
    stream: Optional[int] = None,
    out=None,
    save_z: bool = False,
    z_out=None,
    return_z: bool = False,
):
    M, K, N, dt = _check_operands(A, B)

    # with_bias is inferred from the bias argument on this path
    if bias is not None and not with_bias:
        with_bias = True

    tBias = None
    if with_bias:
        if bias is None:
            raise ValueError("with_bias=True but bias is None")
        if np.isscalar(bias):
            bias = _scalar_bias(bias, A)
        else:
            bias = astype(bias, "float32")
            bshape = tuple(array_info(bias)[1])
            if len(bshape) == 1:
                if bshape[0] != N:
                    raise ValueError(f"bias 1D length must be N={N}, got {bshape[0]}")
                bias = reshape(bias, (1, N))
            elif len(bshape) == 2:
                bm, bn = bshape
                if not ((bm == 1 and bn == N) or (bm == M and bn == 1) or (bm == M and bn == N)):
                    raise ValueError(f"unsupported bias shape {bshape}; expected (1,N)|(M,1)|(M,N)")
            else:
                raise ValueError(f"unsupported bias ndim={len(bshape)}")
        tBias = as_tensor_2d(bias)

    if out is None:
        out = empty((M, N), dt, A)
    elif tuple(array_info(out)[1]) != (M, N) or dtype_of(out) != dt:
        raise ValueError(f"out must be {dt}[{M},{N}]")

    # Z buffer policy (gemm.py:158-172): the caller's z_out; else Y itself when
    # act == none; else a new buffer only when Z is wanted
    if z_out is not None:
        if tuple(array_info(z_out)[1]) != (M, N) or dtype_of(z_out) != dt:
            raise ValueError(f"z_out must be {dt}[{M},{N}]")
        z_arr = z_out
    elif _act_is_none(act):
        z_arr = out
    elif save_z or return_z:
        z_arr = empty((M, N), dt, A)
    else:
        z_arr = None

    tA, tB, tY = as_tensor_2d(A), as_tensor_2d(B), as_tensor_2d(out)
    tZ = as_tensor_2d(z_arr) if z_arr is not None else None
    attrs = _mk_attrs(act, with_bias, leaky_slope)
    attrs.save_z = tZ is not None          # Z tensor passed <=> save_z
    g.forward_ex_attrs(tA, tB, tBias, tY, attrs, tZ, to_voidp_capsule(get_stream_ptr(stream, A)))

    if tZ is not None and (return_z or save_z):
        return out, z_arr
    if return_z:
        return out, (z_arr if z_arr is not None else out)
    return out


# ============================================================
# Backward (allocating), gemm.py:224-311
# ============================================================
def backward(
    A,
    B,
    gY,
    Z,
    *,
    act: str = "none",
    with_bias: bool = False,
    leaky_slope: float = 0.01,
    C=None,
    want_gA: bool = True,
    want_gB: bool = True,
    want_gBias: bool = False,
    stream: Optional[int] = None,
    warn_mismatch: bool = False,
) -> Dict[str, object]:
    M, K, N, dt = _check_operands(A, B)
    Mg, Ng = assert_2d(gY, "gY")
    Mz, Nz = assert_2d(Z, "Z")
    if (Mg, Ng) != (M, N) or (Mz, Nz) != (M, N):
        raise ValueError(f"Shape mismatch: gY(Z) must be (M={M}, N={N})")

    with_bias = bool(with_bias)
    if with_bias is False and want_gBias:
        raise ValueError("want_gBias=True requires with_bias=True")

    tA, tB, tgY, tZ = as_tensor_2d(A), as_tensor_2d(B), as_tensor_2d(gY), as_tensor_2d(Z)
    tC = as_tensor_2d(C) if C is not None else None

    gA_arr = empty_like_2d(A) if want_gA else None
    gB_arr = empty_like_2d(B) if want_gB else None
    gC_arr = empty_like_2d(Z) if C is not None else None
    gBias_arr = empty_2d(1, N, like=A, dtype="float32") if (want_gBias and with_bias) else None

    attrs = _mk_attrs(act, with_bias, leaky_slope)
    g.backward_ex_attrs(
        tA, tB, tC, tgY, tZ,
        as_tensor_2d(gA_arr) if gA_arr is not None else None,
        as_tensor_2d(gB_arr) if gB_arr is not None else None,
        as_tensor_2d(gC_arr) if gC_arr is not None else None,
        as_tensor_2d(gBias_arr) if gBias_arr is not None else None,
        attrs, to_voidp_capsule(get_stream_ptr(stream, A)))

    outd: Dict[str, object] = {}
    if gA_arr is not None:
        outd["gA"] = gA_arr
    if gB_arr is not None:
        outd["gB"] = gB_arr
    if gC_arr is not None:
        outd["gC"] = gC_arr
    if gBias_arr is not None:
        outd["gBias"] = gBias_arr
    return outd


# ============================================================
# Forward (capture-safe, no allocations), gemm.py:317-399
# ============================================================
def forward_into(
    A,
    B,
    *,
    out,
    bias=None,
    act: str = "none",
    with_bias: bool = False,
    leaky_slope: float = 0.01,
    save_z: bool = False,
    z_out=None,
    stream: Optional[int] = None,
) -> None:
    M, K, N, dt = _check_operands(A, B)
    if out is None or dtype_of(out) != dt or tuple(array_info(out)[1]) != (M, N) or not is_c_contiguous(out):
        raise ValueError(f"[capture] out must be C-contiguous {dt}[{M},{N}]")
    if not (is_c_contiguous(A) and is_c_contiguous(B)):
        raise ValueError("[capture] inputs must be C-contiguous")
    if bias is not None and with_bias is False:
        raise ValueError("[capture] bias provided but with_bias=False")

    tBias = None
    if with_bias:
        if bias is None:
            raise ValueError("[capture] with_bias=True but bias is None")
        if np.isscalar(bias) or not (dtype_of(bias) == "float32" and tuple(array_info(bias)[1]) == (1, N)
                                     and is_c_contiguous(bias)):
            raise ValueError("[capture] bias must be C-contiguous float32[1,N] (PerN)")
        tBias = as_tensor_2d(bias)

    if z_out is not None:
        if dtype_of(z_out) != dt or tuple(array_info(z_out)[1]) != (M, N) or not is_c_contiguous(z_out):
            raise ValueError(f"[capture] z_out must be C-contiguous {dt}[{M},{N}]")
        z_arr = z_out
    elif _act_is_none(act):
        z_arr = out
    elif save_z:
        raise ValueError("[capture] save_z=True requires z_out preallocated")
    else:
        z_arr = None

    tZ = as_tensor_2d(z_arr) if z_arr is not None else None
    attrs = _mk_attrs(act, with_bias, leaky_slope)
    attrs.save_z = tZ is not None
    g.forward_ex_attrs(as_tensor_2d(A), as_tensor_2d(B), tBias, as_tensor_2d(out), attrs, tZ,
                       to_voidp_capsule(get_stream_ptr(stream, A)))


# ============================================================
# Backward (capture-safe, no allocations), gemm.py:405-509
# ============================================================
def backward_into(
    A,
    B,
    gY,
    Z,
    *,
    act: str = "none",
    with_bias: bool = False,
    leaky_slope: float = 0.01,
    C=None,
    gA_out=None,
    gB_out=None,
    gC_out=None,
    gBias_out=None,
    stream: Optional[int] = None,
    work_dZ=None,
    lt_workspace=None,
) -> None:
    M, K, N, dt = _check_operands(A, B)
    Mg, Ng = assert_2d(gY, "gY")
    Mz, Nz = assert_2d(Z, "Z")
    if (Mg, Ng) != (M, N) or (Mz, Nz) != (M, N):
        raise ValueError(f"[capture] gY/Z must be (M={M}, N={N})")
    if not (is_c_contiguous(A) and is_c_contiguous(B) and is_c_contiguous(gY) and is_c_contiguous(Z)):
        raise ValueError("[capture] A, B, gY, Z must be C-contiguous")

    def _chk(arr, shape, name, want=dt):
        if arr is None:
            return
        if dtype_of(arr) != want or tuple(array_info(arr)[1]) != shape or not is_c_contiguous(arr):
            raise ValueError(f"[capture] {name} must be C-contiguous {want}{shape}")

    _chk(gA_out, (M, K), "gA_out")
    _chk(gB_out, (K, N), "gB_out")
    if C is None:
        if gC_out is not None:
            raise ValueError("[capture] gC_out must be None when C is None")
    else:
        Mc, Nc = assert_2d(C, "C")
        if (Mc, Nc) != (M, N):
            raise ValueError(f"[capture] C must be (M={M}, N={N})")
        _chk(gC_out, (M, N), "gC_out")
    if with_bias:
        _chk(gBias_out, (1, N), "gBias_out", "float32")
    elif gBias_out is not None:
        raise ValueError("[capture] gBias_out must be None when with_bias=False")

    if (work_dZ is None or dtype_of(work_dZ) != "float32" or array_info(work_dZ)[0] == 0
            or int(np.prod(array_info(work_dZ)[1])) != M * N or not is_c_contiguous(work_dZ)):
        raise ValueError("[capture] work_dZ must be C-contiguous float32 with size M*N")
    dZ_ptr = array_info(work_dZ)[0]
    if lt_workspace is not None:
        if dtype_of(lt_workspace) != "uint8" or not is_c_contiguous(lt_workspace):
            raise ValueError("[capture] lt_workspace must be C-contiguous uint8")
        lt_ptr = array_info(lt_workspace)[0]
        lt_bytes = int(np.prod(array_info(lt_workspace)[1]))
    else:
        lt_ptr, lt_bytes = 0, 0

    attrs = _mk_attrs(act, with_bias, leaky_slope)
    g.backward_into(
        as_tensor_2d(A), as_tensor_2d(B), as_tensor_2d(C) if C is not None else None,
        as_tensor_2d(gY), as_tensor_2d(Z),
        as_tensor_2d(gA_out) if gA_out is not None else None,
        as_tensor_2d(gB_out) if gB_out is not None else None,
        as_tensor_2d(gC_out) if gC_out is not None else None,
        as_tensor_2d(gBias_out) if gBias_out is not None else None,
        attrs, to_voidp_capsule(get_stream_ptr(stream, A)), int(dZ_ptr), int(lt_ptr), int(lt_bytes))
