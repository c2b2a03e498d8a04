"""Python glue of the GEMM operator over the native ``_ops_gemm`` module.

The public surface is the reference's (python/graph_executor_v2/ops/gemm.py:22-509):
the same functions, keyword names, defaults, exception types and messages, and the
same policies:

  forward / backward            allocate their outputs; the bias may be a scalar,
                                (N,), (1,N), (M,1) or (M,N); Z aliases Y when
                                act == "none"; (Y, Z) is returned for save_z / return_z
  forward_into / backward_into  capture-safe: every buffer is the caller's and
                                C-contiguous, the bias is exactly (1,N) float32, and
                                work_dZ (M*N float32) is the backward's workspace
  ensure_workspaces / clear_ws_cache / GemmWorkspaces

How it is built here: each call is described once (operand shapes and dtype, the
bias as a (rows, cols) tensor, the Z target) by a few validators shared by the
allocating and the capture-safe forms, which then differ only in who supplies the
output buffers; one launcher per direction calls the module.  Arrays are device
arrays of any kind (ops.common); float16 / bfloat16 operands are accepted beside the
reference's float32, with float32 bias and gBias.  An (M,N) bias passes the glue and
is dropped by the operator's bias-kind rule (gemm/launcher.cu:47-77), as in the
reference.  There is no host fallback: a missing native module raises at import.
"""
from __future__ import annotations

from typing import Dict, NamedTuple, Optional, Tuple

import numpy as np

from . import _ops_gemm as g
from .common import (array_info, as_tensor_2d, assert_2d, astype, dtype_of, empty, empty_2d, empty_like_2d,
                     get_stream_ptr, is_c_contiguous, reshape, to_voidp_capsule)

_CAP = "[capture] "


# ---------------------------------------------------------------------------
# Workspaces (reference gemm.py:22-58): a float32 dZ[M,N] per (M, N, device) and
# an optional uint8 cuBLASLt-style workspace, which this operator does not use.
# ---------------------------------------------------------------------------
def _shape(x) -> Tuple[int, ...]:
    return tuple(array_info(x)[1])


def _is(x, shape, dtype) -> bool:
    return x is not None and _shape(x) == tuple(shape) and dtype_of(x) == dtype


class GemmWorkspaces:
    """Holder of the backward's dZ buffer and the optional lt workspace."""

    def __init__(self):
        self.dZ = None
        self.lt_ws = None

    def ensure_backward(self, M: int, N: int):
        if not _is(self.dZ, (M, N), "float32"):
            raise ValueError(f"[capture] work.dZ must be preallocated float32[{M},{N}]")
        if self.lt_ws is not None and dtype_of(self.lt_ws) != "uint8":
            raise ValueError("[capture] work.lt_ws must be uint8 or None")


_WS_CACHE: Dict[Tuple[int, int, int], GemmWorkspaces] = {}


def _current_device() -> int:
    import ctypes

    from . import capi
    d = ctypes.c_int()
    capi.check(capi.lib().gev2_get_device(ctypes.byref(d)), "gev2_get_device")
    return int(d.value)


def ensure_workspaces(M: int, N: int, *, lt_bytes: int = 0, like=None) -> GemmWorkspaces:
    """The cached workspaces of (M, N) on the current device, (re)allocated when missing,
    of the wrong shape or type, or (lt) smaller than lt_bytes."""
    ws = _WS_CACHE.setdefault((int(M), int(N), _current_device()), GemmWorkspaces())
    if not _is(ws.dZ, (M, N), "float32"):
        ws.dZ = empty((M, N), "float32", like)
    lt_ok = ws.lt_ws is not None and dtype_of(ws.lt_ws) == "uint8" and _shape(ws.lt_ws)[0] >= lt_bytes
    if lt_bytes > 0 and not lt_ok:
        ws.lt_ws = empty((lt_bytes,), "uint8", like)
    return ws


def clear_ws_cache() -> None:
    _WS_CACHE.clear()


# ---------------------------------------------------------------------------
# Activation names (reference gemm.py:64-94; the binding's parser accepts the same,
# gemm_pybind.cpp:57-69): spelling with spaces, '-' and '_' removed, any case.
# ---------------------------------------------------------------------------
_ACT_MEMBERS = {"none": "None", "relu": "ReLU", "leakyrelu": "LeakyReLU", "lrelu": "LeakyReLU",
                "gelu": "GELU", "sigmoid": "Sigmoid", "tanh": "Tanh"}


def _act_key(act) -> str:
    return "".join(c for c in (act or "none").strip().lower() if c not in " -_")


def _parse_act_to_kind(act):
    member = _ACT_MEMBERS.get(_act_key(act))
    if member is None:
        raise ValueError(f"unknown act: {act}")
    return getattr(g.ActKind, member)


def _mk_attrs(act, with_bias: bool, leaky_slope: float, save_z: bool = False):
    """GemmAttrs with no transposes; save_z is set exactly when a Z tensor is passed."""
    a = g.GemmAttrs()
    a.trans_a = a.trans_b = False
    a.act = _parse_act_to_kind(act)
    a.with_bias = bool(with_bias)
    a.leaky_slope = float(leaky_slope)
    a.save_z = bool(save_z)
    return a


# ---------------------------------------------------------------------------
# Validators shared by the allocating and the capture-safe forms
# ---------------------------------------------------------------------------
class _Problem(NamedTuple):
    M: int
    K: int
    N: int
    dtype: str


def _problem(A, B) -> _Problem:
    M, K = assert_2d(A, "A")
    K2, N = assert_2d(B, "B")
    if K != K2:
        raise ValueError(f"K mismatch: A(K={K}) vs B(K={K2})")
    if dtype_of(B) != dtype_of(A):
        raise TypeError(f"A and B must have the same dtype, got {dtype_of(A)} and {dtype_of(B)}")
    return _Problem(M, K, N, dtype_of(A))


def _require(x, name: str, shape, dtype: str, *, capture: bool, bracket: bool = True) -> None:
    """x must have `shape` and `dtype` (and be C-contiguous in the capture-safe form).
    The message names the expected type as the reference does: dtype[M,N] (bracket) or
    dtype(M, N)."""
    ok = _is(x, shape, dtype) and (not capture or is_c_contiguous(x))
    if not ok:
        dims = "[" + ",".join(str(s) for s in shape) + "]" if bracket else str(tuple(shape))
        raise ValueError(f"{_CAP if capture else ''}{name} must be {'C-contiguous ' if capture else ''}{dtype}{dims}")


def _bias_2d(bias, p: _Problem, like):
    """The allocating form's bias as a float32 2-D device array (reference gemm.py:120-143):
    a scalar becomes (1,1), a length-N vector (1,N); (1,N), (M,1) and (M,N) pass."""
    if np.isscalar(bias):
        out = empty((1, 1), "float32", like)
        (out.fill_ if hasattr(out, "fill_") else out.fill)(float(bias))
        return out
    bias = astype(bias, "float32")
    shape = _shape(bias)
    if len(shape) == 1:
        if shape[0] != p.N:
            raise ValueError(f"bias 1D length must be N={p.N}, got {shape[0]}")
        return reshape(bias, (1, p.N))
    if len(shape) != 2:
        raise ValueError(f"unsupported bias ndim={len(shape)}")
    if shape not in ((1, p.N), (p.M, 1), (p.M, p.N)):
        raise ValueError(f"unsupported bias shape {shape}; expected (1,N)|(M,1)|(M,N)")
    return bias


def _z_target(z_out, out, act, want_z: bool, p: _Problem, *, capture: bool, like=None):
    """Where Z goes (reference gemm.py:158-172, 370-384): the caller's z_out; else Y itself
    when act == none; else a new buffer, of the same array kind as `like`, when Z is wanted
    (allocating form only)."""
    if z_out is not None:
        _require(z_out, "z_out", (p.M, p.N), p.dtype, capture=capture)
        return z_out
    if _act_key(act) == "none":
        return out
    if want_z:
        if capture:
            raise ValueError("[capture] save_z=True requires z_out preallocated")
        return empty((p.M, p.N), p.dtype, like)
    return None


def _tensor(x):
    return as_tensor_2d(x) if x is not None else None


def _stream(stream, like):
    return to_voidp_capsule(get_stream_ptr(stream, like))


def _launch_forward(A, B, bias, out, z, act, with_bias, leaky_slope, stream) -> None:
    attrs = _mk_attrs(act, with_bias, leaky_slope, save_z=z is not None)
    g.forward_ex_attrs(as_tensor_2d(A), as_tensor_2d(B), _tensor(bias), as_tensor_2d(out), attrs, _tensor(z),
                       _stream(stream, A))


def _check_grad_inputs(A, B, gY, Z, *, capture: bool) -> _Problem:
    p = _problem(A, B)
    if assert_2d(gY, "gY") != (p.M, p.N) or assert_2d(Z, "Z") != (p.M, p.N):
        raise ValueError(f"[capture] gY/Z must be (M={p.M}, N={p.N})" if capture
                         else f"Shape mismatch: gY(Z) must be (M={p.M}, N={p.N})")
    return p


# ---------------------------------------------------------------------------
# Forward
# ---------------------------------------------------------------------------
def forward(A, B, bias=None, *, act: str = "none", with_bias: bool = False, leaky_slope: float = 0.01,
            stream: Optional[int] = None, out=None, save_z: bool = False, z_out=None, return_z: bool = False):
    """Y = act(A B + bias) into a new (or the given) array; returns Y, or (Y, Z) when save_z or
    return_z (reference gemm.py:99-218).  A bias argument implies with_bias."""
    p = _problem(A, B)
    with_bias = bool(with_bias) or bias is not None
    if with_bias and bias is None:
        raise ValueError("with_bias=True but bias is None")
    bias2d = _bias_2d(bias, p, A) if with_bias else None
    if out is None:
        out = empty((p.M, p.N), p.dtype, A)
    elif not _is(out, (p.M, p.N), p.dtype):
        raise ValueError(f"out must be {p.dtype}[{p.M},{p.N}]")
    z = _z_target(z_out, out, act, save_z or return_z, p, capture=False, like=A)
    _launch_forward(A, B, bias2d, out, z, act, with_bias, leaky_slope, stream)
    if return_z or (save_z and z is not None):
        return out, (out if z is None else z)
    return out


def forward_into(A, B, *, out, bias=None, act: str = "none", with_bias: bool = False, leaky_slope: float = 0.01,
                 save_z: bool = False, z_out=None, stream: Optional[int] = None) -> None:
    """Capture-safe forward into caller buffers (reference gemm.py:317-399)."""
    p = _problem(A, B)
    _require(out, "out", (p.M, p.N), p.dtype, capture=True)
    if not (is_c_contiguous(A) and is_c_contiguous(B)):
        raise ValueError("[capture] inputs must be C-contiguous")
    if bias is not None and not with_bias:
        raise ValueError("[capture] bias provided but with_bias=False")
    if with_bias:
        if bias is None:
            raise ValueError("[capture] with_bias=True but bias is None")
        if np.isscalar(bias) or not (_is(bias, (1, p.N), "float32") and is_c_contiguous(bias)):
            raise ValueError("[capture] bias must be C-contiguous float32[1,N] (PerN)")
    z = _z_target(z_out, out, act, save_z, p, capture=True)
    _launch_forward(A, B, bias if with_bias else None, out, z, act, with_bias, leaky_slope, stream)


# ---------------------------------------------------------------------------
# Backward
# ---------------------------------------------------------------------------
_GRAD_KEYS = ("gA", "gB", "gC", "gBias")


def backward(A, B, gY, Z, *, act: str = "none", with_bias: bool = False, leaky_slope: float = 0.01, C=None,
             want_gA: bool = True, want_gB: bool = True, want_gBias: bool = False, stream: Optional[int] = None,
             warn_mismatch: bool = False) -> Dict[str, object]:
    """Gradients into new arrays, returned by name: gA and gB as asked, gC when C is given,
    gBias (1,N) float32 when asked with a bias (reference gemm.py:224-311)."""
    p = _check_grad_inputs(A, B, gY, Z, capture=False)
    with_bias = bool(with_bias)
    if want_gBias and not with_bias:
        raise ValueError("want_gBias=True requires with_bias=True")
    grads = {
        "gA": empty_like_2d(A) if want_gA else None,
        "gB": empty_like_2d(B) if want_gB else None,
        "gC": empty_like_2d(Z) if C is not None else None,
        "gBias": empty_2d(1, p.N, like=A, dtype="float32") if want_gBias else None,
    }
    g.backward_ex_attrs(as_tensor_2d(A), as_tensor_2d(B), _tensor(C), as_tensor_2d(gY), as_tensor_2d(Z),
                        *(_tensor(grads[k]) for k in _GRAD_KEYS), _mk_attrs(act, with_bias, leaky_slope),
                        _stream(stream, A))
    return {k: v for k, v in grads.items() if v is not None}


def backward_into(A, B, gY, Z, *, act: str = "none", with_bias: bool = False, leaky_slope: float = 0.01, C=None,
                  gA_out=None, gB_out=None, gC_out=None, gBias_out=None, stream: Optional[int] = None,
                  work_dZ=None, lt_workspace=None) -> None:
    """Capture-safe backward into caller buffers; work_dZ (M*N float32) is the operator's
    dY' workspace, so the call allocates nothing (reference gemm.py:405-509)."""
    p = _check_grad_inputs(A, B, gY, Z, capture=True)
    if not all(is_c_contiguous(x) for x in (A, B, gY, Z)):
        raise ValueError("[capture] A, B, gY, Z must be C-contiguous")
    for arr, name, shape in ((gA_out, "gA_out", (p.M, p.K)), (gB_out, "gB_out", (p.K, p.N))):
        if arr is not None:
            _require(arr, name, shape, p.dtype, capture=True, bracket=False)
    if C is None and gC_out is not None:
        raise ValueError("[capture] gC_out must be None when C is None")
    if C is not None:
        if assert_2d(C, "C") != (p.M, p.N):
            raise ValueError(f"[capture] C must be (M={p.M}, N={p.N})")
        if gC_out is not None:
            _require(gC_out, "gC_out", (p.M, p.N), p.dtype, capture=True, bracket=False)
    if not with_bias and gBias_out is not None:
        raise ValueError("[capture] gBias_out must be None when with_bias=False")
    if with_bias and gBias_out is not None:
        _require(gBias_out, "gBias_out", (1, p.N), "float32", capture=True, bracket=False)
    dz_ok = (work_dZ is not None and dtype_of(work_dZ) == "float32" and array_info(work_dZ)[0] != 0
             and int(np.prod(_shape(work_dZ))) == p.M * p.N and is_c_contiguous(work_dZ))
    if not dz_ok:
        raise ValueError("[capture] work_dZ must be C-contiguous float32 with size M*N")
    lt_ptr = lt_bytes = 0
    if lt_workspace is not None:
        if dtype_of(lt_workspace) != "uint8" or not is_c_contiguous(lt_workspace):
            raise ValueError("[capture] lt_workspace must be C-contiguous uint8")
        lt_ptr, lt_bytes = array_info(lt_workspace)[0], int(np.prod(_shape(lt_workspace)))
    g.backward_into(as_tensor_2d(A), as_tensor_2d(B), _tensor(C), as_tensor_2d(gY), as_tensor_2d(Z),
                    _tensor(gA_out), _tensor(gB_out), _tensor(gC_out), _tensor(gBias_out),
                    _mk_attrs(act, with_bias, leaky_slope), _stream(stream, A), int(array_info(work_dZ)[0]),
                    int(lt_ptr), int(lt_bytes))
