"""Dense layer on the fused GEMM operator (reference: python/graph_executor_v2/layers/dense_gemm.py:40-493).

  W: (in_dim, units), b: (1, units) float32; forward A(M,in) W + b -> act -> Y(M,units)
  Z (pre-activation) is kept for the backward when training and act != "none".
  Bias gradient: sum over rows, shape (1, units).

Same constructor, lifecycle, capture-safe hooks and gradient buffers as the
reference.  Differences, each because this build has no array library beside
the operator:

  - `dtype` (additive) selects float32 (the reference's only type), bfloat16 or
    float16 weights; the bias and its gradient stay float32.
  - Both backward modes run the operator's fused backward.  The reference's
    manual mode (use_native_bwd=False, :310-333) recomputes the same quantities
    with CuPy array math (act'(Z) * dY, x^T go, column sum, go W^T), and its
    native mode cross-checks dBias against such a column sum (:262-282); the
    operator's dBias here is tested directly against the oracle instead.
  - No silent CuPy fallback when the operator raises (:166-189): errors surface.
  - Weights are drawn on the host with numpy (seedable via `seed`) and uploaded.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import numpy as np

from ..ops import gemm as gemm_ops
from ..ops.common import array_info, astype, dtype_of, empty_like_2d, is_c_contiguous
from ..ops.device_array import DeviceArray, dtype_name
from .base import Layer


class Dense(Layer):
    def __init__(
        self,
        units: int,
        activation: Optional[str] = None,
        initializer: str = "he",
        name: Optional[str] = None,
        leaky_slope: float = 0.01,
        use_native_bwd: bool = False,
        *,
        dtype: str = "float32",
        seed: Optional[int] = None,
    ):
        super().__init__(name=name)
        self.units = int(units)
        self.activation = (activation or "none").lower()
        self.initializer = initializer
        self.leaky_slope = float(leaky_slope)
        self.use_native_bwd = bool(use_native_bwd)
        self.dtype = dtype_name(dtype)
        self._rng = np.random.default_rng(seed)

        self.W = None            # (in_dim, units), layer dtype
        self.b = None            # (1, units) float32
        self.last_input = None
        self.last_linear = None  # Z
        self.dW = None
        self.db = None
        self.training: bool = True

    # ---------------- init helpers (:76-109) ----------------
    def _init_weights(self, in_dim: int) -> Tuple[DeviceArray, DeviceArray]:
        shape = (in_dim, self.units)
        r = self._rng
        init = self.initializer
        if init == "zeros":
            W = np.zeros(shape)
        elif init == "ones":
            W = np.ones(shape)
        elif init == "uniform":
            W = r.uniform(-0.05, 0.05, shape)
        elif init == "normal":
            W = r.normal(0.0, 0.05, shape)
        elif init == "xavier":
            lim = np.sqrt(6.0 / (in_dim + self.units))
            W = r.uniform(-lim, lim, shape)
        elif init == "he":
            W = r.normal(0.0, np.sqrt(2.0 / in_dim), shape)
        elif init == "lecun":
            W = r.normal(0.0, np.sqrt(1.0 / in_dim), shape)
        elif init == "small_uniform":
            W = r.uniform(-1e-3, 1e-3, shape)
        else:
            raise ValueError(f"Unknown initializer: {init}")
        b = r.uniform(-1e-3, 1e-3, (1, self.units))
        return (DeviceArray.from_numpy(W.astype(np.float32), self.dtype),
                DeviceArray.from_numpy(b.astype(np.float32), "float32"))

    # ---------------- Layer lifecycle (:112-196) ----------------
    def build(self, input_shape: Tuple[int, ...]) -> None:
        super().build(input_shape)
        if len(input_shape) != 2:
            raise ValueError(f"Dense expects 2D input (batch, in_dim), got {input_shape}")
        _, in_dim = map(int, input_shape)
        self.W, self.b = self._init_weights(in_dim)
        self.dW = DeviceArray.zeros(self.W.shape, self.dtype)
        self.db = DeviceArray.zeros(self.b.shape, "float32")
        self.output_shape = (None, self.units)

    def call(self, x):
        if self.W is None or self.b is None:
            raise RuntimeError("Dense.call called before build")
        if dtype_of(x) != self.dtype:
            x = astype(x, self.dtype)
        save_z = bool(self.training) and (self.activation != "none")
        if save_z:
            out, Z = gemm_ops.forward(x, self.W, self.b, act=self.activation, with_bias=True,
                                      leaky_slope=self.leaky_slope, save_z=True, return_z=True)
            self.last_linear = Z
        else:
            out = gemm_ops.forward(x, self.W, self.b, act=self.activation, with_bias=True,
                                   leaky_slope=self.leaky_slope, save_z=False, return_z=False)
            self.last_linear = None
        self.last_input = x
        return out

    def backward(self, grad_output):
        if self.last_input is None or self.W is None or self.b is None:
            raise RuntimeError("Dense.backward called before forward/build")
        if dtype_of(grad_output) != self.dtype:
            grad_output = astype(grad_output, self.dtype)
        if self.last_linear is None:
            # Z was not kept (inference mode or act == none): recompute it (:218-228)
            _, Z = gemm_ops.forward(self.last_input, self.W, self.b, act="none", with_bias=True,
                                    save_z=True, return_z=True)
            self.last_linear = Z
        outs: Dict[str, object] = gemm_ops.backward(
            self.last_input, self.W, grad_output, self.last_linear, act=self.activation, with_bias=True,
            leaky_slope=self.leaky_slope, C=None, want_gA=True, want_gB=True, want_gBias=True)
        gW_new, gB_new, dx = outs.get("gB"), outs.get("gBias"), outs.get("gA")
        if gW_new is None or gB_new is None or dx is None:
            raise RuntimeError("native backward did not return all required grads")
        self._assign("dW", gW_new)
        self._assign("db", gB_new)
        return dx

    def _assign(self, attr: str, new) -> None:
        cur = getattr(self, attr)
        if (isinstance(cur, DeviceArray) and isinstance(new, DeviceArray) and cur.shape == new.shape
                and cur.dtype == new.dtype):
            cur[...] = new            # keep the gradient buffer (:249-256)
        else:
            setattr(self, attr, new)

    def compute_output_shape(self, input_shape: Tuple[int, ...]) -> Tuple[Optional[int], int]:
        if len(input_shape) != 2:
            raise ValueError(f"Dense expects 2D input, got {input_shape}")
        return (None if input_shape[0] is None else int(input_shape[0]), self.units)

    # ---------------- trainer helpers (:341-365) ----------------
    def param_triples(self):
        lname = type(self).__name__
        if self.W is not None:
            yield (self.W, self.dW, f"{lname}.W")
        if self.b is not None:
            yield (self.b, self.db, f"{lname}.b")

    def parameters(self):
        yield from self.param_triples()

    def grads(self):
        return [self.dW, self.db]

    def zero_grad(self) -> None:
        if self.dW is not None:
            self.dW.fill(0)
        if self.db is not None:
            self.db.fill(0)

    # ---------------- capture-safe, no-allocation paths (:368-493) ----------------
    def forward_into(self, x, out, z_out=None, *, stream: Optional[int] = None, work: Optional[dict] = None,
                     **kwargs) -> None:
        if self.W is None or self.b is None:
            raise RuntimeError("Dense.forward_into called before build")
        if dtype_of(x) != self.dtype:
            raise ValueError(f"[capture] x must be {self.dtype}")
        if not (is_c_contiguous(x) and is_c_contiguous(out)):
            raise ValueError("[capture] inputs/params/out must be C-contiguous")
        M, _ = array_info(x)[1]
        if tuple(array_info(out)[1]) != (M, self.units) or dtype_of(out) != self.dtype:
            raise ValueError(f"[capture] out must be {self.dtype}[{M},{self.units}] with C-contiguous layout")
        save_z = self.activation != "none"
        if save_z and z_out is None:
            key = ("dense_z", array_info(out)[0])
            buf = work.get(key) if work is not None else None
            if buf is None or tuple(array_info(buf)[1]) != (M, self.units) or dtype_of(buf) != self.dtype:
                buf = empty_like_2d(out)   # like the reference (:410-420): allocated once, then cached in `work`
                if work is not None:
                    work[key] = buf
            z_out = buf
        gemm_ops.forward_into(x, self.W, out=out, bias=self.b, act=self.activation, with_bias=True,
                              leaky_slope=self.leaky_slope, save_z=save_z, z_out=z_out, stream=stream)
        self.last_input = x
        self.last_linear = out if self.activation == "none" else (z_out if save_z else None)

    def backward_into(self, grad_output, gA_out, gW_out, gB_out, *, work_dZ, lt_workspace=None,
                      stream: Optional[int] = None, work: Optional[dict] = None, **kwargs) -> None:
        if self.last_input is None or self.last_linear is None:
            raise RuntimeError("[capture] need forward_into (with save_z) before backward_into")
        if dtype_of(grad_output) != self.dtype or not is_c_contiguous(grad_output):
            raise ValueError(f"[capture] grad_output must be C-contiguous {self.dtype}")
        M, in_dim = array_info(self.last_input)[1]
        if tuple(array_info(grad_output)[1]) != (M, self.units):
            raise ValueError("[capture] grad_output shape mismatch")
        if tuple(array_info(gA_out)[1]) != (M, in_dim) or dtype_of(gA_out) != self.dtype:
            raise ValueError(f"[capture] gA_out must be C-contiguous {self.dtype}[(M,in_dim)]")
        if tuple(array_info(gW_out)[1]) != (in_dim, self.units) or dtype_of(gW_out) != self.dtype:
            raise ValueError(f"[capture] gW_out must be C-contiguous {self.dtype}[(in_dim,units)]")
        if tuple(array_info(gB_out)[1]) != (1, self.units) or dtype_of(gB_out) != "float32":
            raise ValueError("[capture] gB_out must be C-contiguous float32[(1,units)]")
        if work_dZ is None:
            key = ("dense_dZ", array_info(self.last_linear)[0])
            buf = work.get(key) if work is not None else None
            if buf is None or tuple(array_info(buf)[1]) != (M, self.units) or dtype_of(buf) != "float32":
                buf = DeviceArray.empty((M, self.units), "float32")
                if work is not None:
                    work[key] = buf
            work_dZ = buf
        gemm_ops.backward_into(self.last_input, self.W, grad_output, self.last_linear, act=self.activation,
                               with_bias=True, leaky_slope=self.leaky_slope, C=None, gA_out=gA_out,
                               gB_out=gW_out, gBias_out=gB_out, gC_out=None, work_dZ=work_dZ,
                               lt_workspace=lt_workspace, stream=stream)
        self.dW = gW_out
        self.db = gB_out
