"""A minimal device array for the glue layer.

The reference's Python glue and layers take CuPy arrays
(graph_executor_v2/python/graph_executor_v2/ops/common.py:28-97).  CuPy is not
part of this build, so the glue accepts any device array that exposes its
pointer (``__cuda_array_interface__`` objects such as CuPy or Numba arrays,
torch tensors on the GPU) and ships this small array type for callers that have
none.  It owns one device allocation made through libgev2 (HBM), is always
C-contiguous, and supports what the glue and ``Dense`` need: allocation,
host upload/download, fill, device-to-device assignment and reshape views.
"""
from __future__ import annotations

from typing import Iterable, Optional, Tuple, Union

import numpy as np

from . import capi

# dtype name -> (itemsize, numpy storage dtype, C ABI dtype or None)
_DTYPES = {
    "float32": (4, np.float32, capi.F32),
    "float16": (2, np.float16, capi.F16),
    "bfloat16": (2, np.uint16, capi.BF16),
    "uint8": (1, np.uint8, None),
}


def dtype_name(dtype) -> str:
    """Normalise a dtype given as a name, a numpy dtype or a C ABI code."""
    if isinstance(dtype, str):
        d = dtype.lower()
        if d in ("bf16",):
            d = "bfloat16"
        if d in ("f32", "float"):
            d = "float32"
        if d in ("f16", "half"):
            d = "float16"
    elif isinstance(dtype, (int, np.integer)) and not isinstance(dtype, bool):
        d = {capi.F32: "float32", capi.F16: "float16", capi.BF16: "bfloat16"}.get(int(dtype), "")
    else:
        d = np.dtype(dtype).name
    if d not in _DTYPES:
        raise TypeError(f"unsupported dtype {dtype!r}")
    return d


class _Flags:
    c_contiguous = True
    f_contiguous = False


class DeviceArray:
    """C-contiguous device array (float32 / float16 / bfloat16 / uint8)."""

    flags = _Flags()

    def __init__(self, shape: Union[int, Iterable[int]], dtype="float32"):
        self.shape: Tuple[int, ...] = (int(shape),) if isinstance(shape, (int, np.integer)) else tuple(
            int(s) for s in shape)
        if any(s < 0 for s in self.shape):
            raise ValueError(f"negative dimension in {self.shape}")
        self.dtype = dtype_name(dtype)
        self.itemsize = _DTYPES[self.dtype][0]
        self._buf = capi.DeviceBuffer(max(self.nbytes, 1))   # reshape views share it
        self._ptr = self._buf.ptr

    # ---- properties ---------------------------------------------------------
    @property
    def size(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def ptr(self) -> int:
        return self._ptr

    @property
    def abi_dtype(self) -> Optional[int]:
        return _DTYPES[self.dtype][2]

    @property
    def __cuda_array_interface__(self):
        if self.dtype == "bfloat16":
            raise AttributeError("bfloat16 has no __cuda_array_interface__ type string")
        return {"shape": self.shape, "typestr": np.dtype(_DTYPES[self.dtype][1]).str,
                "data": (self._ptr, False), "strides": None, "version": 3}

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, ptr=0x{self._ptr:x})"

    # ---- construction -------------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype="float32") -> "DeviceArray":
        return cls(shape, dtype)

    @classmethod
    def zeros(cls, shape, dtype="float32") -> "DeviceArray":
        a = cls(shape, dtype)
        a.fill(0)
        return a

    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype=None) -> "DeviceArray":
        """Upload a host array; float data is rounded (RNE) to a 16-bit `dtype`."""
        a = np.asarray(a)
        d = dtype_name(dtype if dtype is not None else (a.dtype if a.dtype != np.float64 else "float32"))
        out = cls(a.shape, d)
        out.set(a)
        return out

    # ---- host transfer ------------------------------------------------------
    def set(self, a: np.ndarray) -> None:
        a = np.asarray(a)
        if a.shape != self.shape and a.size != self.size:
            raise ValueError(f"cannot set {a.shape} into {self.shape}")
        code = self.abi_dtype
        host = np.ascontiguousarray(capi.to_storage(a.astype(np.float32), code) if code is not None
                                    else a.astype(np.uint8))
        if host.nbytes:
            capi.check(capi.lib().gev2_memcpy_htod(self._ptr, host.ctypes.data, host.nbytes), "htod")

    def get(self) -> np.ndarray:
        """Download; 16-bit float data comes back as float32 values."""
        store = np.empty(self.shape, dtype=_DTYPES[self.dtype][1])
        if store.nbytes:
            capi.synchronize()
            capi.check(capi.lib().gev2_memcpy_dtoh(store.ctypes.data, self._ptr, store.nbytes), "dtoh")
        code = self.abi_dtype
        return capi.from_storage(store, code) if code is not None else store

    # ---- device operations --------------------------------------------------
    def fill(self, value) -> None:
        if value == 0:
            capi.check(capi.lib().gev2_memset(self._ptr, 0, self.nbytes), "memset")
        else:
            self.set(np.full(self.shape, value, dtype=np.float32))

    def copy_from(self, src: "DeviceArray", stream: int = 0) -> None:
        if not isinstance(src, DeviceArray) or src.nbytes != self.nbytes or src.dtype != self.dtype:
            raise ValueError(f"cannot copy {src!r} into {self!r}")
        if self.nbytes:
            capi.check(capi.lib().gev2_memcpy_dtod_async(self._ptr, src.ptr, self.nbytes, stream or None), "dtod")

    def __setitem__(self, key, value) -> None:
        if key is not Ellipsis and key != slice(None):
            raise IndexError("DeviceArray supports whole-array assignment only ([...] or [:])")
        if isinstance(value, DeviceArray):
            self.copy_from(value)
        elif np.isscalar(value):
            self.fill(value)
        else:
            self.set(np.asarray(value))

    def reshape(self, *shape) -> "DeviceArray":
        if len(shape) == 1 and not isinstance(shape[0], (int, np.integer)):
            shape = tuple(shape[0])
        shape = tuple(int(s) for s in shape)
        if -1 in shape:
            known = 1
            for s in shape:
                if s != -1:
                    known *= s
            shape = tuple(self.size // known if s == -1 else s for s in shape)
        n = 1
        for s in shape:
            n *= s
        if n != self.size:
            raise ValueError(f"cannot reshape {self.shape} to {shape}")
        view = DeviceArray.__new__(DeviceArray)
        view.shape, view.dtype, view.itemsize = shape, self.dtype, self.itemsize
        view._buf, view._ptr = self._buf, self._ptr
        return view

    def astype(self, dtype, copy: bool = True) -> "DeviceArray":
        """Convert through the host (the glue uses it only for inputs given in another dtype)."""
        d = dtype_name(dtype)
        if d == self.dtype and not copy:
            return self
        return DeviceArray.from_numpy(self.get(), d)

    def copy(self) -> "DeviceArray":
        out = DeviceArray(self.shape, self.dtype)
        out.copy_from(self)
        return out
