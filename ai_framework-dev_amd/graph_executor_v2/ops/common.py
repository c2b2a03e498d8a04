"""Array plumbing shared by the op glue (reference: python/graph_executor_v2/ops/common.py:28-97).

The reference takes CuPy float32 arrays only.  This build accepts any device
array that exposes its memory:

  - this package's ``DeviceArray``;
  - objects with ``__cuda_array_interface__`` (CuPy, Numba, ...);
  - torch tensors on the GPU (``data_ptr()``; also bfloat16, which has no
    array-interface type string).

and the storage types float32 (the reference's only one) plus float16 and
bfloat16 (additive: the operator computes them with fp32 accumulation).
Outputs the glue allocates are made by the same array library as the input
they are shaped after.  Nothing here runs arithmetic on the host.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

from .device_array import DeviceArray, dtype_name

FLOAT_DTYPES = ("float32", "float16", "bfloat16")


def _kind(x) -> str:
    if isinstance(x, DeviceArray):
        return "gev2"
    mod = type(x).__module__.split(".")[0]
    if mod == "torch":
        return "torch"
    if hasattr(x, "__cuda_array_interface__"):
        return mod or "cai"
    raise TypeError(f"expected a device array (DeviceArray, CuPy array, torch GPU tensor), got {type(x)}")


def array_info(x) -> Tuple[int, Tuple[int, ...], str, bool]:
    """(device pointer, shape, dtype name, C-contiguous) of a device array."""
    k = _kind(x)
    if k == "gev2":
        return x.ptr, x.shape, x.dtype, True
    if k == "torch":
        if not x.is_cuda:
            raise TypeError("torch tensor must live on the GPU")
        return int(x.data_ptr()), tuple(int(s) for s in x.shape), str(x.dtype).split(".")[-1], bool(x.is_contiguous())
    cai = x.__cuda_array_interface__
    shape = tuple(int(s) for s in cai["shape"])
    typestr = cai["typestr"]
    name = {"<f4": "float32", "<f2": "float16", "|u1": "uint8", "<u1": "uint8"}.get(typestr, typestr)
    strides = cai.get("strides")
    contig = True
    if strides is not None:
        item = {"float32": 4, "float16": 2, "uint8": 1}.get(name, 0)
        expect, acc = [], item
        for s in reversed(shape):
            expect.append(acc)
            acc *= s
        contig = tuple(strides) == tuple(reversed(expect))
    return int(cai["data"][0]), shape, name, contig


def dtype_of(x) -> str:
    return array_info(x)[2]


def is_c_contiguous(x) -> bool:
    return array_info(x)[3]


def assert_2d(x, name: str = "array", dtypes=FLOAT_DTYPES) -> Tuple[int, int]:
    """Shape check of assert_f32_2d (common.py:28-35), widened to the 16-bit storage types."""
    _, shape, dt, _ = array_info(x)
    if dt not in dtypes:
        raise TypeError(f"{name}: expected one of {dtypes}, got {dt}")
    if len(shape) != 2:
        raise ValueError(f"{name}: expected 2D, got shape={shape}")
    return int(shape[0]), int(shape[1])


def assert_f32_2d(x, name: str = "array") -> Tuple[int, int]:
    return assert_2d(x, name, ("float32",))


def _module(x):
    import importlib
    return importlib.import_module(type(x).__module__.split(".")[0])


def empty(shape, dtype: str, like=None) -> object:
    """New C-contiguous device array from the array library of `like` (DeviceArray if None)."""
    dt = dtype_name(dtype)
    if like is None:
        return DeviceArray.empty(shape, dt)
    k = _kind(like)
    if k == "gev2":
        return DeviceArray.empty(shape, dt)
    if k == "torch":
        torch = _module(like)
        return torch.empty(tuple(shape), dtype=getattr(torch, dt), device=like.device)
    return _module(like).empty(tuple(shape), dtype=dt)


def empty_like_2d(ref) -> object:
    _, shape, dt, _ = array_info(ref)
    return empty(shape, dt, ref)


def empty_2d(m: int, n: int, *, like, dtype: Optional[str] = None) -> object:
    return empty((int(m), int(n)), dtype or dtype_of(like), like)


def ascontiguous(x):
    """C-contiguous version of x (a copy if it is not), as the reference's as_tensor_2d does."""
    if is_c_contiguous(x):
        return x
    k = _kind(x)
    if k == "torch":
        return x.contiguous()
    return _module(x).ascontiguousarray(x)


def astype(x, dtype: str):
    dt = dtype_name(dtype)
    if dtype_of(x) == dt:
        return x
    k = _kind(x)
    if k == "gev2":
        return x.astype(dt)
    if k == "torch":
        return x.to(getattr(_module(x), dt))
    return x.astype(dt)


def reshape(x, shape):
    return x.reshape(tuple(shape))


def get_stream_ptr(stream: Optional[int] = None, like=None) -> Optional[int]:
    """None -> the array library's current stream (CuPy / torch), or the null stream (0)."""
    if stream is not None:
        return int(stream)
    if like is None:
        return 0
    k = _kind(like)
    if k == "torch":
        return int(_module(like).cuda.current_stream().cuda_stream)
    if k == "cupy":
        return int(_module(like).cuda.get_current_stream().ptr)
    return 0


def to_voidp_capsule(ptr: Optional[int]) -> object:
    """PyCapsule holding a stream pointer, or None for the null stream (common.py:46-62)."""
    if not ptr:
        return None
    new = ctypes.pythonapi.PyCapsule_New
    new.restype = ctypes.py_object
    new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
    return new(ctypes.c_void_p(ptr), None, None)


_ABI_DTYPE = {"float32": "F32", "float16": "F16", "bfloat16": "BF16"}


def as_tensor_2d(x):
    """Wrap a 2-D device array as a shim Tensor (common.py:65-88); non-contiguous arrays are
    copied to C order first."""
    from graph_executor_v2.ops import _ops_common as c

    M, N = assert_2d(x, "as_tensor_2d(x)")
    x = ascontiguous(x)
    ptr, _, dt, _ = array_info(x)
    return c.make_tensor_2d(ptr, [int(M), int(N)], getattr(c.DType, _ABI_DTYPE[dt]), c.Device.CUDA, 0)
