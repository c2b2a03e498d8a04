"""ctypes view of libgev2.so's C ABI (include/gev2_gemm.h).

Used by the Python glue, the tests and the benchmark.  Loading fails loudly
when the HIP library has not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgev2.so")

F32, F16, BF16 = 0, 1, 2
ACT = {"none": 0, "relu": 1, "leakyrelu": 2, "leaky_relu": 2, "lrelu": 2, "gelu": 3,
       "sigmoid": 4, "tanh": 5}
BIAS_NONE, BIAS_SCALAR, BIAS_PERM, BIAS_PERN = 0, 1, 2, 3

EXPORTED = [
    "gev2_gemm_fwd", "gev2_gemm_fwd_noalloc", "gev2_gemm_bwd", "gev2_gemm_fwd_workspace_size", "gev2_gemm_fwd_repeat", "gev2_gemm_bwd_repeat", "gev2_abi_version", "gev2_status_string",
    "gev2_last_error", "gev2_last_path", "gev2_device_count", "gev2_set_device",
    "gev2_get_device", "gev2_device_info", "gev2_malloc", "gev2_free", "gev2_memcpy_htod",
    "gev2_memcpy_dtoh", "gev2_memcpy_dtod_async", "gev2_memset", "gev2_stream_create",
    "gev2_stream_destroy", "gev2_stream_synchronize", "gev2_device_synchronize",
    "gev2_event_create", "gev2_event_destroy", "gev2_event_record", "gev2_event_synchronize",
    "gev2_event_elapsed_ms", "gev2_probe_mfma_bf16", "gev2_probe_hbm_read", "gev2_probe_hbm_write",
    "gev2_conv2d_fwd", "gev2_conv2d_bwd", "gev2_conv2d_last_error",
    "gev2_rnn_fwd", "gev2_rnn_bwd", "gev2_rnn_last_error",
    "gev2_sdpa_fwd", "gev2_sdpa_bwd", "gev2_sdpa_workspace_size", "gev2_sdpa_last_error",
    "gev2_graph_begin", "gev2_graph_end", "gev2_graph_launch", "gev2_graph_destroy",
    "gev2_gemm_bwd_workspace_size",
]


class FwdDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("act", ctypes.c_int32), ("bias_kind", ctypes.c_int32),
        ("trans_a", ctypes.c_int32), ("trans_b", ctypes.c_int32),
        ("leaky_slope", ctypes.c_float), ("alpha", ctypes.c_float), ("reserved0", ctypes.c_int32),
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("batch", ctypes.c_int64),
        ("A", ctypes.c_void_p), ("lda", ctypes.c_int64), ("stride_a", ctypes.c_int64),
        ("B", ctypes.c_void_p), ("ldb", ctypes.c_int64), ("stride_b", ctypes.c_int64),
        ("bias", ctypes.c_void_p), ("stride_bias", ctypes.c_int64),
        ("Y", ctypes.c_void_p), ("ldy", ctypes.c_int64), ("stride_y", ctypes.c_int64),
        ("Z", ctypes.c_void_p), ("ldz", ctypes.c_int64), ("stride_z", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


class BwdDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("act", ctypes.c_int32), ("bias_kind", ctypes.c_int32),
        ("leaky_slope", ctypes.c_float), ("alpha", ctypes.c_float), ("beta", ctypes.c_float),
        ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("batch", ctypes.c_int64),
        ("A", ctypes.c_void_p), ("lda", ctypes.c_int64), ("stride_a", ctypes.c_int64),
        ("B", ctypes.c_void_p), ("ldb", ctypes.c_int64), ("stride_b", ctypes.c_int64),
        ("gY", ctypes.c_void_p), ("ldgy", ctypes.c_int64), ("stride_gy", ctypes.c_int64),
        ("Z", ctypes.c_void_p), ("ldz", ctypes.c_int64), ("stride_z", ctypes.c_int64),
        ("gA", ctypes.c_void_p), ("ldga", ctypes.c_int64), ("stride_ga", ctypes.c_int64),
        ("gB", ctypes.c_void_p), ("ldgb", ctypes.c_int64), ("stride_gb", ctypes.c_int64),
        ("gC", ctypes.c_void_p), ("ldgc", ctypes.c_int64), ("stride_gc", ctypes.c_int64),
        ("gBias", ctypes.c_void_p), ("stride_gbias", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


_CONV_GEOM = [
    ("N", ctypes.c_int32), ("Cin", ctypes.c_int32), ("H", ctypes.c_int32), ("W", ctypes.c_int32),
    ("Cout", ctypes.c_int32), ("Kh", ctypes.c_int32), ("Kw", ctypes.c_int32),
    ("stride_h", ctypes.c_int32), ("stride_w", ctypes.c_int32), ("pad_h", ctypes.c_int32),
    ("pad_w", ctypes.c_int32), ("dil_h", ctypes.c_int32), ("dil_w", ctypes.c_int32), ("groups", ctypes.c_int32),
]


class Conv2dDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("act", ctypes.c_int32), ("leaky_slope", ctypes.c_float),
        ("save_z", ctypes.c_int32), *_CONV_GEOM,
        ("X", ctypes.c_void_p), ("Wt", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("Y", ctypes.c_void_p),
        ("Z", ctypes.c_void_p), ("col", ctypes.c_void_p), ("col_bytes", ctypes.c_int64),
    ]


class Conv2dBwdDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("act", ctypes.c_int32), ("leaky_slope", ctypes.c_float),
        ("reserved0", ctypes.c_int32), *_CONV_GEOM,
        ("X", ctypes.c_void_p), ("Wt", ctypes.c_void_p), ("dY", ctypes.c_void_p), ("Z", ctypes.c_void_p),
        ("dW", ctypes.c_void_p), ("dB", ctypes.c_void_p), ("dX", ctypes.c_void_p),
        ("col", ctypes.c_void_p), ("col_bytes", ctypes.c_int64), ("dcol", ctypes.c_void_p),
        ("dcol_bytes", ctypes.c_int64), ("gw", ctypes.c_void_p), ("gw_bytes", ctypes.c_int64),
        ("acc_b", ctypes.c_void_p), ("acc_b_bytes", ctypes.c_int64), ("acc_w", ctypes.c_void_p),
        ("dz", ctypes.c_void_p), ("dz_bytes", ctypes.c_int64),
    ]


_RNN_HEAD = [("dtype", ctypes.c_int32), ("act", ctypes.c_int32), ("leaky_slope", ctypes.c_float)]
_RNN_DIMS = [("N", ctypes.c_int32), ("T", ctypes.c_int32), ("I", ctypes.c_int32), ("H", ctypes.c_int32)]


class RnnDesc(ctypes.Structure):
    _fields_ = [
        *_RNN_HEAD, ("save_z", ctypes.c_int32), *_RNN_DIMS,
        ("X", ctypes.c_void_p), ("Wx", ctypes.c_void_p), ("Wh", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("h0", ctypes.c_void_p), ("Y", ctypes.c_void_p), ("Z", ctypes.c_void_p), ("xh", ctypes.c_void_p),
        ("wcat", ctypes.c_void_p), ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_int64),
    ]


class RnnBwdDesc(ctypes.Structure):
    _fields_ = [
        *_RNN_HEAD, ("reserved0", ctypes.c_int32), *_RNN_DIMS,
        ("X", ctypes.c_void_p), ("Wx", ctypes.c_void_p), ("Wh", ctypes.c_void_p), ("h0", ctypes.c_void_p),
        ("dY", ctypes.c_void_p), ("Z", ctypes.c_void_p), ("dWx", ctypes.c_void_p), ("dWh", ctypes.c_void_p),
        ("dB", ctypes.c_void_p), ("dh0", ctypes.c_void_p), ("dX", ctypes.c_void_p), ("xh", ctypes.c_void_p),
        ("g", ctypes.c_void_p), ("wcat", ctypes.c_void_p), ("dxh", ctypes.c_void_p), ("dwcat", ctypes.c_void_p),
        ("tmpw", ctypes.c_void_p), ("gb", ctypes.c_void_p), ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_int64),
    ]


MASK_NONE, MASK_I8, MASK_I32, MASK_F32 = 0, 1, 2, 3
_SDPA_HEAD = [("dtype", ctypes.c_int32), ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("M", ctypes.c_int32),
              ("N", ctypes.c_int32), ("D", ctypes.c_int32), ("scale", ctypes.c_float), ("causal", ctypes.c_int32),
              ("dropout_p", ctypes.c_float), ("mask_kind", ctypes.c_int32), ("mask", ctypes.c_void_p)]


class SdpaDesc(ctypes.Structure):
    _fields_ = [
        *_SDPA_HEAD, ("Q", ctypes.c_void_p), ("K", ctypes.c_void_p), ("V", ctypes.c_void_p), ("Y", ctypes.c_void_p),
        ("lse", ctypes.c_void_p), ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("seed", ctypes.c_uint64), ("scale_in_train", ctypes.c_int32), ("reserved1", ctypes.c_int32),
    ]


class SdpaBwdDesc(ctypes.Structure):
    _fields_ = [
        *_SDPA_HEAD, ("Q", ctypes.c_void_p), ("K", ctypes.c_void_p), ("V", ctypes.c_void_p), ("dY", ctypes.c_void_p),
        ("dQ", ctypes.c_void_p), ("dK", ctypes.c_void_p), ("dV", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64), ("seed", ctypes.c_uint64), ("scale_in_train", ctypes.c_int32),
        ("reserved1", ctypes.c_int32),
    ]


_lib: Optional[ctypes.CDLL] = None


class GemmError(RuntimeError):
    def __init__(self, status: int, where: str, msg: str):
        super().__init__(f"[{where}] status {status}: {msg}")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load libgev2.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} not found: build it with `python ai_framework-dev_amd/build.py` "
            "(the GEMM operator has no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    L.gev2_gemm_fwd.argtypes = [ctypes.POINTER(FwdDesc), vp]
    L.gev2_gemm_fwd_noalloc.argtypes = [ctypes.POINTER(FwdDesc), vp]
    L.gev2_gemm_bwd.argtypes = [ctypes.POINTER(BwdDesc), vp]
    L.gev2_gemm_fwd_workspace_size.argtypes = [ctypes.POINTER(FwdDesc)]
    L.gev2_gemm_fwd_workspace_size.restype = i64
    L.gev2_gemm_fwd_repeat.argtypes = [ctypes.POINTER(FwdDesc), i32, i32, vp]
    L.gev2_gemm_bwd_repeat.argtypes = [ctypes.POINTER(BwdDesc), i32, i32, vp]
    for f in ("gev2_status_string",):
        getattr(L, f).restype = ctypes.c_char_p
        getattr(L, f).argtypes = [i32]
    for f in ("gev2_last_error", "gev2_last_path"):
        getattr(L, f).restype = ctypes.c_char_p
        getattr(L, f).argtypes = []
    L.gev2_device_count.argtypes = [ctypes.POINTER(i32)]
    L.gev2_set_device.argtypes = [i32]
    L.gev2_get_device.argtypes = [ctypes.POINTER(i32)]
    L.gev2_device_info.argtypes = [i32, ctypes.c_char_p, sz, ctypes.POINTER(i32), ctypes.POINTER(i32)]
    L.gev2_malloc.argtypes = [ctypes.POINTER(vp), sz]
    L.gev2_free.argtypes = [vp]
    L.gev2_memcpy_htod.argtypes = [vp, vp, sz]
    L.gev2_memcpy_dtoh.argtypes = [vp, vp, sz]
    L.gev2_memcpy_dtod_async.argtypes = [vp, vp, sz, vp]
    L.gev2_memset.argtypes = [vp, i32, sz]
    L.gev2_stream_create.argtypes = [ctypes.POINTER(vp)]
    L.gev2_stream_destroy.argtypes = [vp]
    L.gev2_stream_synchronize.argtypes = [vp]
    L.gev2_event_create.argtypes = [ctypes.POINTER(vp)]
    L.gev2_event_destroy.argtypes = [vp]
    L.gev2_event_record.argtypes = [vp, vp]
    L.gev2_event_synchronize.argtypes = [vp]
    L.gev2_event_elapsed_ms.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
    L.gev2_probe_mfma_bf16.argtypes = [i32, i32, vp]
    L.gev2_probe_hbm_read.argtypes = [vp, sz, i32, i32, i32, i32, vp]
    L.gev2_probe_hbm_write.argtypes = [vp, sz, i32, i32, i32, i32, vp]
    L.gev2_conv2d_fwd.argtypes = [ctypes.POINTER(Conv2dDesc), vp]
    L.gev2_conv2d_bwd.argtypes = [ctypes.POINTER(Conv2dBwdDesc), vp]
    L.gev2_conv2d_last_error.restype = ctypes.c_char_p
    L.gev2_conv2d_last_error.argtypes = []
    L.gev2_rnn_fwd.argtypes = [ctypes.POINTER(RnnDesc), vp]
    L.gev2_rnn_bwd.argtypes = [ctypes.POINTER(RnnBwdDesc), vp]
    L.gev2_rnn_last_error.restype = ctypes.c_char_p
    L.gev2_rnn_last_error.argtypes = []
    L.gev2_gemm_bwd_workspace_size.restype = ctypes.c_int64
    L.gev2_gemm_bwd_workspace_size.argtypes = [ctypes.POINTER(BwdDesc)]
    L.gev2_graph_begin.argtypes = [vp]
    L.gev2_graph_end.argtypes = [vp, ctypes.POINTER(ctypes.c_void_p)]
    L.gev2_graph_launch.argtypes = [vp, vp]
    L.gev2_graph_destroy.argtypes = [vp]
    L.gev2_sdpa_fwd.argtypes = [ctypes.POINTER(SdpaDesc), vp]
    L.gev2_sdpa_bwd.argtypes = [ctypes.POINTER(SdpaBwdDesc), vp]
    L.gev2_sdpa_workspace_size.restype = ctypes.c_int64
    L.gev2_sdpa_workspace_size.argtypes = [ctypes.POINTER(SdpaDesc), ctypes.c_int]
    L.gev2_sdpa_last_error.restype = ctypes.c_char_p
    L.gev2_sdpa_last_error.argtypes = []
    _lib = L
    return L


def check(status: int, where: str) -> None:
    if status != 0:
        L = lib()
        raise GemmError(status, where, (L.gev2_last_error() or b"").decode()
                        or L.gev2_status_string(status).decode())


def check_conv(status: int, where: str) -> None:
    if status != 0:
        L = lib()
        raise GemmError(status, where, (L.gev2_conv2d_last_error() or b"").decode()
                        or L.gev2_status_string(status).decode())


def check_rnn(status: int, where: str) -> None:
    if status != 0:
        L = lib()
        raise GemmError(status, where, (L.gev2_rnn_last_error() or b"").decode()
                        or L.gev2_status_string(status).decode())


def check_sdpa(status: int, where: str) -> None:
    if status != 0:
        L = lib()
        raise GemmError(status, where, (L.gev2_sdpa_last_error() or b"").decode()
                        or L.gev2_status_string(status).decode())


def last_path() -> str:
    return lib().gev2_last_path().decode()


# ---------------------------------------------------------------------------
# Device buffers
# ---------------------------------------------------------------------------
def _np_storage(dtype: int):
    return {F32: np.float32, F16: np.float16, BF16: np.uint16}[dtype]


class DeviceBuffer:
    """Owning device allocation with numpy upload/download."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().gev2_malloc(ctypes.byref(p), max(self.nbytes, 1)), "gev2_malloc")
        self.ptr = int(p.value)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(lib().gev2_memcpy_htod(b.ptr, a.ctypes.data, a.nbytes), "htod")
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().gev2_memcpy_htod(self.ptr, a.ctypes.data, a.nbytes), "htod")

    def download(self, shape, np_dtype) -> np.ndarray:
        out = np.empty(shape, dtype=np_dtype)
        if out.nbytes:
            check(lib().gev2_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes), "dtoh")
        return out

    def fill_bytes(self, value: int) -> None:
        check(lib().gev2_memset(self.ptr, value, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            lib().gev2_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize() -> None:
    check(lib().gev2_device_synchronize(), "sync")


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().gev2_stream_create(ctypes.byref(p)), "stream_create")
        self.ptr = int(p.value)

    def synchronize(self) -> None:
        check(lib().gev2_stream_synchronize(self.ptr), "stream_sync")

    def destroy(self) -> None:
        if self.ptr:
            lib().gev2_stream_destroy(self.ptr)
            self.ptr = 0


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().gev2_event_create(ctypes.byref(p)), "event_create")
        self.ptr = int(p.value)

    def record(self, stream: int = 0) -> None:
        check(lib().gev2_event_record(self.ptr, stream), "event_record")

    def synchronize(self) -> None:
        check(lib().gev2_event_synchronize(self.ptr), "event_sync")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().gev2_event_elapsed_ms(ctypes.byref(ms), self.ptr, end.ptr), "elapsed")
        return float(ms.value)

    def destroy(self) -> None:
        if self.ptr:
            lib().gev2_event_destroy(self.ptr)
            self.ptr = 0


def device_info(device: int = 0) -> Tuple[str, int, int]:
    name = ctypes.create_string_buffer(256)
    cu, clk = ctypes.c_int(), ctypes.c_int()
    check(lib().gev2_device_info(device, name, 256, ctypes.byref(cu), ctypes.byref(clk)), "info")
    return name.value.decode(), cu.value, clk.value


def device_count() -> int:
    n = ctypes.c_int()
    st = lib().gev2_device_count(ctypes.byref(n))
    return n.value if st == 0 else 0


# ---------------------------------------------------------------------------
# Operator calls
# ---------------------------------------------------------------------------
def fwd_desc(*, dtype: int, M: int, N: int, K: int, A: int, B: int, Y: int,
             bias: int = 0, bias_kind: int = BIAS_NONE, Z: int = 0, act="none",
             leaky_slope: float = 0.01, alpha: float = 1.0, trans_a: bool = False,
             trans_b: bool = False, batch: int = 1, lda: int = 0, ldb: int = 0, ldy: int = 0,
             ldz: int = 0, stride_a: int = 0, stride_b: int = 0, stride_y: int = 0,
             stride_z: int = 0, stride_bias: int = 0, workspace: int = 0,
             workspace_bytes: int = 0) -> FwdDesc:
    d = FwdDesc()
    d.dtype, d.act, d.bias_kind = dtype, ACT[act] if isinstance(act, str) else int(act), bias_kind
    d.trans_a, d.trans_b = int(trans_a), int(trans_b)
    d.leaky_slope, d.alpha = leaky_slope, alpha
    d.M, d.N, d.K, d.batch = M, N, K, batch
    d.A, d.lda, d.stride_a = A or None, lda, stride_a
    d.B, d.ldb, d.stride_b = B or None, ldb, stride_b
    d.bias, d.stride_bias = bias or None, stride_bias
    d.Y, d.ldy, d.stride_y = Y or None, ldy, stride_y
    d.Z, d.ldz, d.stride_z = Z or None, ldz, stride_z
    d.workspace, d.workspace_bytes = workspace or None, workspace_bytes
    return d


def fwd_workspace_size(**kw) -> int:
    """Scratch bytes gev2_gemm_fwd needs for these arguments (0: none)."""
    d = fwd_desc(**kw)
    n = lib().gev2_gemm_fwd_workspace_size(ctypes.byref(d))
    if n < 0:
        raise GemmError(1, "gev2_gemm_fwd_workspace_size", lib().gev2_last_error().decode())
    return n


def bwd_desc(*, dtype: int, M: int, N: int, K: int, A: int, B: int, gY: int, Z: int,
             gA: int = 0, gB: int = 0, gC: int = 0, gBias: int = 0, bias_kind: int = BIAS_NONE,
             act="none", leaky_slope: float = 0.01, alpha: float = 1.0, beta: float = 0.0,
             batch: int = 1, lda: int = 0, ldb: int = 0, ldgy: int = 0, ldz: int = 0,
             ldga: int = 0, ldgb: int = 0, ldgc: int = 0, stride_a: int = 0, stride_b: int = 0,
             stride_gy: int = 0, stride_z: int = 0, stride_ga: int = 0, stride_gb: int = 0,
             stride_gc: int = 0, stride_gbias: int = 0, workspace: int = 0,
             workspace_bytes: int = 0) -> BwdDesc:
    d = BwdDesc()
    d.dtype, d.act, d.bias_kind = dtype, ACT[act] if isinstance(act, str) else int(act), bias_kind
    d.leaky_slope, d.alpha, d.beta = leaky_slope, alpha, beta
    d.M, d.N, d.K, d.batch = M, N, K, batch
    d.A, d.lda, d.stride_a = A or None, lda, stride_a
    d.B, d.ldb, d.stride_b = B or None, ldb, stride_b
    d.gY, d.ldgy, d.stride_gy = gY or None, ldgy, stride_gy
    d.Z, d.ldz, d.stride_z = Z or None, ldz, stride_z
    d.gA, d.ldga, d.stride_ga = gA or None, ldga, stride_ga
    d.gB, d.ldgb, d.stride_gb = gB or None, ldgb, stride_gb
    d.gC, d.ldgc, d.stride_gc = gC or None, ldgc, stride_gc
    d.gBias, d.stride_gbias = gBias or None, stride_gbias
    d.workspace, d.workspace_bytes = workspace or None, workspace_bytes
    return d


def gemm_fwd(*, stream: int = 0, **kw) -> None:
    d = fwd_desc(**kw)
    check(lib().gev2_gemm_fwd(ctypes.byref(d), stream or None), "gev2_gemm_fwd")


def gemm_fwd_noalloc(*, stream: int = 0, **kw) -> None:
    """gev2_gemm_fwd_noalloc: the forward with its split-K scratch in the library's fixed
    device array (no allocation; desc.workspace ignored)."""
    d = fwd_desc(**kw)
    check(lib().gev2_gemm_fwd_noalloc(ctypes.byref(d), stream or None), "gev2_gemm_fwd_noalloc")


def gemm_bwd(*, stream: int = 0, **kw) -> None:
    d = bwd_desc(**kw)
    check(lib().gev2_gemm_bwd(ctypes.byref(d), stream or None), "gev2_gemm_bwd")


def gemm_fwd_repeat(descs, reps: int, stream: int = 0) -> None:
    """reps back-to-back forward calls issued from C, cycling through descs."""
    arr = (FwdDesc * len(descs))(*descs)
    check(lib().gev2_gemm_fwd_repeat(arr, len(descs), reps, stream or None), "gev2_gemm_fwd_repeat")


def gemm_bwd_repeat(descs, reps: int, stream: int = 0) -> None:
    arr = (BwdDesc * len(descs))(*descs)
    check(lib().gev2_gemm_bwd_repeat(arr, len(descs), reps, stream or None), "gev2_gemm_bwd_repeat")


# ---------------------------------------------------------------------------
# Host-side storage conversion (bf16 has no numpy dtype: bit patterns in uint16)
# ---------------------------------------------------------------------------
def to_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    """float array -> host array in the device storage format (RNE rounding)."""
    x32 = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == F32:
        return x32
    if dtype == F16:
        return x32.astype(np.float16)
    u = x32.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_storage(a: np.ndarray, dtype: int) -> np.ndarray:
    """host array in storage format -> float32 values."""
    if dtype == F32:
        return np.asarray(a, dtype=np.float32)
    if dtype == F16:
        return np.asarray(a, dtype=np.float16).astype(np.float32)
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def storage_dtype(dtype: int):
    return _np_storage(dtype)


def elem_bytes(dtype: int) -> int:
    return 4 if dtype == F32 else 2
