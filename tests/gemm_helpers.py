"""Shared helpers for the parity tests: seeded inputs, device round trips through
the C ABI, and the tolerance bounds (oracle/gemm_oracle.py is the checker)."""
from __future__ import annotations

import numpy as np

from oracle import gemm_oracle as O

F32, F16, BF16 = O.DT_F32, O.DT_F16, O.DT_BF16
DT_NAMES = {F32: "f32", F16: "f16", BF16: "bf16"}
# unit roundoff of the output storage type (one RNE rounding)
U_OUT = {F32: 2.0 ** -24, F16: 2.0 ** -11, BF16: 2.0 ** -8}
U_ACC = 2.0 ** -24   # fp32 accumulation
# absolute error of one RNE rounding in the subnormal range: half the subnormal spacing
# (fp16 2^-24, bf16 2^-133, fp32 2^-149), where the relative bound u*|x| no longer holds
TINY_OUT = {F32: 2.0 ** -150, F16: 2.0 ** -25, BF16: 2.0 ** -134}


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def rounded(x, dtype):
    return O.round_to(x, dtype)


def fwd_bound(X, W, K, dtype, bias_vals=None):
    """Componentwise bound on |Z_dev - Z_64| for inputs already in storage precision:
    fp32 accumulation over K terms (gamma_K) plus one rounding of the stored result."""
    absprod = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64))
    b = 1.01 * K * U_ACC * absprod
    if bias_vals is not None:
        b = b + U_ACC * np.abs(bias_vals)
    return b


def act_lipschitz(act) -> float:
    a = O.parse_act(act)
    return {O.ACT_NONE: 1.0, O.ACT_RELU: 1.0, O.ACT_LEAKY: 1.0, O.ACT_GELU: 1.13,
            O.ACT_SIGMOID: 0.25, O.ACT_TANH: 1.0}[a]


def assert_close(dev, ref, bound, what, rel_norm=None):
    dev = np.asarray(dev, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(dev - ref)
    bad = ~(err <= bound)          # NaN counts as a failure
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements outside the bound; worst at {i}: "
            f"dev={dev[i]!r} ref={ref[i]!r} err={err[i]:.3e} bound={np.asarray(bound)[i] if np.ndim(bound) else bound:.3e}")
    if rel_norm is not None:
        den = np.linalg.norm(ref)
        if den > 0:
            rel = np.linalg.norm(dev - ref) / den
            assert rel <= rel_norm, f"{what}: normwise relative error {rel:.3e} > {rel_norm}"


class Dev:
    """Upload numpy arrays (in storage format) through the C ABI; free at close."""

    def __init__(self, capi):
        self.capi = capi
        self.bufs = []

    def put(self, host_storage: np.ndarray) -> int:
        b = self.capi.DeviceBuffer.from_numpy(host_storage)
        self.bufs.append(b)
        return b.ptr

    def empty(self, nbytes: int, fill: int = 0x7f) -> int:
        b = self.capi.DeviceBuffer(nbytes)
        b.fill_bytes(fill)   # poison: untouched outputs show up as huge values
        self.bufs.append(b)
        return b.ptr

    def get(self, ptr: int, shape, dtype) -> np.ndarray:
        b = next(x for x in self.bufs if x.ptr == ptr)
        raw = b.download(shape, self.capi.storage_dtype(dtype))
        return self.capi.from_storage(raw, dtype)

    def get_f32(self, ptr: int, shape) -> np.ndarray:
        b = next(x for x in self.bufs if x.ptr == ptr)
        return b.download(shape, np.float32)

    def close(self):
        for b in self.bufs:
            b.free()
        self.bufs = []


def make_fwd_inputs(seed, M, N, K, dtype, bias_kind, dist="normal"):
    g = rng(seed)
    if dist == "normal":
        X = g.standard_normal((M, K)) / np.sqrt(max(K, 1))
        W = g.standard_normal((K, N))
    else:
        X = g.uniform(-1, 1, (M, K)) / np.sqrt(max(K, 1))
        W = g.uniform(-1, 1, (K, N))
    X = rounded(X, dtype)
    W = rounded(W, dtype)
    nb = {O.BIAS_NONE: 0, O.BIAS_SCALAR: 1, O.BIAS_PERM: M, O.BIAS_PERN: N}[bias_kind]
    b = (0.5 * g.standard_normal(nb)).astype(np.float32) if nb else None
    return X, W, b


def run_fwd(capi, dev: Dev, X, W, b, bias_kind, act, dtype, save_z=True, slope=0.01, alpha=1.0):
    M, K = X.shape
    N = W.shape[1]
    es = capi.elem_bytes(dtype)
    pX = dev.put(capi.to_storage(X, dtype))
    pW = dev.put(capi.to_storage(W, dtype))
    pb = dev.put(b) if b is not None else 0
    pY = dev.empty(M * N * es)
    pZ = dev.empty(M * N * es) if save_z else 0
    capi.gemm_fwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb,
                  bias_kind=bias_kind if b is not None else 0, act=act, leaky_slope=slope,
                  alpha=alpha)
    path = capi.last_path()
    capi.synchronize()
    Y = dev.get(pY, (M, N), dtype)
    Z = dev.get(pZ, (M, N), dtype) if save_z else None
    return Y, Z, path
