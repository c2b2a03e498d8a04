"""CPU oracle for graph_executor_v2's fused GEMM + bias + activation operator.

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP path is
compared against; it is imported by ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` and nowhere else.  The product path
(``ai_framework-dev_amd``) never imports, calls or falls back to it.

It restates, in float64 NumPy, the host math of the reference:

* activation forward   -- ``backends/cuda/ops/_common/shim/activations.hpp:14-30``
  (GELU is the tanh form with c = 0.7978845608, k1 = 0.044715 and the inner
  argument ``fmaf(c*k1, x^3, c*x)``; Sigmoid is the branch-stable form)
* activation derivative -- ``activations.hpp:45-70`` (LeakyReLU' is ``slope`` at
  z == 0; the GELU derivative clamps tanh to +-0.999999)
* epilogue             -- ``_common/shim/traits.hpp:43-71``
  (pre = alpha*acc + bias; Z = pre; Y = act(pre))
* bias-kind inference  -- ``_common/shim/bias.hpp:70-78`` then
  ``backends/cuda/ops/gemm/launcher.cu:47-77``
* backward             -- ``gemm/kernels/regemm_backward.cu:91-130,271-291``
  (gZ = gY * act'(Z); gA = alpha*gZ B^T; gB = alpha*A^T gZ; gC = beta*gZ;
  gBias = sum of gZ over rows / columns / everything for PerN / PerM / Scalar)
* the reference's own NumPy test math -- ``tests/cuda_pyd_test/smoke_gemm_binding.py:84-123``
* batched slices       -- ``backends/cuda/ops/sdpa/launcher.cu:166-170``
  (slice (b,h) starts at ((b*H+h)*rows*cols))
* 2-D convolution      -- ``backends/cuda/ops/conv2d/launcher.cu:106-459`` and
  ``kernels.cu:12-87`` (output size, zero padding, dilation; column order
  (c*Kh + kh)*Kw + kw; bias per output channel; dB summed over all images),
  written here as direct sums over the kernel window, not as im2col
* attention (SDPA)      -- ``backends/cuda/ops/sdpa/launcher.cu:129-747``
  (S = scale Q K^T, scale 0 -> 1/sqrt(D); external mask [B,1,M,N] then causal,
  each adding -1e9 in fp32 (F32 masks add their value); softmax over keys;
  Y = P V; backward dV = P^T dY, dS = P (dP - rowsum(dP P)) zeroed where
  masked, dQ = scale dS K, dK = scale dS^T Q; dropout with the stateless
  splitmix64 stream of ``dropout/kernels.cu:8-45``, P dropped in Y = P V and
  in dV, dP dropped before dS)
* Elman RNN             -- ``backends/cuda/ops/rnn/launcher.cu:129-383``
  (h_t = act(X_t Wx + h_{t-1} Wh + b); backward through time with
  dh_next = dZ_t Wh^T; dB summed over all steps)

Parity pins (what keeps this restatement honest) live in ``tests/test_oracle.py``:
exact-integer brute force for the GEMMs, the convolution and the RNN recurrence (pure-Python loops), central finite
differences for every activation derivative and for the GEMM, conv and RNN backwards (a scalar loss), the erf form of GELU
for the tanh approximation, and the C restatement in ``gemm_oracle.c`` (fp32,
sequential-k ``fmaf`` -- the reference's own small-kernel order).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np

# ---------------------------------------------------------------------------
# Enum values (ABI anchors of the reference: _common/shim/enums.hpp:10-24,
# ai_device.hpp:14-27)
# ---------------------------------------------------------------------------
ACT_NONE, ACT_RELU, ACT_LEAKY, ACT_GELU, ACT_SIGMOID, ACT_TANH = 0, 1, 2, 3, 4, 5
BIAS_NONE, BIAS_SCALAR, BIAS_PERM, BIAS_PERN = 0, 1, 2, 3
DT_F32, DT_F16, DT_BF16 = 0, 1, 2

GELU_C = 0.7978845608      # activations.hpp:19
GELU_K1 = 0.044715         # activations.hpp:20
GELU_TH_CLAMP = 0.999999   # activations.hpp:55-56

_ACT_NAMES = {
    "none": ACT_NONE, "relu": ACT_RELU, "leakyrelu": ACT_LEAKY,
    "leaky_relu": ACT_LEAKY, "lrelu": ACT_LEAKY, "gelu": ACT_GELU,
    "sigmoid": ACT_SIGMOID, "tanh": ACT_TANH,
}


def parse_act(act) -> int:
    """String or int -> ActKind value (gemm_pybind.cpp:57-69 accepts these names)."""
    if isinstance(act, (int, np.integer)):
        return int(act)
    k = str(act).lower()
    if k not in _ACT_NAMES:
        raise ValueError(f"unknown act: {act}")
    return _ACT_NAMES[k]


# ---------------------------------------------------------------------------
# Activations (float64)
# ---------------------------------------------------------------------------
def act_forward(z, act, slope: float = 0.01) -> np.ndarray:
    """act_apply<AK>(x, leaky) -- activations.hpp:14-39."""
    a = parse_act(act)
    z = np.asarray(z, dtype=np.float64)
    if a == ACT_NONE:
        return z.copy()
    if a == ACT_RELU:
        return np.where(z > 0.0, z, 0.0)
    if a == ACT_LEAKY:
        return np.where(z > 0.0, z, slope * z)
    if a == ACT_GELU:
        t = (GELU_C * GELU_K1) * (z * z * z) + GELU_C * z
        return 0.5 * z * (1.0 + np.tanh(t))
    if a == ACT_SIGMOID:
        # branch-stable form, activations.hpp:25-29
        e = np.exp(-np.abs(z))
        return np.where(z >= 0.0, 1.0 / (1.0 + e), e / (1.0 + e))
    if a == ACT_TANH:
        return np.tanh(z)
    raise ValueError(f"bad act {act}")


def act_deriv(z, act, slope: float = 0.01) -> np.ndarray:
    """act_deriv<AK>(x, leaky) -- activations.hpp:45-70."""
    a = parse_act(act)
    z = np.asarray(z, dtype=np.float64)
    if a == ACT_NONE:
        return np.ones_like(z)
    if a == ACT_RELU:
        return np.where(z > 0.0, 1.0, 0.0)
    if a == ACT_LEAKY:
        return np.where(z > 0.0, 1.0, slope)        # slope at z == 0 (:47)
    if a == ACT_GELU:
        x2 = z * z
        t = (GELU_C * GELU_K1) * (x2 * z) + GELU_C * z
        th = np.clip(np.tanh(t), -GELU_TH_CLAMP, GELU_TH_CLAMP)
        sech2 = 1.0 - th * th
        dt = GELU_C * (1.0 + 3.0 * GELU_K1 * x2)
        return 0.5 * (1.0 + th) + 0.5 * z * sech2 * dt
    if a == ACT_SIGMOID:
        s = act_forward(z, ACT_SIGMOID)
        return s * (1.0 - s)
    if a == ACT_TANH:
        th = np.tanh(z)
        return 1.0 - th * th
    raise ValueError(f"bad act {act}")


# ---------------------------------------------------------------------------
# Bias-kind inference (host logic)
# ---------------------------------------------------------------------------
def infer_bias_kind_1d_lenMN(shape: Optional[Sequence[int]], M: int, N: int) -> int:
    """bias.hpp:70-78: only rank-1; len 1 -> Scalar, == N -> PerN, == M -> PerM."""
    if shape is None or len(shape) != 1:
        return BIAS_NONE
    n = int(shape[0])
    if n == 1:
        return BIAS_SCALAR
    if n == N:
        return BIAS_PERN
    if n == M:
        return BIAS_PERM
    return BIAS_NONE


def infer_bias_kind_fallback(shape: Optional[Sequence[int]], M: int, N: int) -> int:
    """gemm/launcher.cu:47-71."""
    if shape is None:
        return BIAS_NONE
    s = [int(v) for v in shape]
    if any(v < 0 for v in s):
        return BIAS_NONE
    numel = 1
    for v in s:
        numel *= v
    if numel == 0:
        return BIAS_NONE
    if len(s) == 2 and s[0] == 1 and s[1] == N:
        return BIAS_PERN
    if len(s) == 1 and s[0] == N:
        return BIAS_PERN
    if len(s) == 2 and s[0] == M and s[1] == 1:
        return BIAS_PERM
    if len(s) == 1 and s[0] == M:
        return BIAS_PERM
    if (len(s) == 2 and s[0] == 1 and s[1] == 1) or (len(s) == 1 and s[0] == 1):
        return BIAS_SCALAR
    if numel == N:
        return BIAS_PERN
    if numel == M:
        return BIAS_PERM
    if numel == 1:
        return BIAS_SCALAR
    return BIAS_NONE


def decide_bias_kind(shape: Optional[Sequence[int]], M: int, N: int) -> int:
    """gemm/launcher.cu:73-77: strict 1-D rule first, then the fallback."""
    k = infer_bias_kind_1d_lenMN(shape, M, N)
    if k != BIAS_NONE:
        return k
    return infer_bias_kind_fallback(shape, M, N)


def bias_add(pre: np.ndarray, bias, kind: int) -> np.ndarray:
    """Broadcast a bias of the given kind onto pre[M,N] (bias.hpp:155-176)."""
    if bias is None or kind == BIAS_NONE:
        return pre
    b = np.asarray(bias, dtype=np.float64).reshape(-1)
    if kind == BIAS_SCALAR:
        return pre + b[0]
    if kind == BIAS_PERN:
        return pre + b[None, : pre.shape[1]]
    if kind == BIAS_PERM:
        return pre + b[: pre.shape[0], None]
    raise ValueError(kind)


# ---------------------------------------------------------------------------
# Forward / backward (float64)
# ---------------------------------------------------------------------------
def gemm_forward(A, B, bias=None, bias_kind: Optional[int] = None, act="none",
                 slope: float = 0.01, alpha: float = 1.0,
                 trans_a: bool = False, trans_b: bool = False
                 ) -> Tuple[np.ndarray, np.ndarray]:
    """Z = alpha * op(A) @ op(B) + bias; Y = act(Z).  Returns (Y, Z), float64."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    if trans_a:
        A = A.T
    if trans_b:
        B = B.T
    acc = A @ B
    pre = acc if alpha == 1.0 else alpha * acc          # traits.hpp:44
    if bias is not None:
        if bias_kind is None:
            bias_kind = decide_bias_kind(np.shape(bias), A.shape[0], B.shape[1])
        pre = bias_add(pre, bias, bias_kind)
    return act_forward(pre, act, slope), pre


def gemm_backward(A, B, gY, Z, act="none", slope: float = 0.01,
                  bias_kind: int = BIAS_NONE, alpha: float = 1.0,
                  beta: float = 0.0) -> dict:
    """regemm_backward.cu:91-130 (epilogue) + :271-291 (the two GEMMs), float64."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    gZ = np.asarray(gY, dtype=np.float64) * act_deriv(Z, act, slope)
    out = {
        "gZ": gZ,
        "gA": alpha * (gZ @ B.T),
        "gB": alpha * (A.T @ gZ),
        "gC": beta * gZ,
    }
    if bias_kind == BIAS_PERN:
        out["gBias"] = gZ.sum(axis=0)
    elif bias_kind == BIAS_PERM:
        out["gBias"] = gZ.sum(axis=1)
    elif bias_kind == BIAS_SCALAR:
        out["gBias"] = np.array([gZ.sum()])
    else:
        out["gBias"] = None
    return out


def slice_offset(b: int, h: int, H: int, rows: int, cols: int) -> int:
    """Flat element offset of slice (b,h) -- sdpa/launcher.cu:166-170."""
    return (b * H + h) * rows * cols


def gemm_forward_batched(A_flat, B_flat, batch: int, M: int, N: int, K: int,
                         sA: int, sB: int, lda: int, ldb: int,
                         trans_b: bool = False, alpha: float = 1.0,
                         bias=None, bias_kind: int = BIAS_NONE, sBias: int = 0,
                         act="none", slope: float = 0.01
                         ) -> Tuple[np.ndarray, np.ndarray]:
    """Batched strided form over flat buffers, one slice at a time.

    Slice i of A starts at ``i*sA`` (row-major, leading dimension lda);
    B slice i at ``i*sB`` and is [K,N] (ldb) or, with trans_b, [N,K] (ldb).
    Returns (Y, Z) as [batch, M, N] float64 arrays.
    """
    A_flat = np.asarray(A_flat, dtype=np.float64).reshape(-1)
    B_flat = np.asarray(B_flat, dtype=np.float64).reshape(-1)
    Y = np.empty((batch, M, N))
    Z = np.empty((batch, M, N))
    for i in range(batch):
        a = np.lib.stride_tricks.as_strided(
            A_flat[i * sA:], shape=(M, K), strides=(lda * 8, 8))
        if trans_b:
            b = np.lib.stride_tricks.as_strided(
                B_flat[i * sB:], shape=(N, K), strides=(ldb * 8, 8)).T
        else:
            b = np.lib.stride_tricks.as_strided(
                B_flat[i * sB:], shape=(K, N), strides=(ldb * 8, 8))
        bi = None
        if bias is not None and bias_kind != BIAS_NONE:
            bi = np.asarray(bias, dtype=np.float64).reshape(-1)[i * sBias:]
        Y[i], Z[i] = gemm_forward(a, b, bi, bias_kind if bi is not None else None,
                                  act, slope, alpha)
    return Y, Z


# ---------------------------------------------------------------------------
# Reduced-precision storage emulation
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit pattern, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(x, dtype: int) -> np.ndarray:
    """Values of x (any float) after one rounding to the storage dtype, as float32."""
    x32 = np.asarray(x, dtype=np.float32)
    if dtype == DT_F32:
        return x32.copy()
    if dtype == DT_BF16:
        return bf16_bits_to_f32(f32_to_bf16_bits(x32))
    if dtype == DT_F16:
        return x32.astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


def storage_eps(dtype: int) -> float:
    """Machine epsilon of the storage type (bf16 2^-7, fp16 2^-10, fp32 2^-23)."""
    return {DT_F32: 2.0 ** -23, DT_BF16: 2.0 ** -7, DT_F16: 2.0 ** -10}[dtype]


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own NumPy path (smoke_gemm_binding.py:84-123)
# ---------------------------------------------------------------------------
def numpy_fp32_step(A, B, bias, gY, act="relu", slope: float = 0.01):
    """fp32 forward + backward exactly as the reference test computes it.

    Used as the timed CPU baseline; float32 throughout like the reference.
    """
    Z = A @ B
    if bias is not None:
        Z = Z + bias
    if parse_act(act) == ACT_RELU:
        Y = np.maximum(Z, np.float32(0))
        gZ = gY * (Z > 0)
    else:
        Y = act_forward(Z, act, slope).astype(np.float32)
        gZ = (gY * act_deriv(Z, act, slope)).astype(np.float32)
    gA = gZ @ B.T
    gB = A.T @ gZ
    gBias = gZ.sum(axis=0, keepdims=True)
    return Y, Z, gA, gB, gBias


def forward_error_bound(A, B, K: int, dtype: int, bias=None) -> np.ndarray:
    """Componentwise bound 4*K*eps*(|A||B|)_mn + eps*|bias| for the tolerance tests."""
    eps = storage_eps(dtype) if dtype != DT_F32 else 2.0 ** -24
    absprod = np.abs(np.asarray(A, np.float64)) @ np.abs(np.asarray(B, np.float64))
    bnd = 4.0 * K * eps * absprod
    if bias is not None:
        bnd = bnd + eps * np.abs(np.asarray(bias, np.float64))
    return bnd


def gelu_erf(z) -> np.ndarray:
    """Exact GELU 0.5*z*(1+erf(z/sqrt(2))) -- what the tanh form approximates."""
    z = np.asarray(z, dtype=np.float64)
    erf = np.vectorize(math.erf)
    return 0.5 * z * (1.0 + erf(z / math.sqrt(2.0)))


# ---------------------------------------------------------------------------
# 2-D convolution (conv2d/launcher.cu:106-459, kernels.cu:12-87), float64
# ---------------------------------------------------------------------------
def conv2d_out_size(H: int, W: int, Kh: int, Kw: int, stride=(1, 1), pad=(0, 0), dil=(1, 1)) -> Tuple[int, int]:
    """launcher.cu:134-135."""
    Ho = (H + 2 * pad[0] - dil[0] * (Kh - 1) - 1) // stride[0] + 1
    Wo = (W + 2 * pad[1] - dil[1] * (Kw - 1) - 1) // stride[1] + 1
    return Ho, Wo


def _window(Xp, kh, kw, Ho, Wo, stride, dil):
    """X padded [N,C,Hp,Wp] -> the input samples under kernel tap (kh, kw): [N,C,Ho,Wo]."""
    h0, w0 = kh * dil[0], kw * dil[1]
    return Xp[:, :, h0:h0 + stride[0] * (Ho - 1) + 1:stride[0], w0:w0 + stride[1] * (Wo - 1) + 1:stride[1]]


def conv2d_forward(X, W, bias=None, stride=(1, 1), pad=(0, 0), dil=(1, 1), act="none",
                   slope: float = 0.01) -> Tuple[np.ndarray, np.ndarray]:
    """Z[n,co] = sum_{c,kh,kw} W[co,c,kh,kw] * Xpad[n,c,ho*s+kh*d, wo*s+kw*d] + bias[co];
    Y = act(Z).  Returns (Y, Z), float64 [N,Cout,Ho,Wo]."""
    X = np.asarray(X, np.float64)
    W = np.asarray(W, np.float64)
    N, C, H, Wd = X.shape
    Cout, C2, Kh, Kw = W.shape
    assert C == C2
    Ho, Wo = conv2d_out_size(H, Wd, Kh, Kw, stride, pad, dil)
    Xp = np.pad(X, ((0, 0), (0, 0), (pad[0], pad[0]), (pad[1], pad[1])))
    Z = np.zeros((N, Cout, Ho, Wo))
    for kh in range(Kh):
        for kw in range(Kw):
            win = _window(Xp, kh, kw, Ho, Wo, stride, dil)            # [N,C,Ho,Wo]
            Z += np.einsum("nchw,oc->nohw", win, W[:, :, kh, kw], optimize=True)
    if bias is not None:
        Z = Z + np.asarray(bias, np.float64).reshape(1, Cout, 1, 1)
    return act_forward(Z, act, slope), Z


def conv2d_backward(X, W, dY, Z, stride=(1, 1), pad=(0, 0), dil=(1, 1), act="none",
                    slope: float = 0.01) -> dict:
    """dZ = dY * act'(Z); dB[co] = sum over n, ho, wo of dZ; dW[co,c,kh,kw] = sum of
    dZ * the tap's input samples; dX = the transpose scatter of dZ through W (zero padding
    dropped).  float64."""
    X = np.asarray(X, np.float64)
    W = np.asarray(W, np.float64)
    N, C, H, Wd = X.shape
    Cout, _, Kh, Kw = W.shape
    Ho, Wo = conv2d_out_size(H, Wd, Kh, Kw, stride, pad, dil)
    dZ = np.asarray(dY, np.float64) * act_deriv(Z, act, slope)
    Xp = np.pad(X, ((0, 0), (0, 0), (pad[0], pad[0]), (pad[1], pad[1])))
    dXp = np.zeros_like(Xp)
    dW = np.zeros_like(W)
    for kh in range(Kh):
        for kw in range(Kw):
            win = _window(Xp, kh, kw, Ho, Wo, stride, dil)
            dW[:, :, kh, kw] = np.einsum("nohw,nchw->oc", dZ, win, optimize=True)
            h0, w0 = kh * dil[0], kw * dil[1]
            dXp[:, :, h0:h0 + stride[0] * (Ho - 1) + 1:stride[0], w0:w0 + stride[1] * (Wo - 1) + 1:stride[1]] += \
                np.einsum("nohw,oc->nchw", dZ, W[:, :, kh, kw], optimize=True)
    dX = dXp[:, :, pad[0]:pad[0] + H, pad[1]:pad[1] + Wd]
    return {"dZ": dZ, "dW": dW, "dB": dZ.sum(axis=(0, 2, 3)), "dX": dX}


def rnn_forward(X, Wx, Wh, h0, bias=None, act="none", slope: float = 0.01) -> Tuple[np.ndarray, np.ndarray]:
    """h_t = act(X[:,t] Wx + h_{t-1} Wh + b) for t = 0..T-1 from h0 (rnn/launcher.cu:186-227).
    Returns (Y, Z), float64 [N,T,H]: Y[:,t] = h_t, Z[:,t] = the pre-activation."""
    X = np.asarray(X, np.float64)
    Wx, Wh = np.asarray(Wx, np.float64), np.asarray(Wh, np.float64)
    N, T, _ = X.shape
    H = Wx.shape[1]
    b = np.zeros(H) if bias is None else np.asarray(bias, np.float64).reshape(H)
    Y, Z = np.zeros((N, T, H)), np.zeros((N, T, H))
    h = np.asarray(h0, np.float64)
    for t in range(T):
        Z[:, t] = X[:, t] @ Wx + h @ Wh + b
        h = act_forward(Z[:, t], act, slope)
        Y[:, t] = h
    return Y, Z


def rnn_backward(X, Wx, Wh, h0, dY, Z, act="none", slope: float = 0.01) -> dict:
    """Backward through time (rnn/launcher.cu:300-370): from t = T-1 down to 0,
    dZ_t = (dY[:,t] + dh_next) * act'(Z[:,t]); dWx += X_t^T dZ_t; dWh += h_{t-1}^T dZ_t
    (h_{-1} = h0, h_{t-1} = act(Z[:,t-1])); dB += column sums of dZ_t; dX[:,t] = dZ_t Wx^T;
    dh_next = dZ_t Wh^T; dh0 = the last dh_next.  float64."""
    X, dY, Z = (np.asarray(a, np.float64) for a in (X, dY, Z))
    Wx, Wh = np.asarray(Wx, np.float64), np.asarray(Wh, np.float64)
    h0 = np.asarray(h0, np.float64)
    N, T, I = X.shape
    H = Wx.shape[1]
    dWx, dWh, dB = np.zeros((I, H)), np.zeros((H, H)), np.zeros(H)
    dX = np.zeros((N, T, I))
    dh = np.zeros((N, H))
    for t in range(T - 1, -1, -1):
        dZ = (dY[:, t] + dh) * act_deriv(Z[:, t], act, slope)
        hprev = h0 if t == 0 else act_forward(Z[:, t - 1], act, slope)
        dWx += X[:, t].T @ dZ
        dWh += hprev.T @ dZ
        dB += dZ.sum(axis=0)
        dX[:, t] = dZ @ Wx.T
        dh = dZ @ Wh.T
    return {"dWx": dWx, "dWh": dWh, "dB": dB, "dX": dX, "dh0": dh}


MASK_NONE, MASK_I8, MASK_I32, MASK_F32 = 0, 1, 2, 3


def _sdpa_scores(Q, K, scale, causal, mask, mask_kind):
    """Scaled scores with the masks of launcher.cu:179-215 (external mask, then causal).  A
    masked entry is formed as the reference forms it, by an fp32 addition of -1e9 (or of the
    F32 mask value) to the fp32-rounded score; unmasked entries stay float64."""
    Q, K = np.asarray(Q, np.float64), np.asarray(K, np.float64)
    S = np.einsum("bhmd,bhnd->bhmn", Q, K, optimize=True) * scale
    M, N = S.shape[2], S.shape[3]
    add = np.zeros(S.shape, np.float32)
    hit = np.zeros(S.shape, bool)
    if mask_kind != MASK_NONE:
        mk = np.asarray(mask)[:, :1]                     # [B,1,M,N], broadcast over H
        if mask_kind == MASK_F32:
            add = add + mk.astype(np.float32)
            hit = hit | (mk != 0)
        else:
            add = add + np.where(mk != 0, np.float32(-1e9), np.float32(0))
            hit = hit | (mk != 0)
    if causal:
        cm = np.triu(np.ones((M, N), bool), 1)
        hit = hit | cm
    out = S.copy()
    if hit.any():
        s32 = S.astype(np.float32)
        if mask_kind != MASK_NONE:
            s32 = (s32 + np.broadcast_to(add, S.shape)).astype(np.float32)
        if causal:
            s32 = np.where(np.triu(np.ones((M, N), bool), 1), (s32 + np.float32(-1e9)).astype(np.float32), s32)
        out = np.where(hit, s32.astype(np.float64), S)
    return out, np.broadcast_to(hit, S.shape)


_U64 = np.uint64


def splitmix64(x) -> np.ndarray:
    """The reference's mixing function (dropout/kernels.cu:8-15; Steele, Lea and Flood's
    SplitMix64 output step), on uint64 arrays with arithmetic modulo 2^64."""
    with np.errstate(over="ignore"):
        z = np.asarray(x, dtype=np.uint64) + _U64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> _U64(30))) * _U64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> _U64(27))) * _U64(0x94D049BB133111EB)
        return z ^ (z >> _U64(31))


def dropout_factors(seed: int, B: int, H: int, M: int, N: int, p: float, scale_in_train: bool = True) -> np.ndarray:
    """The factor dropout multiplies each attention probability by, [B,H,M,N] float32:
    kept -> 1/(1-p) (scale_in_train and 1-p > 0; else 1), dropped -> 0.  Element (b,h,q,k)
    uses counter (b*H+h)*M*N + q*N + k (sdpa/launcher.cu:249-258) and is kept when the low 32
    bits u of splitmix64(seed ^ counter) give float32(u) * 2^-32 >= p (dropout/kernels.cu:17-45)."""
    ctr = np.arange(B * H * M * N, dtype=np.uint64)
    u = (splitmix64(_U64(seed) ^ ctr) & _U64(0xFFFFFFFF)).astype(np.uint32)
    r = u.astype(np.float32) * np.float32(1.0 / 4294967296.0)
    keep = r >= np.float32(p)
    one_m_p = np.float32(1.0) - np.float32(p)
    s = np.float32(1.0) / one_m_p if (scale_in_train and one_m_p > 0) else np.float32(1.0)
    return np.where(keep, s, np.float32(0)).astype(np.float32).reshape(B, H, M, N)


def sdpa_forward(Q, K, V, scale: float = 0.0, causal: bool = False, mask=None, mask_kind: int = MASK_NONE,
                 dropout_p: float = 0.0, seed: int = 0, scale_in_train: bool = True):
    """Y = dropout(softmax(scale Q K^T + masks)) V over [B,H,M,N] (launcher.cu:129-274).
    Returns (Y, P, lse) in float64, with P and lse those of the softmax before dropout;
    lse = log sum exp of the masked scaled scores per row."""
    D = np.asarray(Q).shape[-1]
    sc = scale if scale != 0.0 else 1.0 / math.sqrt(D)
    S, _ = _sdpa_scores(Q, K, sc, causal, mask, mask_kind)
    mx = S.max(axis=-1, keepdims=True)
    E = np.exp(S - mx)
    l = E.sum(axis=-1, keepdims=True)
    P = E / l
    Pd = P
    if dropout_p > 0:
        Pd = P * dropout_factors(seed, *P.shape, dropout_p, scale_in_train)
    Y = np.einsum("bhmn,bhnd->bhmd", Pd, np.asarray(V, np.float64), optimize=True)
    return Y, P, (mx + np.log(l))[..., 0]


def sdpa_backward(Q, K, V, dY, scale: float = 0.0, causal: bool = False, mask=None, mask_kind: int = MASK_NONE,
                  dropout_p: float = 0.0, seed: int = 0, scale_in_train: bool = True):
    """dQ, dK, dV of sdpa_forward for upstream dY (launcher.cu:333-747), float64.  With
    dropout (launcher.cu:454-590): dV = dropout(P)^T dY, and dP = dropout-backward(dY V^T)
    enters dS = P (dP - rowsum(dP P))."""
    Q, K, V, dY = (np.asarray(a, np.float64) for a in (Q, K, V, dY))
    D = Q.shape[-1]
    sc = scale if scale != 0.0 else 1.0 / math.sqrt(D)
    _, P, _ = sdpa_forward(Q, K, V, scale, causal, mask, mask_kind)
    _, hit = _sdpa_scores(Q, K, sc, causal, mask, mask_kind)
    f = dropout_factors(seed, *P.shape, dropout_p, scale_in_train) if dropout_p > 0 else 1.0
    dV = np.einsum("bhmn,bhmd->bhnd", P * f, dY, optimize=True)
    dP = np.einsum("bhmd,bhnd->bhmn", dY, V, optimize=True) * f
    dS = P * (dP - (dP * P).sum(axis=-1, keepdims=True))
    dS = np.where(hit, 0.0, dS)
    dQ = sc * np.einsum("bhmn,bhnd->bhmd", dS, K, optimize=True)
    dK = sc * np.einsum("bhmn,bhmd->bhnd", dS, Q, optimize=True)
    return {"dQ": dQ, "dK": dK, "dV": dV}
