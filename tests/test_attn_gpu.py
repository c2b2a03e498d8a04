"""GPU parity of scaled dot-product attention through the C ABI (gev2_sdpa_fwd / _bwd,
the sdpa op of sdpa/launcher.cu:129-747) against the float64 oracle:
  - the fused 16-bit kernel (bf16 / fp16, D = 64 and 128) with ragged M / N, causal and the
    three external mask kinds, and its row log-sum-exp;
  - the fp32 path (the reference's type) forward and backward, with the same masks;
  - dropout with the reference's stateless splitmix64 stream: the dropped set bit-exact
    against the oracle, forward and backward within tolerance on both paths;
  - the reference's validation results (dropout_p range, all-null outputs)."""
import ctypes
import math

import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, F16, F32, rounded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def capi(gpu):
    from graph_executor_v2.ops import capi as c
    return c


def _mask(kind, B, M, N, seed):
    if kind == O.MASK_NONE:
        return None
    r = np.random.default_rng(seed)
    hit = r.random((B, 1, M, N)) < 0.25
    hit[..., 0] = False                         # every row keeps a key
    if kind == O.MASK_I8:
        return hit.astype(np.int8)
    if kind == O.MASK_I32:
        return hit.astype(np.int32)
    return np.where(hit, -2.5, 0.0).astype(np.float32)


def _fwd(capi, Q, K, V, dtype, causal=False, mask=None, mask_kind=O.MASK_NONE, scale=0.0, want_lse=True,
         dropout_p=0.0, seed=0, scale_in_train=True):
    B, H, M, D = Q.shape
    N = K.shape[2]
    bufs = [capi.DeviceBuffer.from_numpy(capi.to_storage(a, dtype)) for a in (Q, K, V)]
    es = capi.elem_bytes(dtype)
    Y = capi.DeviceBuffer(B * H * M * D * es)
    lse = capi.DeviceBuffer(B * H * M * 4) if want_lse else None
    mk = capi.DeviceBuffer.from_numpy(mask) if mask is not None else None
    d = capi.SdpaDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, scale=scale, causal=int(causal), mask_kind=mask_kind,
                      mask=mk.ptr if mk else None, Q=bufs[0].ptr, K=bufs[1].ptr, V=bufs[2].ptr, Y=Y.ptr,
                      lse=lse.ptr if lse else None, dropout_p=dropout_p, seed=seed,
                      scale_in_train=int(scale_in_train))
    L = capi.lib()
    wsb = L.gev2_sdpa_workspace_size(ctypes.byref(d), 0)
    ws = capi.DeviceBuffer(max(wsb, 1)) if wsb > 0 else None
    if ws:
        d.workspace, d.workspace_bytes = ws.ptr, wsb
    capi.check_sdpa(L.gev2_sdpa_fwd(ctypes.byref(d), None), "sdpa fwd")
    capi.synchronize()
    y = capi.from_storage(Y.download((B, H, M, D), capi.to_storage(np.zeros(1, np.float32), dtype).dtype), dtype)
    return y, (lse.download((B, H, M), np.float32) if lse else None)


def _qkv(seed, B, H, M, N, D, dtype):
    r = np.random.default_rng(seed)
    Q, K, V = (r.standard_normal(s).astype(np.float32) for s in ((B, H, M, D), (B, H, N, D), (B, H, N, D)))
    if dtype != F32:
        Q, K, V = (rounded(a, dtype).astype(np.float32) for a in (Q, K, V))
    return Q, K, V


FUSED_CASES = [
    # (B, H, M, N, D, causal, mask kind)
    (2, 3, 200, 136, 64, False, O.MASK_NONE),
    (1, 2, 128, 256, 128, False, O.MASK_NONE),
    (2, 2, 192, 192, 64, True, O.MASK_NONE),
    (1, 3, 70, 100, 64, False, O.MASK_I8),
    (2, 1, 130, 64, 128, True, O.MASK_I32),
    (1, 2, 96, 160, 64, False, O.MASK_F32),
    (1, 1, 1, 1, 64, False, O.MASK_NONE),          # one query, one key: Y = V
    (1, 2, 3, 200, 128, True, O.MASK_NONE),        # M < N with causal
    (8, 8, 512, 512, 64, False, O.MASK_NONE),      # the C4 shape (8 sequences x 8 heads)
]


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "B{}H{}M{}N{}D{}{}{}".format(
    *c[:5], "-causal" if c[5] else "", ["", "-i8", "-i32", "-f32"][c[6]]))
def test_fused_forward(capi, dtype, case):
    """Per element: |Y - Y64| <= 2 eps (P |V|) + 1e-4, eps the storage epsilon (P is rounded
    to the storage type for the P V product); lse within 1e-4 (1 + |lse|)."""
    B, H, M, N, D, causal, mk = case
    Q, K, V = _qkv(21, B, H, M, N, D, dtype)
    mask = _mask(mk, B, M, N, 22)
    y, lse = _fwd(capi, Q, K, V, dtype, causal, mask, mk)
    Y64, P64, lse64 = O.sdpa_forward(Q, K, V, causal=causal, mask=mask, mask_kind=mk)
    eps = O.storage_eps(dtype)
    bound = 2 * eps * np.einsum("bhmn,bhnd->bhmd", P64, np.abs(V)) + 1e-4 + eps * np.abs(Y64)
    err = np.abs(y - Y64)
    assert np.all(err <= bound), (float(err.max()), np.unravel_index(int(np.argmax(err - bound)), err.shape))
    assert np.all(np.abs(lse - lse64) <= 1e-4 * (1 + np.abs(lse64)))


def test_fused_forward_scale_attr(capi):
    """attrs.scale overrides 1/sqrt(D)."""
    Q, K, V = _qkv(23, 1, 2, 64, 64, 64, BF16)
    y, _ = _fwd(capi, Q, K, V, BF16, scale=0.3)
    Y64, P64, _ = O.sdpa_forward(Q, K, V, scale=0.3)
    eps = O.storage_eps(BF16)
    assert np.all(np.abs(y - Y64) <= 2 * eps * np.einsum("bhmn,bhnd->bhmd", P64, np.abs(V)) + 1e-4 + eps * np.abs(Y64))


@pytest.mark.parametrize("causal,mk", [(False, O.MASK_NONE), (True, O.MASK_NONE), (False, O.MASK_I8),
                                       (True, O.MASK_F32)], ids=["plain", "causal", "i8", "causal-f32"])
def test_f32_forward_backward(capi, causal, mk):
    B, H, M, N, D = 2, 2, 48, 40, 16
    Q, K, V = _qkv(24, B, H, M, N, D, F32)
    mask = _mask(mk, B, M, N, 25)
    y, _ = _fwd(capi, Q, K, V, F32, causal, mask, mk, want_lse=False)
    Y64, _, _ = O.sdpa_forward(Q, K, V, causal=causal, mask=mask, mask_kind=mk)
    np.testing.assert_allclose(y, Y64, rtol=1e-4, atol=1e-5)
    dY = np.random.default_rng(26).standard_normal(Q.shape).astype(np.float32)
    bufs = [capi.DeviceBuffer.from_numpy(a) for a in (Q, K, V, dY)]
    outs = [capi.DeviceBuffer(a.nbytes) for a in (Q, K, V)]
    mkb = capi.DeviceBuffer.from_numpy(mask) if mask is not None else None
    d = capi.SdpaBwdDesc(dtype=F32, B=B, H=H, M=M, N=N, D=D, causal=int(causal), mask_kind=mk,
                         mask=mkb.ptr if mkb else None, Q=bufs[0].ptr, K=bufs[1].ptr, V=bufs[2].ptr, dY=bufs[3].ptr,
                         dQ=outs[0].ptr, dK=outs[1].ptr, dV=outs[2].ptr)
    L = capi.lib()
    fd = capi.SdpaDesc(dtype=F32, B=B, H=H, M=M, N=N, D=D)
    wsb = L.gev2_sdpa_workspace_size(ctypes.byref(fd), 1)
    ws = capi.DeviceBuffer(wsb)
    d.workspace, d.workspace_bytes = ws.ptr, wsb
    capi.check_sdpa(L.gev2_sdpa_bwd(ctypes.byref(d), None), "sdpa bwd")
    capi.synchronize()
    ref = O.sdpa_backward(Q, K, V, dY, causal=causal, mask=mask, mask_kind=mk)
    for name, buf, a in zip(("dQ", "dK", "dV"), outs, (Q, K, V)):
        np.testing.assert_allclose(buf.download(a.shape, np.float32), ref[name], rtol=1e-4, atol=1e-4, err_msg=name)


def test_validation(capi):
    L = capi.lib()
    d = capi.SdpaDesc(dtype=BF16, B=1, H=1, M=8, N=8, D=64, dropout_p=1.5, Q=16, K=32, V=48, Y=64)
    assert L.gev2_sdpa_fwd(ctypes.byref(d), None) == 4            # dropout_p outside [0, 1]
    d.dropout_p = -0.1
    assert L.gev2_sdpa_fwd(ctypes.byref(d), None) == 4
    d.dropout_p, d.mask_kind = 0.0, O.MASK_I8
    assert L.gev2_sdpa_fwd(ctypes.byref(d), None) == 10           # mask kind without a mask
    b = capi.SdpaBwdDesc(dtype=F32, B=1, H=1, M=8, N=8, D=16, Q=16, K=32, V=48, dY=64)
    assert L.gev2_sdpa_bwd(ctypes.byref(b), None) == 1            # all outputs null (launcher.cu:342)


BWD_CASES = [
    # (B, H, M, N, D, causal, mask kind)
    (1, 2, 40, 56, 64, False, O.MASK_NONE),
    (1, 2, 40, 56, 64, True, O.MASK_I32),
    (2, 1, 130, 70, 64, False, O.MASK_NONE),
    (1, 2, 96, 128, 128, True, O.MASK_NONE),
    (1, 1, 72, 100, 128, False, O.MASK_I8),
    (1, 2, 64, 80, 64, False, O.MASK_F32),
    (1, 1, 1, 1, 64, False, O.MASK_NONE),
    (1, 1, 5, 130, 64, True, O.MASK_NONE),
    (8, 8, 512, 512, 64, False, O.MASK_NONE),      # the C4 shape
]


@pytest.mark.parametrize("path", ["fused", "wide"])
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: "B{}H{}M{}N{}D{}{}{}".format(
    *c[:5], "-causal" if c[5] else "", ["", "-i8", "-i32", "-f32"][c[6]]))
def test_16bit_backward(capi, dtype, case, path, monkeypatch):
    """16-bit tensors.  wide: fp32 arithmetic on the exact 16-bit inputs, each gradient
    rounded once: |g - g64| <= eps |g64| + 1e-5 max|g64|.  fused: P and dS enter the MFMAs
    as 16-bit values: max|g - g64| <= 8 eps (max|g64| + t), where t bounds what the 16-bit O
    does to Dq = rowsum(dO O) (|dDq| <= eps sum_d |dO||O|) through scale K (dQ) or scale Q (dK);
    it is what remains when the exact gradient vanishes (one key).  An indexing mistake is O(1)."""
    if path == "wide":
        monkeypatch.setenv("GEV2_ATTN_BWD_WIDE", "1")
    else:
        monkeypatch.delenv("GEV2_ATTN_BWD_WIDE", raising=False)
    B, H, M, N, D, causal, mk = case
    Q, K, V = _qkv(27, B, H, M, N, D, dtype)
    dY = rounded(np.random.default_rng(28).standard_normal(Q.shape), dtype).astype(np.float32)
    mask = _mask(mk, B, M, N, 29)
    bufs = [capi.DeviceBuffer.from_numpy(capi.to_storage(a, dtype)) for a in (Q, K, V, dY)]
    es = capi.elem_bytes(dtype)
    outs = [capi.DeviceBuffer(a.size * es) for a in (Q, K, V)]
    mkb = capi.DeviceBuffer.from_numpy(mask) if mask is not None else None
    L = capi.lib()
    fd = capi.SdpaDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D)
    wsb = L.gev2_sdpa_workspace_size(ctypes.byref(fd), 1)
    ws = capi.DeviceBuffer(wsb)
    d = capi.SdpaBwdDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, causal=int(causal), mask_kind=mk,
                         mask=mkb.ptr if mkb else None, Q=bufs[0].ptr, K=bufs[1].ptr, V=bufs[2].ptr, dY=bufs[3].ptr,
                         dQ=outs[0].ptr, dK=outs[1].ptr, dV=outs[2].ptr, workspace=ws.ptr, workspace_bytes=wsb)
    capi.check_sdpa(L.gev2_sdpa_bwd(ctypes.byref(d), None), "sdpa bwd 16-bit")
    capi.synchronize()
    ref = O.sdpa_backward(Q, K, V, dY, causal=causal, mask=mask, mask_kind=mk)
    Y64, _, _ = O.sdpa_forward(Q, K, V, causal=causal, mask=mask, mask_kind=mk)
    dq_term = (np.abs(dY) * np.abs(Y64)).sum(-1).max() / np.sqrt(D)
    t = {"dQ": dq_term * np.abs(K).max(), "dK": dq_term * np.abs(Q).max(), "dV": 0.0}
    st = capi.to_storage(np.zeros(1, np.float32), dtype).dtype
    eps = O.storage_eps(dtype)
    for name, buf, a in zip(("dQ", "dK", "dV"), outs, (Q, K, V)):
        g = capi.from_storage(buf.download(a.shape, st), dtype)
        r = ref[name]
        if path == "wide":
            assert np.all(np.abs(g - r) <= eps * np.abs(r) + 1e-5 * np.abs(r).max()), name
        else:
            err = float(np.abs(g - r).max())
            assert err <= 8 * eps * (np.abs(r).max() + t[name]), (name, err, float(np.abs(r).max()), t[name])


@pytest.fixture(scope="module")
def host(gpu):
    from graph_executor_v2.ops import _ops_sdpa as s
    from graph_executor_v2.ops.device_array import DeviceArray
    return s, DeviceArray


@pytest.mark.parametrize("dtype,causal,mk", [(F32, False, O.MASK_I8), (BF16, True, O.MASK_NONE),
                                             (F16, False, O.MASK_F32)], ids=["f32-i8", "bf16-causal", "f16-f32mask"])
def test_host_api(capi, host, dtype, causal, mk):
    """SDPACudaLaunch / SDPACudaBackwardLaunch (workspace allocated per call, as the
    reference does) give what the C ABI gives."""
    sd, DA = host
    B, H, M, N, D = 1, 2, 48, 72, 64
    Q, K, V = _qkv(33, B, H, M, N, D, dtype)
    dY = rounded(np.random.default_rng(34).standard_normal(Q.shape), dtype).astype(np.float32) if dtype != F32 \
        else np.random.default_rng(34).standard_normal(Q.shape).astype(np.float32)
    mask = _mask(mk, B, M, N, 35)
    name = {F32: "float32", BF16: "bfloat16", F16: "float16"}[dtype]
    code = {F32: sd.DType.F32, BF16: sd.DType.BF16, F16: sd.DType.F16}[dtype]
    dq, dk, dv, dy = (DA.from_numpy(a, name) for a in (Q, K, V, dY))
    y = DA.empty(Q.shape, name)
    gq, gk, gv = DA.empty(Q.shape, name), DA.empty(K.shape, name), DA.empty(V.shape, name)
    mb = capi.DeviceBuffer.from_numpy(mask) if mask is not None else None
    mdt = {O.MASK_I8: sd.DType.I8, O.MASK_I32: sd.DType.I32, O.MASK_F32: sd.DType.F32}.get(mk, sd.DType.I8)
    a = sd.SDPAAttrs()
    a.causal = causal
    sd.forward(dq.ptr, list(Q.shape), dk.ptr, list(K.shape), dv.ptr, list(V.shape), y.ptr, list(Q.shape),
               mask_ptr=mb.ptr if mb else None, mask_dtype=mdt, attrs=a, dtype=code)
    sd.backward(dq.ptr, list(Q.shape), dk.ptr, list(K.shape), dv.ptr, list(V.shape), dy.ptr, dq_ptr=gq.ptr,
                dk_ptr=gk.ptr, dv_ptr=gv.ptr, mask_ptr=mb.ptr if mb else None, mask_dtype=mdt, attrs=a, dtype=code)
    Y64, _, _ = O.sdpa_forward(Q, K, V, causal=causal, mask=mask, mask_kind=mk)
    ref = O.sdpa_backward(Q, K, V, dY, causal=causal, mask=mask, mask_kind=mk)
    tol = 1e-4 if dtype == F32 else 8 * O.storage_eps(dtype)
    assert np.abs(y.get() - Y64).max() <= tol * max(1.0, np.abs(Y64).max())
    for g_, r in ((gq, ref["dQ"]), (gk, ref["dK"]), (gv, ref["dV"])):
        assert np.abs(g_.get() - r).max() <= tol * max(1.0, np.abs(r).max())


# ---------------------------------------------------------------------------
# Dropout (the reference's stateless stream, dropout/kernels.cu:8-45)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,D", [(BF16, 64), (F16, 128), (F32, 64)], ids=["bf16-d64", "f16-d128", "f32-d64"])
@pytest.mark.parametrize("scale_in_train", [True, False], ids=["scaled", "unscaled"])
def test_dropout_mask_exact(capi, dtype, D, scale_in_train):
    """Q = K = 0 make every probability 1/N, and V = I (N = D keys) makes Y = dropout(P) itself:
    Y must equal factor / N bit for bit (1.25 / N and 1 / N are exact in every storage type),
    so the kept set of every (b, h, query, key) is checked against the oracle's stream."""
    B, H, M, N, p, seed = 2, 3, 96, D, 0.2, 20261202
    Q = np.zeros((B, H, M, D), np.float32)
    K = np.zeros((B, H, N, D), np.float32)
    V = np.broadcast_to(np.eye(N, D, dtype=np.float32), (B, H, N, D)).copy()
    y, _ = _fwd(capi, Q, K, V, dtype, want_lse=False, dropout_p=p, seed=seed, scale_in_train=scale_in_train)
    f = O.dropout_factors(seed, B, H, M, N, p, scale_in_train)
    assert np.array_equal(y != 0, f != 0), int(((y != 0) != (f != 0)).sum())
    assert np.array_equal(y, (f / np.float32(N)).astype(np.float32))


@pytest.mark.parametrize("dtype,D,causal", [(BF16, 64, False), (F16, 128, True), (F32, 32, False)],
                         ids=["bf16-d64", "f16-d128-causal", "f32-d32"])
def test_dropout_forward_backward(capi, dtype, D, causal, monkeypatch):
    """Random inputs with dropout p = 0.3: the forward within the fused / fp32 bounds used above
    (computed with the dropped probabilities), and dQ / dK / dV of the fused (16-bit) or batched
    fp32 backward against the oracle's gradient of the same dropped function."""
    B, H, M, N, p, seed = 1, 2, 130, 100, 0.3, 77
    Q, K, V = _qkv(61, B, H, M, N, D, dtype)
    y, lse = _fwd(capi, Q, K, V, dtype, causal, want_lse=dtype != F32, dropout_p=p, seed=seed)
    Y64, P64, lse64 = O.sdpa_forward(Q, K, V, causal=causal, dropout_p=p, seed=seed)
    Pd = P64 * O.dropout_factors(seed, B, H, M, N, p)
    if dtype == F32:
        np.testing.assert_allclose(y, Y64, rtol=1e-4, atol=1e-5)
    else:
        eps = O.storage_eps(dtype)
        bound = 2 * eps * np.einsum("bhmn,bhnd->bhmd", Pd, np.abs(V)) + 1e-4 + eps * np.abs(Y64)
        err = np.abs(y - Y64)
        assert np.all(err <= bound), (float(err.max()), np.unravel_index(int(np.argmax(err - bound)), err.shape))
        assert np.all(np.abs(lse - lse64) <= 1e-4 * (1 + np.abs(lse64)))   # lse of the undropped softmax
    dY = rounded(np.random.default_rng(62).standard_normal(Q.shape), dtype).astype(np.float32)
    bufs = [capi.DeviceBuffer.from_numpy(capi.to_storage(a, dtype)) for a in (Q, K, V, dY)]
    es = capi.elem_bytes(dtype)
    outs = [capi.DeviceBuffer(a.size * es) for a in (Q, K, V)]
    L = capi.lib()
    fd = capi.SdpaDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, causal=int(causal), dropout_p=p, seed=seed,
                       scale_in_train=1)
    wsb = L.gev2_sdpa_workspace_size(ctypes.byref(fd), 1)
    ws = capi.DeviceBuffer(wsb)
    d = capi.SdpaBwdDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, causal=int(causal), dropout_p=p, seed=seed,
                         scale_in_train=1, Q=bufs[0].ptr, K=bufs[1].ptr, V=bufs[2].ptr, dY=bufs[3].ptr,
                         dQ=outs[0].ptr, dK=outs[1].ptr, dV=outs[2].ptr, workspace=ws.ptr, workspace_bytes=wsb)
    capi.check_sdpa(L.gev2_sdpa_bwd(ctypes.byref(d), None), "sdpa bwd dropout")
    capi.synchronize()
    ref = O.sdpa_backward(Q, K, V, dY, causal=causal, dropout_p=p, seed=seed)
    st = capi.to_storage(np.zeros(1, np.float32), dtype).dtype
    dq_term = (np.abs(dY) * np.abs(Y64)).sum(-1).max() / np.sqrt(D)
    t = {"dQ": dq_term * np.abs(K).max(), "dK": dq_term * np.abs(Q).max(), "dV": 0.0}
    for name, buf, a in zip(("dQ", "dK", "dV"), outs, (Q, K, V)):
        g = capi.from_storage(buf.download(a.shape, st), dtype)
        r = ref[name]
        if dtype == F32:
            np.testing.assert_allclose(g, r, rtol=1e-4, atol=1e-4, err_msg=name)
        else:
            eps = O.storage_eps(dtype)
            err = float(np.abs(g - r).max())
            # the dropped P enters dV as a 16-bit value scaled by 1/(1-p): one more factor of it
            assert err <= 8 * eps * (np.abs(r).max() + t[name]) / (1 - p), (name, err, float(np.abs(r).max()))
