"""The forward entry point that allocates nothing (gev2_gemm_fwd_noalloc): its split-K
scratch lives in a fixed device array of the library, so its results must equal
gev2_gemm_fwd's bit for bit (same kernels, same summation order), call after call, with the
array reused by the next (here smaller) problem; a problem that needs more scratch than the
array holds is refused before anything is launched."""
import ctypes

import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, F16, F32, DT_NAMES, Dev, make_fwd_inputs

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 16 << 20


def _both(capi, M, N, K, dtype, act, seed):
    """Y, Z from gev2_gemm_fwd (with its own workspace) and from gev2_gemm_fwd_noalloc."""
    X, W, b = make_fwd_inputs(seed, M, N, K, dtype, O.BIAS_PERN)
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pX, pW, pb = dev.put(capi.to_storage(X, dtype)), dev.put(capi.to_storage(W, dtype)), dev.put(b)
        outs = {}
        for name in ("fwd", "noalloc"):
            pY, pZ = dev.empty(M * N * es), dev.empty(M * N * es)
            kw = dict(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb, bias_kind=O.BIAS_PERN, act=act)
            if name == "fwd":
                need = capi.fwd_workspace_size(**kw)
                ws = dev.empty(max(need, 256)) if need else 0
                capi.gemm_fwd(workspace=ws, workspace_bytes=need, **kw)
            else:
                capi.gemm_fwd_noalloc(**kw)
            path = capi.last_path()
            capi.synchronize()
            outs[name] = (dev.get(pY, (M, N), dtype), dev.get(pZ, (M, N), dtype), path, need if name == "fwd" else None)
    finally:
        dev.close()
    return outs


@pytest.mark.parametrize("dtype", [BF16, F16, F32], ids=lambda d: DT_NAMES[d])
def test_noalloc_matches_fwd_two_calls(gpu, dtype):
    """Two calls in a row: C5b's 8x4096x4096 (2 MiB of split-K partials), then a smaller
    problem (5x1024x2048) that reuses the front of the array."""
    for (M, N, K), act, seed in (((8, 4096, 4096), "none", 91), ((5, 1024, 2048), "gelu", 92)):
        o = _both(gpu, M, N, K, dtype, act, seed)
        Yf, Zf, pf, need = o["fwd"]
        Yn, Zn, pn, _ = o["noalloc"]
        assert pf == pn, (pf, pn)
        if dtype != F32:
            assert pf == "skinny:split" and 0 < need <= NOALLOC_BYTES
        assert np.array_equal(Yf, Yn) and np.array_equal(Zf, Zn), (M, N, K, DT_NAMES[dtype])
        Y64, Z64 = O.gemm_forward(*make_fwd_inputs(seed, M, N, K, dtype, O.BIAS_PERN), O.BIAS_PERN, act)
        assert np.linalg.norm(Zn - Z64) <= 1e-2 * np.linalg.norm(Z64)


def test_noalloc_tile_path_matches(gpu):
    """A problem that needs no scratch (the tile path) gives the same results too."""
    o = _both(gpu, 200, 264, 96, BF16, "relu", 93)
    assert o["fwd"][2] == o["noalloc"][2] and o["fwd"][2].startswith(("dl:", "tile:"))
    assert np.array_equal(o["fwd"][0], o["noalloc"][0]) and np.array_equal(o["fwd"][1], o["noalloc"][1])


def test_noalloc_refuses_oversized_scratch(gpu):
    """M = 16, N = K = 16384 needs 64 MiB of partials: InvalidArgument, nothing launched
    (the pointers are never dereferenced: validation fails first)."""
    capi = gpu
    d = capi.fwd_desc(dtype=BF16, M=16, N=16384, K=16384, A=1 << 20, B=1 << 30, Y=1 << 40)
    assert capi.lib().gev2_gemm_fwd_workspace_size(ctypes.byref(d)) > NOALLOC_BYTES
    st = capi.lib().gev2_gemm_fwd_noalloc(ctypes.byref(d), None)
    assert st == 4, st
    assert b"more than" in capi.lib().gev2_last_error()
