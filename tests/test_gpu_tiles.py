"""GPU parity of every large-tile kernel variant, forced one at a time.

The tile dispatcher picks the kernel by cost; here GEV2_TILE_CFG pins the tile
(256x256, 128x256, 128x128, 128x64) so that each shape runs through each variant:
the direct-to-LDS kernel for 16-bit data (both epilogue forms: LDS-staged
16-byte rows when N % 8 == 0, 4-column stores when only N % 4 == 0), and
with GEV2_DL=0 the register-staged kernel it replaces.

Inputs are small integers, so every dot product is exact in fp32 and the
device result must equal the oracle's after one rounding to the storage type,
bit for bit (reference semantics: launcher.cu:147-274, epilogue traits.hpp:43-71).
Shapes are ragged against every tile (M, N) and against BK = 32 and 64 (K).
"""
import os

import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, F16, F32, DT_NAMES, Dev, rounded

pytestmark = pytest.mark.gpu

CFGS = {0: "256x256", 3: "128x256", 1: "128x128", 4: "128x64"}
# the register-staged kernel has no 128x64 tile and runs that request as 128x128
PIPE_NAME = {**{c: n for c, n in CFGS.items()}, 4: "128x128"}

# (layout, M, N, K, ldy_pad): NT keeps K contiguous on both operands, so N may
# be 4 mod 8 there (the 4-column epilogue); NN / TN need N (and TN M) % 8 == 0
# for vector loads.  ldy_pad = 4 makes the output rows 8-byte aligned only.
CASES = [
    ("NN", 300, 264, 328, 0),
    ("NT", 300, 264, 328, 0),
    ("TN", 296, 264, 328, 0),
    ("NT", 300, 268, 328, 0),
    ("NN", 300, 264, 200, 4),
    ("NN", 520, 1040, 96, 0),
]


def _ints(g, shape, lo=-2, hi=2):
    return g.integers(lo, hi + 1, size=shape).astype(np.float32)


def _run(capi, layout, M, N, K, ldy_pad, dtype, bias_kind, act, seed):
    g = np.random.default_rng(seed)
    X = _ints(g, (M, K))
    W = _ints(g, (K, N))
    nb = {O.BIAS_PERN: N, O.BIAS_PERM: M, O.BIAS_SCALAR: 1}[bias_kind]
    b = _ints(g, (nb,), -3, 3)
    ta, tb = layout[0] == "T", layout[1] == "T"
    A = np.ascontiguousarray(X.T) if ta else X
    B = np.ascontiguousarray(W.T) if tb else W
    ldy = N + ldy_pad
    es = capi.elem_bytes(dtype)
    dev = Dev(capi)
    try:
        pA, pB = dev.put(capi.to_storage(A, dtype)), dev.put(capi.to_storage(B, dtype))
        pb = dev.put(b)
        pY = dev.empty(M * ldy * es)
        pZ = dev.empty(M * ldy * es)
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=K, A=pA, B=pB, Y=pY, Z=pZ, bias=pb, bias_kind=bias_kind,
                      act=act, trans_a=ta, trans_b=tb, ldy=ldy, ldz=ldy)
        path = capi.last_path()
        capi.synchronize()
        Y = dev.get(pY, (M, ldy), dtype)[:, :N]
        Z = dev.get(pZ, (M, ldy), dtype)[:, :N]
    finally:
        dev.close()
    Y64, Z64 = O.gemm_forward(X, W, b, bias_kind, act)
    return Y, Z, rounded(Y64, dtype), rounded(Z64, dtype), path


@pytest.mark.parametrize("cfg", list(CFGS), ids=lambda c: CFGS[c])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-pad{c[4]}")
@pytest.mark.parametrize("kernel", ["dl", "pipe"])
def test_tile_variants_exact(gpu, monkeypatch, cfg, case, kernel):
    capi = gpu
    monkeypatch.setenv("GEV2_TILE_CFG", str(cfg))
    monkeypatch.setenv("GEV2_DL", "1" if kernel == "dl" else "0")
    layout, M, N, K, pad = case
    Y, Z, Yr, Zr, path = _run(capi, layout, M, N, K, pad, BF16, O.BIAS_PERN, "relu", seed=cfg * 7 + M)
    assert path == (f"dl:{CFGS[cfg]}" if kernel == "dl" else f"tile:{PIPE_NAME[cfg]}"), path
    assert np.array_equal(Z, Zr), f"Z {layout} {M}x{N}x{K} {path}"
    assert np.array_equal(Y, Yr), f"Y {layout} {M}x{N}x{K} {path}"


CFGS_F32 = {**CFGS, 2: "64x64"}


@pytest.mark.parametrize("cfg", list(CFGS_F32), ids=lambda c: CFGS_F32[c])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-pad{c[4]}")
@pytest.mark.parametrize("kernel", ["dl", "pipe"])
def test_tile_variants_exact_f32(gpu, monkeypatch, cfg, case, kernel):
    """fp32 on every tile, through the direct-to-LDS kernel (K-contiguous operands read as
    16-byte fragments, M/N-contiguous ones as four k rows) and the register-staged one."""
    capi = gpu
    monkeypatch.setenv("GEV2_TILE_CFG", str(cfg))
    monkeypatch.setenv("GEV2_DL", "1" if kernel == "dl" else "0")
    monkeypatch.setenv("GEV2_NO_SPLITK", "1")        # one launch over all of K
    monkeypatch.setenv("GEV2_NO_SMALL", "1")         # the tile kernels, not the small one
    layout, M, N, K, pad = case
    Y, Z, Yr, Zr, path = _run(capi, layout, M, N, K, pad, F32, O.BIAS_PERN, "relu", seed=cfg * 11 + M)
    assert path == (f"dl:{CFGS_F32[cfg]}" if kernel == "dl" else f"tile:{PIPE_NAME.get(cfg, CFGS_F32[cfg])}"), path
    assert np.array_equal(Z, Zr), f"Z {layout} {M}x{N}x{K} {path}"
    assert np.array_equal(Y, Yr), f"Y {layout} {M}x{N}x{K} {path}"


@pytest.mark.parametrize("bias_kind", [O.BIAS_PERM, O.BIAS_SCALAR])
@pytest.mark.parametrize("dtype", [BF16, F16], ids=lambda d: DT_NAMES[d])
def test_dl_bias_kinds_exact(gpu, monkeypatch, bias_kind, dtype):
    capi = gpu
    monkeypatch.setenv("GEV2_TILE_CFG", "0")
    Y, Z, Yr, Zr, path = _run(capi, "NN", 300, 264, 328, 0, dtype, bias_kind, "relu", seed=5)
    assert path == "dl:256x256", path
    assert np.array_equal(Z, Zr)
    assert np.array_equal(Y, Yr)


# Skinny forward (M <= 16): the split-K MFMA kernel (one K block when K <= 256,
# otherwise fp32 partials in the workspace plus the fixed-order reduction),
# and the dot-product kernel it replaces for 16-bit data (GEV2_SKINNY_DOT=1).
SKINNY = [(8, 4096, 4096), (13, 264, 328), (1, 72, 64), (16, 1000, 1032), (5, 136, 2056), (3, 520, 256)]


@pytest.mark.parametrize("variant", ["0", "1"], ids=["dl", "dot2"])
@pytest.mark.parametrize("shape", SKINNY, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", [BF16, F16], ids=lambda d: DT_NAMES[d])
def test_skinny_variants_exact(gpu, monkeypatch, variant, shape, dtype):
    capi = gpu
    monkeypatch.setenv("GEV2_SKINNY_DOT", variant)
    M, N, K = shape
    Y, Z, Yr, Zr, path = _run(capi, "NN", M, N, K, 0, dtype, O.BIAS_PERN, "relu", seed=M + N)
    assert path == ("skinny" if variant == "1" else "skinny:split"), path
    assert np.array_equal(Z, Zr), f"Z {shape}"
    assert np.array_equal(Y, Yr), f"Y {shape}"


@pytest.mark.parametrize("shape", [(13, 264, 328), (5, 136, 2056), (8, 1024, 1536)], ids=lambda s: "x".join(map(str, s)))
def test_skinny_256_row_blocks_exact(gpu, monkeypatch, shape):
    """GEV2_SKINNY_ROWS=256 keeps 256-row K blocks where the default takes 128-row ones (fewer
    than 128 workgroups of 256 rows): both exact on integer inputs."""
    capi = gpu
    monkeypatch.setenv("GEV2_SKINNY_ROWS", "256")
    M, N, K = shape
    Y, Z, Yr, Zr, path = _run(capi, "NN", M, N, K, 0, BF16, O.BIAS_PERN, "relu", seed=M + K)
    assert path == "skinny:split", path
    assert np.array_equal(Z, Zr), f"Z {shape}"
    assert np.array_equal(Y, Yr), f"Y {shape}"


def test_skinny_explicit_workspace(gpu):
    """A caller-provided workspace (gev2_gemm_fwd_workspace_size bytes) gives the same
    bits as the library's per-stream buffer, and two problems in a row that share it
    (the second smaller) are both right."""
    capi = gpu
    g = np.random.default_rng(21)
    dev = Dev(capi)
    try:
        for (M, N, K) in [(8, 4096, 4096), (3, 520, 1032)]:
            X, W = _ints(g, (M, K)), _ints(g, (K, N))
            b = _ints(g, (N,), -3, 3)
            pX, pW, pb = dev.put(capi.to_storage(X, BF16)), dev.put(capi.to_storage(W, BF16)), dev.put(b)
            outs = []
            for own in (False, True):
                pY = dev.empty(M * N * 2)
                kw = dict(dtype=BF16, M=M, N=N, K=K, A=pX, B=pW, Y=pY, bias=pb, bias_kind=O.BIAS_PERN,
                          act="relu")
                need = capi.fwd_workspace_size(**kw)
                # K blocks x column slabs x (cols / 16) tiles x 16*ceil(M/4) lanes x 16 bytes, for
                # 256-column x 256-row W blocks (GEV2_SKINNY_COLS=512: 512 x 128; 256 x 128 when
                # 256-row blocks would give fewer than 128 workgroups and K > 256)
                cols = 512 if os.environ.get("GEV2_SKINNY_COLS") == "512" else 256
                rows = 65536 // cols
                if cols == 256 and K > 256 and -(-N // 256) * -(-K // 256) < 128 and \
                        os.environ.get("GEV2_SKINNY_ROWS") != "256":
                    rows = 128
                assert need == -(-K // rows) * -(-N // cols) * (cols // 16) * 16 * -(-M // 4) * 16
                if own:
                    kw.update(workspace=dev.empty(need), workspace_bytes=need)
                capi.gemm_fwd(**kw)
                assert capi.last_path() == "skinny:split"
                capi.synchronize()
                outs.append(dev.get(pY, (M, N), BF16))
            Y64, _ = O.gemm_forward(X, W, b, O.BIAS_PERN, "relu")
            assert np.array_equal(outs[0], rounded(Y64, BF16))
            assert np.array_equal(outs[1], outs[0])
    finally:
        dev.close()
