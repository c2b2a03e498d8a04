"""Exact-integer golden fixtures (tests/golden/gemm_int_fixtures.npz).

The fixtures' expected outputs come from Python-integer loops in
tests/golden/make_gemm_int_fixtures.py, not from the oracle.  Every value is
exact in fp32 whatever the summation order, so the oracle (CPU) and the HIP
path (GPU, through the C ABI) must both match them bit for bit.  A 16-bit
storage type is checked wherever every input and expected value of the case is
representable in it (integers up to 256 in bf16, 2048 in fp16).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import gemm_oracle as O
from gemm_helpers import BF16, DT_NAMES, F16, F32, Dev

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemm_int_fixtures.npz")
SLOPE = 0.25   # the fixtures' LeakyReLU slope (exact in every storage type)


def _load() -> dict:
    with np.load(PATH, allow_pickle=False) as z:
        names = [str(n) for n in z["names"]]
        cases = {}
        for n in names:
            c = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(n + "/")}
            M, N, K, act, kind = (int(v) for v in c["dims"])
            c.update(M=M, N=N, K=K, act=act, kind=kind)
            cases[n] = c
    return cases


CASES = _load()
OUTS = ("Z", "Y", "dX", "dW")


def test_fixture_file_covers_edges():
    dims = [(c["M"], c["N"], c["K"]) for c in CASES.values()]
    assert (1, 1, 1) in dims
    assert {c["kind"] for c in CASES.values()} == {O.BIAS_NONE, O.BIAS_SCALAR, O.BIAS_PERM, O.BIAS_PERN}
    assert {c["act"] for c in CASES.values()} == {O.ACT_NONE, O.ACT_RELU, O.ACT_LEAKY}
    # ReLU' at z = 0 is pinned only if some pre-activation is exactly zero
    assert any(c["act"] == O.ACT_RELU and np.any(c["Z"] == 0) for c in CASES.values())


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_fixture(name):
    c = CASES[name]
    X, W, dY = (c[k].astype(np.float64) for k in ("X", "W", "dY"))
    b = c["bias"].astype(np.float64) if c["kind"] != O.BIAS_NONE else None
    Y, Z = O.gemm_forward(X, W, b, c["kind"] if b is not None else None, c["act"], SLOPE)
    assert np.array_equal(Z, c["Z"]), name
    assert np.array_equal(Y, c["Y"]), name
    g = O.gemm_backward(X, W, dY, Z, c["act"], SLOPE, c["kind"])
    assert np.array_equal(g["gA"], c["dX"]), name
    assert np.array_equal(g["gB"], c["dW"]), name
    if c["kind"] != O.BIAS_NONE:
        assert np.array_equal(g["gBias"], c["dBias"]), name


def test_planted_mistake_is_caught():
    """A ReLU' that is 1 at z = 0 (a plausible slip) disagrees with the fixtures."""
    c = next(c for c in CASES.values() if c["act"] == O.ACT_RELU and np.any((c["Z"] == 0) & (c["dY"] != 0)))
    gZ = c["dY"].astype(np.float64) * np.where(c["Z"] >= 0, 1.0, 0.0)
    assert not np.array_equal(gZ @ c["W"].astype(np.float64).T, c["dX"])


def _exact_in(c: dict, dtype: int) -> bool:
    vals = [c[k] for k in ("X", "W", "dY") + OUTS]
    return all(np.array_equal(O.round_to(v.astype(np.float64), dtype), v) for v in vals)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: DT_NAMES[d])
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_matches_fixture(gpu, name, dtype):
    capi = gpu
    c = CASES[name]
    if not _exact_in(c, dtype):
        pytest.skip(f"{name}: values not representable in {DT_NAMES[dtype]}")
    M, N, K, act, kind = c["M"], c["N"], c["K"], c["act"], c["kind"]
    es = capi.elem_bytes(dtype)
    st = lambda a: capi.to_storage(a.astype(np.float64), dtype)
    print(f"golden {name} {DT_NAMES[dtype]} {M}x{N}x{K}", flush=True)
    dev = Dev(capi)
    try:
        pX, pW, pdY = dev.put(st(c["X"])), dev.put(st(c["W"])), dev.put(st(c["dY"]))
        pb = dev.put(c["bias"].astype(np.float32)) if kind != O.BIAS_NONE else 0
        pY, pZ = dev.empty(M * N * es), dev.empty(M * N * es)
        capi.gemm_fwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb, bias_kind=kind,
                      act=act, leaky_slope=SLOPE)
        capi.synchronize()
        Y, Z = dev.get(pY, (M, N), dtype), dev.get(pZ, (M, N), dtype)
        pdX, pdW = dev.empty(M * K * es), dev.empty(K * N * es)
        nb = c["dBias"].size
        pdb = dev.empty(max(nb, 1) * 4) if nb else 0
        capi.gemm_bwd(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, gY=pdY, Z=pZ, gA=pdX, gB=pdW, gBias=pdb,
                      bias_kind=kind, act=act, leaky_slope=SLOPE)
        capi.synchronize()
        dX, dW = dev.get(pdX, (M, K), dtype), dev.get(pdW, (K, N), dtype)
        db = dev.get_f32(pdb, (nb,)) if nb else None
    finally:
        dev.close()
    tag = f"{name} {DT_NAMES[dtype]}"
    assert np.array_equal(Z, c["Z"]), "Z " + tag
    assert np.array_equal(Y, c["Y"]), "Y " + tag
    assert np.array_equal(dX, c["dX"]), "dX " + tag
    assert np.array_equal(dW, c["dW"]), "dW " + tag
    if nb:
        assert np.array_equal(db, c["dBias"]), "dBias " + tag
