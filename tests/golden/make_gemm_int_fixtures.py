"""Writes gemm_int_fixtures.npz: exact-integer GEMM + bias + activation cases.

Every input is an integer in [-2, 2] and the LeakyReLU slope is 1/4, so every
product, partial sum, bias add and activation is exact in fp32, whatever the
summation order.  The expected outputs are computed here with Python integers
(values scaled by 4 so the LeakyReLU branch stays integral), independently of
the float64 oracle, following the reference's rules:

  forward  Z = X W + bias, Y = act(Z)       regemm_gemm_bias_act.cu:239-258
  bias     scalar / per-column / per-row    bias.hpp:155-176
  act      ReLU z > 0 ? z : 0; Leaky z > 0 ? z : a z      activations.hpp:14-39
  act'     ReLU z > 0 ? 1 : 0 (0 at z = 0); Leaky z > 0 ? 1 : a   activations.hpp:44-46
  backward gZ = dY * act'(Z), dX = gZ W^T, dW = X^T gZ, dBias = sums of gZ
                                            regemm_backward.cu:91-130, :271-291

Run from the repository root: python tests/golden/make_gemm_int_fixtures.py
"""
from __future__ import annotations

import os

import numpy as np

# bias kinds as the operator numbers them (none, scalar, per-row M, per-column N)
BIAS_NONE, BIAS_SCALAR, BIAS_PERM, BIAS_PERN = 0, 1, 2, 3
ACTS = {"none": 0, "relu": 1, "leaky": 2}
SLOPE_X4 = 1   # LeakyReLU slope 1/4, held as 1/4 of the scale 4

CASES = [
    # (name, M, N, K, act, bias kind)
    ("one", 1, 1, 1, "relu", BIAS_SCALAR),
    ("ragged_none_pern", 5, 7, 3, "none", BIAS_PERN),
    ("relu_perm", 17, 33, 9, "relu", BIAS_PERM),
    ("relu_pern", 40, 36, 24, "relu", BIAS_PERN),
    ("skinny_leaky", 8, 64, 16, "leaky", BIAS_PERN),
    ("tile_edge_relu", 65, 72, 20, "relu", BIAS_NONE),
]


def _case(g: np.random.Generator, M: int, N: int, K: int, act: str, kind: int) -> dict:
    X = g.integers(-2, 3, (M, K)).astype(np.int8)
    W = g.integers(-2, 3, (K, N)).astype(np.int8)
    dY = g.integers(-2, 3, (M, N)).astype(np.int8)
    nb = {BIAS_NONE: 0, BIAS_SCALAR: 1, BIAS_PERM: M, BIAS_PERN: N}[kind]
    b = g.integers(-2, 3, (nb,)).astype(np.int8)
    Xl, Wl, dYl, bl = X.tolist(), W.tolist(), dY.tolist(), b.tolist()

    Z = [[0] * N for _ in range(M)]
    for i in range(M):
        for j in range(N):
            s = 0
            for k in range(K):
                s += Xl[i][k] * Wl[k][j]
            if kind == BIAS_SCALAR:
                s += bl[0]
            elif kind == BIAS_PERM:
                s += bl[i]
            elif kind == BIAS_PERN:
                s += bl[j]
            Z[i][j] = s
    # Y and gZ scaled by 4
    Y4 = [[0] * N for _ in range(M)]
    gZ4 = [[0] * N for _ in range(M)]
    for i in range(M):
        for j in range(N):
            z = Z[i][j]
            if act == "none":
                Y4[i][j], d4 = 4 * z, 4
            elif act == "relu":
                Y4[i][j], d4 = (4 * z if z > 0 else 0), (4 if z > 0 else 0)
            else:
                Y4[i][j], d4 = (4 * z if z > 0 else SLOPE_X4 * z), (4 if z > 0 else SLOPE_X4)
            gZ4[i][j] = dYl[i][j] * d4
    dX4 = [[sum(gZ4[i][j] * Wl[k][j] for j in range(N)) for k in range(K)] for i in range(M)]
    dW4 = [[sum(Xl[i][k] * gZ4[i][j] for i in range(M)) for j in range(N)] for k in range(K)]
    if kind == BIAS_SCALAR:
        db4 = [sum(sum(r) for r in gZ4)]
    elif kind == BIAS_PERM:
        db4 = [sum(r) for r in gZ4]
    elif kind == BIAS_PERN:
        db4 = [sum(gZ4[i][j] for i in range(M)) for j in range(N)]
    else:
        db4 = []
    q = lambda v: (np.asarray(v, dtype=np.float64) / 4.0).astype(np.float32)  # exact
    return {
        "dims": np.array([M, N, K, ACTS[act], kind], dtype=np.int32),
        "X": X, "W": W, "dY": dY, "bias": b,
        "Z": np.asarray(Z, dtype=np.float32), "Y": q(Y4),
        "dX": q(dX4), "dW": q(dW4), "dBias": q(db4),
    }


def main() -> None:
    g = np.random.default_rng(20260501)
    out = {}
    for name, M, N, K, act, kind in CASES:
        for key, val in _case(g, M, N, K, act, kind).items():
            out[f"{name}/{key}"] = val
    out["names"] = np.array([c[0] for c in CASES])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_int_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(CASES)} cases")


if __name__ == "__main__":
    main()
