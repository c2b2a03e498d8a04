#!/usr/bin/env python3
"""Benchmark of the GEMM + bias + activation operator on one MI355X.

Headline: bf16 X[4096,4096] W[4096,4096] + bias,
ReLU, Z stash; one *step* = forward + backward (gA, gB, gBias), inputs resident
in HBM.  value = 6*M*N*K / step time (TFLOP/s).

roofline: the forward GEMM+bias+ReLU kernel timed alone with HIP events on the
stream it is launched on; achieved = 2*M*N*K / average launch time, against the
dense bf16 MFMA peak (2516.6 TFLOP/s).  Beside it, the sustained rate of
back-to-back bf16 MFMAs with zero and with random operands (gev2_probe_mfma_bf16)
shows how far below the published peak the matrix cores run on real data.

cpu_baseline: the reference's NumPy path (smoke_gemm_binding.py:84-123,
restated in oracle/gemm_oracle.py) in fp32 on the host's cores, on a bounded
row-slice of the same workload.

Extra fields time the other BASELINE configs (C1, C2, C3-fp16, C4 SDPA batched,
C5a conv-as-GEMM, C5b skinny); the bandwidth-bound ones rotate buffer sets
totalling > 256 MB so that reads come from HBM, not the MALL.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "ai_framework-dev_amd"))

PEAK_BF16 = 2516.6   # dense bf16/fp16 MFMA TFLOP/s (MI355X)
PEAK_F32 = 157.3     # fp32 MFMA TFLOP/s
PEAK_HBM = 8000.0    # GB/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline only (no extra configs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of extra configs to run")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 256 MiB device-to-device copy (the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return ap.parse_args()


class Ctx:
    def __init__(self, capi):
        self.capi = capi
        self.stream = capi.Stream()
        self.bufs = []

    def put(self, a):
        b = self.capi.DeviceBuffer.from_numpy(a)
        self.bufs.append(b)
        return b.ptr

    def empty(self, nbytes):
        b = self.capi.DeviceBuffer(nbytes)
        self.bufs.append(b)
        return b.ptr

    def free(self):
        for b in self.bufs:
            b.free()
        self.bufs = []

    def time_repeat(self, descs, iters, kind="fwd", warmup=3):
        """Average ms per launch of `iters` back-to-back calls issued from C
        (gev2_gemm_*_repeat), cycling through descs; HIP events on self.stream."""
        capi = self.capi
        rep = capi.gemm_fwd_repeat if kind == "fwd" else capi.gemm_bwd_repeat
        rep(descs, warmup, self.stream.ptr)
        self.stream.synchronize()
        e0, e1 = capi.Event(), capi.Event()
        e0.record(self.stream.ptr)
        rep(descs, iters, self.stream.ptr)
        e1.record(self.stream.ptr)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / iters
        e0.destroy()
        e1.destroy()
        return ms

    def time_ms(self, fn, iters, warmup=3):
        """Average ms per call of fn() (which launches on self.stream)."""
        capi = self.capi
        for _ in range(warmup):
            fn()
        self.stream.synchronize()
        e0, e1 = capi.Event(), capi.Event()
        e0.record(self.stream.ptr)
        for _ in range(iters):
            fn()
        e1.record(self.stream.ptr)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / iters
        e0.destroy()
        e1.destroy()
        return ms


def normal(g, shape, scale=1.0):
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale))


# ---------------------------------------------------------------------------
def headline(ctx, steps, warmup, dtype, M=4096, N=4096, K=4096, seed=3):
    capi = ctx.capi
    g = np.random.default_rng(seed)
    X = capi.to_storage(normal(g, (M, K), 1 / np.sqrt(K)), dtype)
    W = capi.to_storage(normal(g, (K, N), 1 / np.sqrt(K)), dtype)
    b = normal(g, (N,), 0.02)
    gY = capi.to_storage(normal(g, (M, N)), dtype)
    es = capi.elem_bytes(dtype)
    pX, pW, pb, pgY = ctx.put(X), ctx.put(W), ctx.put(b), ctx.put(gY)
    pY, pZ = ctx.empty(M * N * es), ctx.empty(M * N * es)
    pgA, pgB, pgb = ctx.empty(M * K * es), ctx.empty(K * N * es), ctx.empty(N * 4)
    s = ctx.stream.ptr
    fd = capi.fwd_desc(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb,
                       bias_kind=capi.BIAS_PERN, act="relu")
    bd = capi.bwd_desc(dtype=dtype, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, gA=pgA, gB=pgB,
                       gBias=pgb, bias_kind=capi.BIAS_PERN, act="relu")

    def step():
        capi.gemm_fwd_repeat([fd], 1, s)
        capi.gemm_bwd_repeat([bd], 1, s)

    capi.gemm_fwd_repeat([fd], 1, s)
    path = capi.last_path()
    # timed region: exactly `steps` steps, synchronised on both sides
    for _ in range(warmup):
        step()
    ctx.stream.synchronize()
    e0, e1 = capi.Event(), capi.Event()
    t0 = time.perf_counter()
    e0.record(s)
    for _ in range(steps):
        step()
    e1.record(s)
    e1.synchronize()
    wall = time.perf_counter() - t0
    step_ms = e0.elapsed_ms(e1) / steps
    fwd_ms = ctx.time_repeat([fd], max(steps, 20), "fwd")
    bwd_ms = ctx.time_repeat([bd], max(steps, 20), "bwd")
    flop = 2.0 * M * N * K
    return {
        "step_ms": step_ms, "fwd_ms": fwd_ms, "bwd_ms": bwd_ms, "wall_s": wall, "path": path,
        "tflops_step": 3 * flop / (step_ms * 1e-3) / 1e12,
        "tflops_fwd": flop / (fwd_ms * 1e-3) / 1e12,
        "tflops_bwd": 2 * flop / (bwd_ms * 1e-3) / 1e12,
        "fwd_bytes": (M * K + K * N + 2 * M * N) * es + N * 4,
    }


def fp32_cfg(ctx, M, N, K, act, iters, seed):
    """C1 / C2: fp32 GEMM + bias + act, forward and forward+backward."""
    capi = ctx.capi
    g = np.random.default_rng(seed)
    if M == 64:
        X = g.uniform(-1, 1, (M, K)).astype(np.float32) / np.float32(np.sqrt(K))
        W = g.uniform(-1, 1, (K, N)).astype(np.float32) / np.float32(np.sqrt(K))
        b = g.uniform(-1, 1, (N,)).astype(np.float32) / np.float32(np.sqrt(K))
    else:
        X, W, b = normal(g, (M, K), 1 / np.sqrt(K)), normal(g, (K, N), 1 / np.sqrt(K)), normal(g, (N,), 0.02)
    gY = normal(g, (M, N))
    pX, pW, pb, pgY = ctx.put(X), ctx.put(W), ctx.put(b), ctx.put(gY)
    pY, pZ = ctx.empty(M * N * 4), ctx.empty(M * N * 4)
    pgA, pgB, pgb = ctx.empty(M * K * 4), ctx.empty(K * N * 4), ctx.empty(N * 4)
    fd = capi.fwd_desc(dtype=capi.F32, M=M, N=N, K=K, A=pX, B=pW, Y=pY, Z=pZ, bias=pb,
                       bias_kind=capi.BIAS_PERN, act=act)
    bd = capi.bwd_desc(dtype=capi.F32, M=M, N=N, K=K, A=pX, B=pW, gY=pgY, Z=pZ, gA=pgA, gB=pgB,
                       gBias=pgb, bias_kind=capi.BIAS_PERN, act=act)
    fwd_ms = ctx.time_repeat([fd], iters, "fwd")
    step_ms = fwd_ms + ctx.time_repeat([bd], iters, "bwd")
    flop = 2.0 * M * N * K
    return {"fwd_us": fwd_ms * 1e3, "step_us": step_ms * 1e3,
            "tflops_fwd": flop / (fwd_ms * 1e-3) / 1e12,
            "tflops_step": 3 * flop / (step_ms * 1e-3) / 1e12,
            "frac_fwd": flop / (fwd_ms * 1e-3) / 1e12 / PEAK_F32}


def sdpa_cfg(ctx, dtype, iters, sets=8):
    """C4: batched QK^T (scale 1/8, trans_b) and P.V, B*H = 64, 512x512x64."""
    capi = ctx.capi
    BH, L, D = 64, 512, 64
    es = capi.elem_bytes(dtype)
    g = np.random.default_rng(44)
    bufs = []
    for _ in range(sets):
        Q = capi.to_storage(normal(g, (BH, L, D)), dtype)
        Kt = capi.to_storage(normal(g, (BH, L, D)), dtype)
        V = capi.to_storage(normal(g, (BH, L, D)), dtype)
        logits = normal(g, (BH, L, L))
        P = np.exp(logits - logits.max(-1, keepdims=True))
        P /= P.sum(-1, keepdims=True)
        bufs.append((ctx.put(Q), ctx.put(Kt), ctx.put(V), ctx.put(capi.to_storage(P, dtype)),
                     ctx.empty(BH * L * L * es), ctx.empty(BH * L * D * es)))
    qk = [capi.fwd_desc(dtype=dtype, M=L, N=L, K=D, A=q, B=k, Y=S, trans_b=True, alpha=0.125,
                        batch=BH, stride_a=L * D, stride_b=L * D, stride_y=L * L)
          for q, k, _, _, S, _ in bufs]
    pv = [capi.fwd_desc(dtype=dtype, M=L, N=D, K=L, A=p, B=v, Y=y, batch=BH,
                        stride_a=L * L, stride_b=L * D, stride_y=L * D)
          for _, _, v, p, _, y in bufs]
    qk_ms = ctx.time_repeat(qk, iters, "fwd")
    pv_ms = ctx.time_repeat(pv, iters, "fwd")
    flop = 2.0 * BH * L * L * D
    byt_qk = (2 * BH * L * D + BH * L * L) * es
    byt_pv = (BH * L * L + 2 * BH * L * D) * es
    # the plain streaming write of S alone, and read of P alone, on this part
    wprobe = hbm_write_ceiling(ctx, nbytes=BH * L * L * es)
    rprobe = hbm_read_ceiling(ctx, nbytes=BH * L * L * es)
    return {"qk_us": qk_ms * 1e3, "pv_us": pv_ms * 1e3,
            "s_write_probe_us": wprobe["us"], "p_read_probe_us": rprobe["us"],
            "qk_gbps": byt_qk / (qk_ms * 1e-3) / 1e9, "pv_gbps": byt_pv / (pv_ms * 1e-3) / 1e9,
            "qk_frac_hbm": byt_qk / (qk_ms * 1e-3) / 1e9 / PEAK_HBM,
            "pv_frac_hbm": byt_pv / (pv_ms * 1e-3) / 1e9 / PEAK_HBM,
            "tflops_qk": flop / (qk_ms * 1e-3) / 1e12, "tflops_pv": flop / (pv_ms * 1e-3) / 1e12}


def conv_cfg(ctx, dtype, iters):
    """C5a: im2col-lowered conv2d as one GEMM, M=100352, K=576, N=128, bias + ReLU (Z saved)."""
    capi = ctx.capi
    M, K, N = 32 * 56 * 56, 64 * 9, 128
    es = capi.elem_bytes(dtype)
    g = np.random.default_rng(55)
    col = capi.to_storage(g.random((M, K), dtype=np.float32), dtype)
    W = capi.to_storage(normal(g, (K, N), np.sqrt(2 / 576)), dtype)
    b = normal(g, (N,), 0.02)
    pA, pW, pb = ctx.put(col), ctx.put(W), ctx.put(b)
    pY, pZ = ctx.empty(M * N * es), ctx.empty(M * N * es)
    fd = capi.fwd_desc(dtype=dtype, M=M, N=N, K=K, A=pA, B=pW, Y=pY, Z=pZ, bias=pb,
                       bias_kind=capi.BIAS_PERN, act="relu")
    ms = ctx.time_repeat([fd], iters, "fwd")
    flop = 2.0 * M * N * K
    byt = (M * K + K * N + 2 * M * N) * es + N * 4
    peak = PEAK_F32 if dtype == capi.F32 else PEAK_BF16
    t_roof = max(flop / (peak * 1e12), byt / (PEAK_HBM * 1e9))
    return {"fwd_us": ms * 1e3, "tflops": flop / (ms * 1e-3) / 1e12,
            "gbps": byt / (ms * 1e-3) / 1e9, "roofline_frac": t_roof / (ms * 1e-3)}


def conv_op_cfg(ctx, dtype, iters, images_per_call):
    """C5a through the conv2d operator (gev2_conv2d_fwd / _bwd): X[32,64,56,56], W[128,64,3,3],
    3x3 / stride 1 / pad 1, bias + ReLU, Z saved; im2col + batched GEMM forward, and the backward
    (dW, dB, dX) with workspaces for `images_per_call` images per batched call."""
    capi = ctx.capi
    N, Cin, H, Wd, Cout, Kh, Kw = 32, 64, 56, 56, 128, 3, 3
    K, HWo = Cin * Kh * Kw, H * Wd
    es = capi.elem_bytes(dtype)
    g = np.random.default_rng(56)
    X = capi.to_storage(g.random((N, Cin, H, Wd), dtype=np.float32), dtype)
    W = capi.to_storage(normal(g, (Cout, Cin, Kh, Kw), np.sqrt(2 / K)), dtype)
    dY = capi.to_storage(normal(g, (N, Cout, H, Wd)), dtype)
    b = normal(g, (Cout,), 0.02)
    pX, pW, pdY, pb = ctx.put(X), ctx.put(W), ctx.put(dY), ctx.put(b)
    pY, pZ = ctx.empty(N * Cout * HWo * es), ctx.empty(N * Cout * HWo * es)
    pdW, pdB, pdX = ctx.empty(Cout * K * es), ctx.empty(Cout * 4), ctx.empty(N * Cin * H * Wd * es)
    c = images_per_call
    col_bytes = c * K * HWo * es
    pcol, pdcol, pgw = ctx.empty(col_bytes), ctx.empty(col_bytes), ctx.empty(c * Cout * K * es)
    acc_b_bytes = (c + 1) * Cout * 4
    pacc_w, pacc_b = ctx.empty(Cout * K * 4), ctx.empty(acc_b_bytes)
    dz_bytes = ((c * Cout * HWo * es + 255) // 256) * 256
    pdz = ctx.empty(dz_bytes)
    geom = dict(N=N, Cin=Cin, H=H, W=Wd, Cout=Cout, Kh=Kh, Kw=Kw, stride_h=1, stride_w=1, pad_h=1, pad_w=1,
                dil_h=1, dil_w=1, groups=1)
    fd = capi.Conv2dDesc(dtype=dtype, act=capi.ACT["relu"], save_z=1, X=pX, Wt=pW, bias=pb, Y=pY, Z=pZ,
                         col=pcol, col_bytes=col_bytes, **geom)
    bd = capi.Conv2dBwdDesc(dtype=dtype, act=capi.ACT["relu"], X=pX, Wt=pW, dY=pdY, Z=pZ, dW=pdW, dB=pdB, dX=pdX,
                            col=pcol, col_bytes=col_bytes, dcol=pdcol, dcol_bytes=col_bytes, gw=pgw,
                            gw_bytes=c * Cout * K * es, acc_b=pacc_b, acc_b_bytes=acc_b_bytes, acc_w=pacc_w,
                            dz=pdz, dz_bytes=dz_bytes, **geom)
    L = capi.lib()

    def fwd():
        capi.check_conv(L.gev2_conv2d_fwd(ctypes.byref(fd), ctx.stream.ptr), "conv fwd")

    def bwd():
        capi.check_conv(L.gev2_conv2d_bwd(ctypes.byref(bd), ctx.stream.ptr), "conv bwd")

    fwd_ms = ctx.time_ms(fwd, iters)
    bwd_ms = ctx.time_ms(bwd, iters)
    flop = 2.0 * N * HWo * K * Cout
    return {"images_per_call": c, "fwd_us": fwd_ms * 1e3, "bwd_us": bwd_ms * 1e3,
            "tflops_fwd": flop / (fwd_ms * 1e-3) / 1e12, "tflops_bwd": 2 * flop / (bwd_ms * 1e-3) / 1e12}


def rnn_op_cfg(ctx, dtype, iters, N=8, T=32, I=512, H=1024):
    """Elman RNN through the operator (gev2_rnn_fwd / _bwd): X[N,T,I], tanh, bias, Z saved;
    forward (T steps of gather + one operator GEMM [N, I+H] x [I+H, H]) and the backward through
    time (dWx, dWh, dB, dh0, dX)."""
    capi = ctx.capi
    es = capi.elem_bytes(dtype)
    g = np.random.default_rng(57)
    X = capi.to_storage(normal(g, (N, T, I)), dtype)
    Wx = capi.to_storage(normal(g, (I, H), 1 / np.sqrt(I)), dtype)
    Wh = capi.to_storage(normal(g, (H, H), 0.5 / np.sqrt(H)), dtype)
    h0 = capi.to_storage(normal(g, (N, H)), dtype)
    dY = capi.to_storage(normal(g, (N, T, H)), dtype)
    b = normal(g, (H,), 0.1)
    pX, pWx, pWh, ph0, pdY, pb = (ctx.put(a) for a in (X, Wx, Wh, h0, dY, b))
    pY, pZ = ctx.empty(N * T * H * es), ctx.empty(N * T * H * es)
    IH = I + H
    pxh, pwcat = ctx.empty(N * IH * es), ctx.empty(IH * H * es)
    ws_bytes = 8 << 20
    pws = ctx.empty(ws_bytes)
    fd = capi.RnnDesc(dtype=dtype, act=capi.ACT["tanh"], save_z=1, N=N, T=T, I=I, H=H, X=pX, Wx=pWx, Wh=pWh,
                      bias=pb, h0=ph0, Y=pY, Z=pZ, xh=pxh, wcat=pwcat, ws=pws, ws_bytes=ws_bytes)
    bd = capi.RnnBwdDesc(dtype=dtype, act=capi.ACT["tanh"], N=N, T=T, I=I, H=H, X=pX, Wx=pWx, Wh=pWh, h0=ph0,
                         dY=pdY, Z=pZ, dWx=ctx.empty(I * H * es), dWh=ctx.empty(H * H * es), dB=ctx.empty(H * 4),
                         dh0=ctx.empty(N * H * es), dX=ctx.empty(N * T * I * es), xh=pxh, g=ctx.empty(N * H * es),
                         wcat=pwcat, dxh=ctx.empty(N * IH * es), dwcat=ctx.empty(IH * H * 4),
                         tmpw=ctx.empty(IH * H * es), gb=ctx.empty(H * 4), ws=pws, ws_bytes=ws_bytes)
    L = capi.lib()

    def fwd():
        capi.check_rnn(L.gev2_rnn_fwd(ctypes.byref(fd), ctx.stream.ptr), "rnn fwd")

    def bwd():
        capi.check_rnn(L.gev2_rnn_bwd(ctypes.byref(bd), ctx.stream.ptr), "rnn bwd")

    fwd_ms = ctx.time_ms(fwd, iters)
    bwd_ms = ctx.time_ms(bwd, iters)
    return {"shape": f"N={N} T={T} I={I} H={H} tanh", "fwd_us": fwd_ms * 1e3, "bwd_us": bwd_ms * 1e3,
            "fwd_us_per_step": fwd_ms * 1e3 / T, "bwd_us_per_step": bwd_ms * 1e3 / T}


def attn_cfg(ctx, dtype, iters, B=8, H=8, M=512, N=512, D=64, causal=False, sets=8):
    """C4 shape through the attention entry point (gev2_sdpa_fwd): fused kernel for 16-bit
    tensors (S and P never leave the chip), the batched fp32 path otherwise; `sets` buffer sets
    rotate so that the MALL does not hold the inputs between launches."""
    capi = ctx.capi
    es = capi.elem_bytes(dtype)
    g = np.random.default_rng(58)
    L = capi.lib()
    descs = []
    for _ in range(sets):
        Q, K, V = (capi.to_storage(normal(g, s), dtype) for s in ((B, H, M, D), (B, H, N, D), (B, H, N, D)))
        d = capi.SdpaDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, causal=int(causal), Q=ctx.put(Q), K=ctx.put(K),
                          V=ctx.put(V), Y=ctx.empty(B * H * M * D * es), lse=ctx.empty(B * H * M * 4))
        wsb = L.gev2_sdpa_workspace_size(ctypes.byref(d), 0)
        if wsb > 0:
            d.workspace, d.workspace_bytes = ctx.empty(wsb), wsb
            d.lse = None
        descs.append(d)
    it = [0]

    def fwd():
        d = descs[it[0] % sets]
        it[0] += 1
        capi.check_sdpa(L.gev2_sdpa_fwd(ctypes.byref(d), ctx.stream.ptr), "sdpa fwd")

    ms = ctx.time_ms(fwd, iters)
    flop = 4.0 * B * H * M * N * D * (0.5 if causal else 1.0)
    byt = (B * H * (M + 2 * N) * D + B * H * M * D) * es + B * H * M * 4
    return {"shape": f"B={B} H={H} M={M} N={N} D={D}" + (" causal" if causal else ""), "fwd_us": ms * 1e3,
            "tflops": flop / (ms * 1e-3) / 1e12, "gbps_algorithmic": byt / (ms * 1e-3) / 1e9}


def attn_bwd_cfg(ctx, dtype, iters, B=8, H=8, M=512, N=512, D=64, causal=False):
    """C4 shape through gev2_sdpa_bwd (dQ, dK, dV): for 16-bit tensors the fused backward
    (forward recomputed for O and lse, Dq, dK/dV kernel, dQ kernel); GEV2_ATTN_BWD_WIDE=1 selects
    the batched fp32 path on widened copies."""
    capi = ctx.capi
    es = capi.elem_bytes(dtype)
    g = np.random.default_rng(59)
    L = capi.lib()
    Q, K, V, dY = (capi.to_storage(normal(g, s), dtype) for s in ((B, H, M, D), (B, H, N, D), (B, H, N, D),
                                                                    (B, H, M, D)))
    fd = capi.SdpaDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, causal=int(causal))
    wsb = L.gev2_sdpa_workspace_size(ctypes.byref(fd), 1)
    d = capi.SdpaBwdDesc(dtype=dtype, B=B, H=H, M=M, N=N, D=D, causal=int(causal), Q=ctx.put(Q), K=ctx.put(K),
                         V=ctx.put(V), dY=ctx.put(dY), dQ=ctx.empty(B * H * M * D * es),
                         dK=ctx.empty(B * H * N * D * es), dV=ctx.empty(B * H * N * D * es),
                         workspace=ctx.empty(wsb), workspace_bytes=wsb)

    def bwd():
        capi.check_sdpa(L.gev2_sdpa_bwd(ctypes.byref(d), ctx.stream.ptr), "sdpa bwd")

    ms = ctx.time_ms(bwd, iters)
    flop = 10.0 * B * H * M * N * D * (0.5 if causal else 1.0)    # incl. the recomputed forward
    return {"shape": f"B={B} H={H} M={M} N={N} D={D}" + (" causal" if causal else ""), "bwd_us": ms * 1e3,
            "tflops": flop / (ms * 1e-3) / 1e12, "workspace_bytes": wsb}


def skinny_cfg(ctx, iters, sets=10):
    """C5b: bf16 M=8, N=K=4096 + bias; 10 distinct W (335 MB) rotate past the MALL.
    The split-K partials go to a caller workspace (gev2_gemm_fwd_workspace_size)."""
    capi = ctx.capi
    M, N, K = 8, 4096, 4096
    g = np.random.default_rng(66)
    X = capi.to_storage(normal(g, (M, K), 1 / np.sqrt(K)), capi.BF16)
    pX = ctx.put(X)
    pb = ctx.put(normal(g, (N,), 0.02))
    Ws = [ctx.put(capi.to_storage(normal(g, (K, N), 1 / np.sqrt(K)), capi.BF16)) for _ in range(sets)]
    pY = ctx.empty(M * N * 2)
    kw = dict(dtype=capi.BF16, M=M, N=N, K=K, A=pX, Y=pY, bias=pb, bias_kind=capi.BIAS_PERN, act="none")
    need = capi.fwd_workspace_size(B=Ws[0], **kw)
    ws = ctx.empty(max(need, 256))
    fds = [capi.fwd_desc(B=w, workspace=ws, workspace_bytes=need, **kw) for w in Ws]
    capi.gemm_fwd_repeat(fds, 1, ctx.stream.ptr)
    path = capi.last_path()
    ms = ctx.time_repeat(fds, iters, "fwd")
    byt = (M * K + K * N + M * N) * 2 + N * 4
    probe = hbm_read_ceiling(ctx)
    gbps = byt / (ms * 1e-3) / 1e9
    return {"fwd_us": ms * 1e3, "gbps": gbps, "frac_hbm": gbps / PEAK_HBM, "path": path,
            "read_probe_gbps": probe["gbps"], "read_probe_us": probe["us"],
            "frac_of_read_probe": gbps / probe["gbps"]}


def cpu_baseline(M=4096, N=4096, K=4096, min_seconds=10.0, max_reps=200):
    """fp32 NumPy forward+backward (the reference's CPU path) on the full C3 step,
    repeated until about min_seconds of CPU work; the median step is reported."""
    from oracle import gemm_oracle as O
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        blas = ",".join(sorted({i.get("internal_api", "?") for i in threadpool_info()}))
    except Exception:
        threads, blas = len(os.sched_getaffinity(0)), "?"
    g = np.random.default_rng(7)
    X = normal(g, (M, K), 1 / np.sqrt(K))
    W = normal(g, (K, N), 1 / np.sqrt(K))
    b = normal(g, (1, N), 0.02)
    gY = normal(g, (M, N))
    O.numpy_fp32_step(X, W, b, gY, "relu")   # warm-up
    ts = []
    while len(ts) < max_reps and (len(ts) < 3 or sum(ts) < min_seconds):
        t0 = time.perf_counter()
        O.numpy_fp32_step(X, W, b, gY, "relu")
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    flop = 6.0 * M * N * K
    return {"value": flop / t / 1e12, "unit": "TFLOP/s", "cores": int(threads),
            "kind": "port",
            "sample": f"fp32 numpy forward+backward (np.matmul via {blas}) of the full {M}x{K} @ "
                      f"{K}x{N} ReLU step, {len(ts)} repetitions ({sum(ts):.1f} s wall on {threads} threads), "
                      f"median {t * 1e3:.1f} ms per step",
            "per_config": cpu_config_baselines()}


def _cpu_time(fn, budget_s, max_reps=50):
    """Median seconds of fn() over repetitions filling about budget_s (at least 3)."""
    fn()
    ts = []
    while len(ts) < max_reps and (len(ts) < 3 or sum(ts) < budget_s):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)


def cpu_config_baselines(budget_s=3.0):
    """The other BASELINE configs on the same host cores, fp32 numpy (the reference's CPU
    path as the oracle restates it): C1 and C2 forward + backward steps, C4's two batched
    products, and C5a's im2col-lowered forward with im2col timed on its own."""
    from oracle import gemm_oracle as O
    out = {}
    g = np.random.default_rng(8)
    for key, (M, N, K, act) in (("c1_mlp_f32_64x784x256_relu", (64, 256, 784, "relu")),
                                ("c2_f32_1024_gelu", (1024, 1024, 1024, "gelu"))):
        X = normal(g, (M, K), 1 / np.sqrt(K))
        W = normal(g, (K, N), 1 / np.sqrt(K))
        b = normal(g, (1, N), 0.02)
        gY = normal(g, (M, N))
        t, n = _cpu_time(lambda: O.numpy_fp32_step(X, W, b, gY, act), budget_s)
        out[key] = {"step_us": t * 1e6, "tflops_step": 6.0 * M * N * K / t / 1e12, "reps": n}
    # C4: 64 slices of Q K^T (scale 1/8) then P V, [64,512,64]
    Q, Kt, V = (normal(g, (64, 512, 64)) for _ in range(3))
    P = normal(g, (64, 512, 512))
    t_qk, n1 = _cpu_time(lambda: np.matmul(Q, Kt.transpose(0, 2, 1)) * np.float32(0.125), budget_s)
    t_pv, n2 = _cpu_time(lambda: np.matmul(P, V), budget_s)
    f = 2.0 * 64 * 512 * 512 * 64
    out["c4_sdpa_batched_f32"] = {"qk_us": t_qk * 1e6, "pv_us": t_pv * 1e6, "tflops_qk": f / t_qk / 1e12,
                                  "tflops_pv": f / t_pv / 1e12, "reps": n1 + n2}
    # C5a: X[32,64,56,56], W[128,64,3,3], stride 1, pad 1: col[n, (c,kh,kw), hw], then W col + b, ReLU
    N_, C, H, Wd, Co = 32, 64, 56, 56, 128
    Xc = g.random((N_, C, H, Wd), dtype=np.float32)
    Wc = normal(g, (Co, C * 9), np.sqrt(2 / 576))
    bc = normal(g, (1, Co, 1), 0.02)
    Ho, Wo = O.conv2d_out_size(H, Wd, 3, 3, (1, 1), (1, 1), (1, 1))

    def im2col():
        Xp = np.pad(Xc, ((0, 0), (0, 0), (1, 1), (1, 1)))
        col = np.empty((N_, C, 9, Ho * Wo), np.float32)
        for kh in range(3):
            for kw in range(3):
                col[:, :, kh * 3 + kw, :] = O._window(Xp, kh, kw, Ho, Wo, (1, 1), (1, 1)).reshape(N_, C, Ho * Wo)
        return col.reshape(N_, C * 9, Ho * Wo)

    col = im2col()
    t_col, n1 = _cpu_time(im2col, budget_s, max_reps=10)
    t_gemm, n2 = _cpu_time(lambda: np.maximum(np.matmul(Wc, col) + bc, np.float32(0)), budget_s, max_reps=10)
    f = 2.0 * N_ * Ho * Wo * 576 * Co
    out["c5a_conv_f32"] = {"im2col_us": t_col * 1e6, "gemm_us": t_gemm * 1e6, "fwd_us": (t_col + t_gemm) * 1e6,
                           "tflops_gemm": f / t_gemm / 1e12, "tflops_fwd": f / (t_col + t_gemm) / 1e12,
                           "reps": n1 + n2}
    return {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
            for k, v in out.items()}


def measured_traffic():
    """HBM bytes per forward launch, as recorded from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (scaled by a copy of known size) in profiles/; None if absent."""
    path = os.path.join(REPO, "profiles", "gemm_dl_bf16_256x256_nn_4096_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def mfma_ceiling(ctx, iters=4096):
    """Sustained back-to-back bf16 MFMA rate (TFLOP/s) with zero and with random operands
    (gev2_probe_mfma_bf16): the clock the matrix cores hold depends on the data."""
    capi = ctx.capi
    _, cus, _ = capi.device_info(0)
    flop = cus * 4 * iters * 16 * 32768.0
    out = {}
    for name, rnd in (("zero", 0), ("random", 1)):
        ms = ctx.time_ms(lambda: capi.check(capi.lib().gev2_probe_mfma_bf16(rnd, iters, ctx.stream.ptr),
                                            "probe"), 10, warmup=2)
        out[name] = round(flop / (ms * 1e-3) / 1e12, 1)
    return out


def hbm_read_ceiling(ctx, nbytes=32 << 20, sets=10, reps=50):
    """Rate of the fastest plain streaming read of nbytes on this part
    (gev2_probe_hbm_read: 2048 workgroups, eight 16-byte loads in flight per
    thread, the best of a sweep over 256-4096 workgroups and 8-32 loads),
    rotating `sets` buffers past the MALL: the ceiling for a kernel that must
    read that many bytes once."""
    capi = ctx.capi
    lib = capi.lib()
    buf = ctx.empty(nbytes * sets)
    capi.check(lib.gev2_memset(buf, 0, nbytes * sets), "memset")
    ms = ctx.time_ms(lambda: capi.check(lib.gev2_probe_hbm_read(buf, nbytes, sets, reps, 2048, 8, ctx.stream.ptr),
                                        "read probe"), 3, warmup=1) / reps
    return {"bytes": nbytes, "us": round(ms * 1e3, 3), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def hbm_write_ceiling(ctx, nbytes=32 << 20, sets=10, reps=50):
    """Rate of the fastest plain streaming write of nbytes on this part
    (gev2_probe_hbm_write: 512 workgroups, sixteen 16-byte stores per thread,
    the best of a sweep over 512-4096 workgroups and 4-16 stores), rotating
    `sets` buffers: the ceiling for a kernel that must write that many bytes."""
    capi = ctx.capi
    lib = capi.lib()
    buf = ctx.empty(nbytes * sets)
    ms = ctx.time_ms(lambda: capi.check(lib.gev2_probe_hbm_write(buf, nbytes, sets, reps, 512, 16, ctx.stream.ptr),
                                        "write probe"), 3, warmup=1) / reps
    return {"bytes": nbytes, "us": round(ms * 1e3, 3), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def kernel_name(path):
    return {"dl": "gemm_dl_kernel", "tile": "gemm_pipe_kernel"}.get(path.split(":")[0], path)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the operator's multi-GPU "
                          "sharding is a design, not code; run with --gpus 1"}))
        return 2
    from graph_executor_v2.ops import capi
    capi.lib()
    if capi.device_count() < 1:
        raise SystemExit("no HIP device visible")
    name, cus, clk = capi.device_info(0)
    ctx = Ctx(capi)
    if args.calib_copy:
        nb = 256 << 20
        src, dst = ctx.empty(nb), ctx.empty(nb)
        capi.check(capi.lib().gev2_memcpy_dtod_async(dst, src, nb, ctx.stream.ptr), "calib copy")
        ctx.stream.synchronize()
        ctx.free()
    res = headline(ctx, args.steps, args.warmup, capi.BF16)
    print(f"# headline bf16 4096^3: step {res['step_ms']:.3f} ms, fwd {res['fwd_ms'] * 1e3:.1f} us "
          f"({res['tflops_fwd']:.0f} TFLOP/s), bwd {res['bwd_ms'] * 1e3:.1f} us", file=sys.stderr, flush=True)
    ctx.free()
    extra = {"device": name, "cus": cus, "peak_clock_mhz": clk / 1000.0,
             "fwd_ms": res["fwd_ms"], "bwd_ms": res["bwd_ms"], "path": res["path"],
             "tflops_fwd": res["tflops_fwd"], "tflops_bwd": res["tflops_bwd"]}
    if not args.quick:
        only = set(filter(None, args.only.split(",")))
        todo = [
            ("c1_mlp_f32_64x784x256_relu", lambda: fp32_cfg(ctx, 64, 256, 784, "relu", 200, 1)),
            ("c2_f32_1024_gelu", lambda: fp32_cfg(ctx, 1024, 1024, 1024, "gelu", 50, 2)),
            ("c3_f16_4096_relu", lambda: headline(ctx, 10, 3, capi.F16)),
            ("c4_sdpa_bf16", lambda: sdpa_cfg(ctx, capi.BF16, 50)),
            ("c4_attn_fused_bf16", lambda: attn_cfg(ctx, capi.BF16, 50)),
            ("c4_attn_fused_bf16_causal", lambda: attn_cfg(ctx, capi.BF16, 50, causal=True)),
            ("c4_attn_f32", lambda: attn_cfg(ctx, capi.F32, 10, sets=2)),
            ("c4_attn_bwd_bf16", lambda: attn_bwd_cfg(ctx, capi.BF16, 20)),
            ("c4_attn_bwd_bf16_causal", lambda: attn_bwd_cfg(ctx, capi.BF16, 20, causal=True)),
            ("attn_long_d128_bf16", lambda: attn_cfg(ctx, capi.BF16, 20, B=2, H=16, M=2048, N=2048, D=128, sets=2)),
            ("attn_long_d128_bwd_bf16", lambda: attn_bwd_cfg(ctx, capi.BF16, 10, B=2, H=16, M=2048, N=2048, D=128)),
            ("attn_long_d64_bf16", lambda: attn_cfg(ctx, capi.BF16, 20, B=2, H=32, M=2048, N=2048, D=64, sets=2)),
            ("c5a_conv_f32", lambda: conv_cfg(ctx, capi.F32, 20)),
            ("c5a_conv_bf16", lambda: conv_cfg(ctx, capi.BF16, 20)),
            ("c5a_conv2d_op_f32_per_image", lambda: conv_op_cfg(ctx, capi.F32, 5, 1)),
            ("c5a_conv2d_op_f32", lambda: conv_op_cfg(ctx, capi.F32, 5, 32)),
            ("c5a_conv2d_op_bf16", lambda: conv_op_cfg(ctx, capi.BF16, 10, 32)),
            ("c5b_skinny_bf16", lambda: skinny_cfg(ctx, 100)),
            ("rnn_op_f32", lambda: rnn_op_cfg(ctx, capi.F32, 10)),
            ("rnn_op_bf16", lambda: rnn_op_cfg(ctx, capi.BF16, 10)),
        ]
        for key, fn in todo:
            if only and key not in only:
                continue
            r = fn()
            ctx.free()
            if key == "c3_f16_4096_relu":
                r = {k: r[k] for k in ("step_ms", "fwd_ms", "bwd_ms", "tflops_step", "tflops_fwd")}
            extra[key] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
            print(f"# {key}: {extra[key]}", file=sys.stderr, flush=True)
    ceiling = mfma_ceiling(ctx)
    print(f"# mfma probe: {ceiling}", file=sys.stderr, flush=True)
    flop = 2.0 * 4096 ** 3
    achieved = flop / (res["fwd_ms"] * 1e-3) / 1e12
    line = {
        "metric": "GEMM+bias+act TFLOP/s and % MFMA peak at 4096^3 bf16; fwd+bwd step ms",
        "value": round(res["tflops_step"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1/K) X and W, N(0,0.02) bias, N(0,1) dY)",
        "config": {"workload": "C3: Y=ReLU(X W + b), X[4096,4096] W[4096,4096] bf16, fp32 accumulate, "
                               "Z saved; step = forward + backward (dX, dW, dBias)",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4), "traffic": measured_traffic(),
                     "kernel": kernel_name(res["path"]) + " (forward, bf16, " + res["path"] + ")",
                     "flop_per_launch": flop,
                     "mfma_probe_tflops": ceiling,
                     "frac_of_random_operand_probe": round(achieved / ceiling["random"], 4)},
        "extra": extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
