#!/usr/bin/env python
"""Benchmark of the Mamba-2 SSD / decode / KDA scan path on one MI355X (gfx950).

Headline (``value``): SSD chunked-scan prefill throughput in Mtok/s at the
1b shape ``ssd2`` (b2 L4096 H64 P64 N128 G1, bf16 I/O, fp32 final state),
with inputs resident in HBM.  A step is one ``selective_scan`` pass over one
batch; three input/output buffer sets rotate so the 256 MB MALL cannot serve
a step from the previous one.  The same JSON line carries:

* ``roofline`` -- one launch of the prefill op (``mh_ssd_chunk_scan_fwd``: the
  ``ssd_lb_state_kernel`` (chunk states) and ``ssd_lb_scan_kernel`` (look-back +
  scan) dispatches): algorithmic bytes per launch (compulsory I/O only) / average
  launch duration from HIP events on the launch stream, against 8 TB/s (the op is
  HBM-bound by intensity).
* ``cpu_baseline`` -- the reference's pure-PyTorch CPU prefill
  (``oracle/baseline.py``, mamba2.py:84-126 structure) timed on the host cores
  on a bounded token sample of the same workload, with the CPU model, core counts
  and torch threads; ``other`` holds the decode step at B = 64 and 256 and the
  reference-mode KDA operator at the kda5 shape.
* ``decode`` -- selective state update at B=64 and B=256 (HBM GB/s vs 8 TB/s).
* ``other`` -- ssd4 (128K prefill with state carry), kda5 (gated KDA scan), ssd2_bwd (the backward of
  the ssd2 prefill: all input gradients from dy and d_final) and kda5_bwd (the backward of the reference-mode
  KDA scan with the fused differential output at the kda5 shape: dq1, dq2, dk, dv and d lambda), conv1d (the
  layer's conv + SiLU forward and backward at the ssd2 layer shape), kda5_ref (the reference-mode scan at the kda5
  shape) and kda_step (the KDA decode step, B 64, H 32).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu] [--only LEGS]
                       [--copy-calibration BYTES]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8.0e12        # B/s, MI355X HBM3E
PEAK_BF16 = 2.5e15       # FLOP/s, dense bf16 MFMA
METRIC = "SSD prefill Mtok/s (% MFMA/HBM roofline) + decode-step HBM GB/s vs peak"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


# ----------------------------------------------------------------- algorithmic counts (compulsory I/O, dense FLOPs)

def ssd_alg(cfg, Q=256, gated=False):
    """Bytes: x, B, C, dt read once, y and the fp32 final state written once (+ h0 read, + z read with the gate);
    A, D (2H floats) omitted.  FLOPs: per (b, chunk of Q): 2Q^2 N G (C B^T) + H (2Q^2 P + 4 Q N P)."""
    b, L, H, P, N, G = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    es = 2 if cfg.dtype == torch.bfloat16 else 4
    nbytes = ((3 if gated else 2) * b * L * H * P * es + 2 * b * L * G * N * es + b * L * H * 4
              + b * H * P * N * 4 * (2 if cfg.init_state else 1))
    nchunks = L // Q
    flops = b * nchunks * (2 * Q * Q * N * G + H * (2 * Q * Q * P + 4 * Q * N * P))
    return nbytes, flops


def ssd_bwd_alg(cfg, Q=64):
    """Backward of the prefill.  Bytes: x, dy, B, C, dt and d_final read once; dx, dB, dC, ddt and the fp32 dh0
    written once (+ h0 read).  FLOPs per (b, 64-token segment): 2 Q^2 N G (C B^T) + H (4 Q^2 P + 4 Q^2 N +
    10 Q P N): dy x^T, the dx / dB / dC token-pair products, their four state products, the adjoint update and the
    forward state recompute."""
    b, L, H, P, N, G = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    es = 2 if cfg.dtype == torch.bfloat16 else 4
    nbytes = (3 * b * L * H * P * es + 4 * b * L * G * N * es + 2 * b * L * H * 4
              + b * H * P * N * 4 * (3 if cfg.init_state else 2))
    nseg = -(-L // Q)
    flops = b * nseg * (2 * Q * Q * N * G + H * (4 * Q * Q * P + 4 * Q * Q * N + 10 * Q * P * N))
    return nbytes, flops


def decode_alg(cfg):
    """Bytes: fp32 state read + written, x and y, B, C, dt, A, D, dt_bias."""
    b, H, P, N, G = cfg.batch, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    es = 2 if cfg.dtype == torch.bfloat16 else 4
    return 2 * b * H * P * N * 4 + 2 * b * H * P * es + 2 * b * G * N * es + b * H * 4 + 3 * H * 4


def kda_alg(cfg):
    """Bytes: q1, q2, k, v (bf16), g (fp32) read, o (bf16) and the fp32 final state written.
    FLOPs (q_e = q1 - lam q2 fused): per (b, h, chunk Q): 2Q^2 K + 2Q^2 V + 2QKV (read-out) + 2QKV (state)."""
    B, H, S, K, V, Q = cfg.batch, cfg.nheads, cfg.seqlen, cfg.dk, cfg.dv, cfg.chunk
    nbytes = B * H * S * (3 * K * 2 + V * 2 + K * 4 + V * 2) + B * H * K * V * 4
    flops = B * H * (S // Q) * (2 * Q * Q * K + 2 * Q * Q * V + 4 * Q * K * V)
    return nbytes, flops


def kda_bwd_alg(cfg):
    """Backward of the reference-mode scan with the fused differential output (the training path of
    LinearDiffAttention): q1, q2, k, v, dout read and dq1, dq2, dk, dv written (bf16).  FLOPs of the chunked
    gradient per (b, h, chunk Q), both queries: the recomputed forward products (A, A V, phi(q) S), the
    gradient products (G, G phi(k), dnum S^T, W g, phi(k) dS, Psi M, dS v) and the two state updates."""
    B, H, S, K, V, Q = cfg.batch, cfg.nheads, cfg.seqlen, cfg.dk, cfg.dv, 64
    nbytes = B * H * S * (5 * K * 2 + 4 * V * 2)
    per_q = 2 * Q * Q * (2 * K + 2 * V) + 3 * 2 * Q * K * V       # kernel A, one query
    comb = 2 * Q * Q * (3 * K + 2 * V) + 3 * 2 * Q * K * V        # kernel B, combined stream
    flops = B * H * (S // Q) * (2 * per_q + comb)
    return nbytes, flops


# ----------------------------------------------------------------- timing

def time_plans(plans, steps, warmup):
    """Spin up the clocks, warm up `warmup` launches, then time exactly `steps` launches cycling through `plans`.

    Returns (wall ms/step, HIP-event ms/step).  Events are recorded on the
    current torch stream, which is the stream the plans launch on.
    """
    # bring the GPU to its working clocks first (about 0.3 s of the same launches), then the W warmup steps
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < 0.3:
        plans[i % len(plans)]()
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    for i in range(warmup):
        plans[i % len(plans)]()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for i in range(steps):
        plans[i % len(plans)]()
    ev1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, ev0.elapsed_time(ev1) / steps


def bench_ssd(cfg, steps, warmup, nsets, chunk=None, gated=False):
    """The prefill op (plans on `nsets` rotating buffer sets); `gated`: with the output gate y * silu(z) fused into
    the stores (the form Mamba2Block.forward runs, mamba2.py:337-338), z drawn like x."""
    import mamformer_amd as mh
    from mamformer_amd import workloads as W

    plans = []
    for i in range(nsets):
        inp = W.ssd_inputs(cfg.scaled(seed=cfg.seed + 1000 * i), device="cuda")
        z = torch.randn_like(inp["x"]) if gated else None
        plans.append(mh.plan_selective_scan(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"],
                                            return_final_state=True, initial_state=inp["initial_state"],
                                            chunk_size=chunk, z=z))
    wall, ev = time_plans(plans, steps, warmup)
    nbytes, flops = ssd_alg(cfg, gated=gated)
    t = ev * 1e-3
    chunk_len = mh.ssd_chunk_len(cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups,
                                 cfg.dtype, chunk)
    t_roof = max(nbytes / PEAK_HBM, flops / PEAK_BF16)
    res = dict(mtok_s=cfg.batch * cfg.seqlen / t / 1e6, us_per_step=ev * 1e3, wall_us_per_step=wall * 1e3,
               alg_bytes=nbytes, alg_flops=flops, hbm_GBs=nbytes / t / 1e9, tflops=flops / t / 1e12,
               roofline_frac=t_roof / t, chunk_len=chunk_len)
    del plans
    torch.cuda.empty_cache()
    return res, wall, ev


def bench_ssd_hstates(cfg, steps, warmup):
    """Cost of return_h_states at the headline shape: selective_scan with and without h_states through the same
    Python entry (allocation of outputs and workspace included in both), and the h_states computation alone
    (``mh_ssd_h_states``: the local, carry and output kernels over the state's channel sums, reading the sums of
    x per half head that the prefill writes alongside y, ``xsum``)."""
    import mamformer_amd as mh
    from mamformer_amd import ops
    from mamformer_amd import workloads as W

    inp = W.ssd_inputs(cfg, device="cuda")
    args = (inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"])
    x4 = inp["x"]
    B4 = inp["B"] if inp["B"].dim() == 4 else inp["B"].unsqueeze(2)
    with torch.no_grad():
        _, plain = time_plans([lambda: mh.selective_scan(*args, return_final_state=True)], steps, warmup)
        _, both = time_plans([lambda: mh.selective_scan(*args, return_h_states=True, return_final_state=True)],
                             steps, warmup)
        b_, L_, H_, P_ = x4.shape
        xsum = x4.float().view(b_, L_, H_, 2, P_ // 2).sum(-1).contiguous()
        _, alone = time_plans([lambda: ops._h_states(x4, inp["dt"], inp["A"], B4, None, None, False, None, None,
                                                     xsum=xsum)], steps, warmup)
    # training: forward + backward of <gy, y> (+ <ghs, h_states>) through autograd
    leaves = [t.clone().requires_grad_() for t in (inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"])]
    gy = torch.randn_like(inp["x"])
    ghs = torch.randn((cfg.batch, cfg.seqlen, cfg.dstate), device="cuda", dtype=inp["x"].dtype)

    def train(with_hs):
        def step():
            out = mh.selective_scan(*leaves, return_h_states=with_hs)
            y = out[0] if with_hs else out
            loss = (y.float() * gy.float()).sum()
            if with_hs:
                loss = loss + (out[1].float() * ghs.float()).sum()
            torch.autograd.grad(loss, leaves)
        return step

    _, tr_plain = time_plans([train(False)], max(5, steps // 5), 2)
    _, tr_both = time_plans([train(True)], max(5, steps // 5), 2)
    del inp
    torch.cuda.empty_cache()
    return dict(us_plain=plain * 1e3, us_with_h_states=both * 1e3, us_h_states=alone * 1e3,
                overhead=both / plain, us_train_plain=tr_plain * 1e3, us_train_with_h_states=tr_both * 1e3)


def bench_ssd_bwd(cfg, steps, warmup, nsets):
    import mamformer_amd as mh
    from mamformer_amd import workloads as W

    plans = []
    for i in range(nsets):
        c = cfg.scaled(seed=cfg.seed + 1000 * i)
        inp = W.ssd_inputs(c, device="cuda")
        g = torch.Generator(device="cuda").manual_seed(c.seed + 7)
        dy = torch.randn(inp["x"].shape, device="cuda", generator=g).to(inp["x"].dtype)
        dfin = 0.1 * torch.randn((c.batch, c.nheads, c.headdim, c.dstate), device="cuda", generator=g)
        plans.append(mh.plan_selective_scan_bwd(dy, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"],
                                                d_final_state=dfin, initial_state=inp["initial_state"]))
    wall, ev = time_plans(plans, steps, warmup)
    nbytes, flops = ssd_bwd_alg(cfg)
    t = ev * 1e-3
    t_roof = max(nbytes / PEAK_HBM, flops / PEAK_BF16)
    res = dict(mtok_s=cfg.batch * cfg.seqlen / t / 1e6, us_per_step=ev * 1e3, wall_us_per_step=wall * 1e3,
               alg_bytes=nbytes, alg_flops=flops, hbm_GBs=nbytes / t / 1e9, tflops=flops / t / 1e12,
               roofline_frac=t_roof / t)
    del plans
    torch.cuda.empty_cache()
    return res


def bench_kda_bwd(cfg, steps, warmup):
    import mamformer_amd as mh
    from mamformer_amd import workloads as W

    inp = W.kda_inputs(cfg, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(cfg.seed + 7)
    dout = (torch.randn(inp["v"].shape, device="cuda", generator=g) / cfg.dv ** 0.5).to(inp["v"].dtype)
    lam = mh.diff_lambda(torch.linspace(-2.0, 3.0, cfg.nheads, device="cuda"))

    def step():
        mh.linear_attn_scan_bwd(inp["q1"], inp["q2"], inp["k"], inp["v"], kernel_dim=cfg.dk, lam=lam, do1=dout,
                                need_initial=False)

    wall, ev = time_plans([step], steps, warmup)
    nbytes, flops = kda_bwd_alg(cfg)
    t = ev * 1e-3
    res = dict(mtok_s=cfg.batch * cfg.seqlen / t / 1e6, us_per_step=ev * 1e3, wall_us_per_step=wall * 1e3,
               alg_bytes=nbytes, alg_flops=flops, hbm_GBs=nbytes / t / 1e9, tflops=flops / t / 1e12,
               roofline_frac=max(nbytes / PEAK_HBM, flops / PEAK_BF16) / t)
    del inp, dout
    torch.cuda.empty_cache()
    return res


def bench_conv1d(steps, warmup):
    """Causal conv1d + SiLU (the Mamba layer prologue) at the ssd2 layer shape: x (2, 4096, d_inner 4096) bf16, width 4.
    Forward: x read, y written; backward: x and dy read, dx written (dweight / dbias and the per-run partials are
    small).  Launched through fixed-buffer plans, timed with HIP events."""
    import ctypes as ct
    from mamformer_amd import _lib, ops
    b, L, D, K = 2, 4096, 4096, 4
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(b, L, D, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(b, L, D, device="cuda", generator=g).to(torch.bfloat16)
    w = (0.5 * torch.randn(D, K, device="cuda", generator=g)).contiguous()
    bias = torch.randn(D, device="cuda", generator=g)
    y = torch.empty_like(x)
    a = ops._conv_args(x, w, bias, None, True)
    a.y, a.y_stride_b, a.y_stride_l = ops._ptr(y), y.stride(0), y.stride(1)
    fwd = ops.Plan("mh_causal_conv1d_fwd", a, x.device, keep=(x, w, bias, y))
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    db = torch.empty_like(bias)
    q = _lib.Conv1dBwdArgs()
    q.fwd = ops._conv_args(x, w, bias, None, True)
    q.dy, q.dy_stride_b, q.dy_stride_l = ops._ptr(dy), dy.stride(0), dy.stride(1)
    q.dx, q.dx_stride_b, q.dx_stride_l = ops._ptr(dx), dx.stride(0), dx.stride(1)
    q.dweight, q.dbias = ops._ptr(dw), ops._ptr(db)
    n = ct.c_size_t()
    _lib.call("mh_conv1d_bwd_workspace_bytes", ct.byref(q), ct.byref(n))
    ws = torch.empty(n.value, device="cuda", dtype=torch.uint8)
    q.workspace, q.workspace_bytes = ws.data_ptr(), n.value
    bwd = ops.Plan("mh_causal_conv1d_bwd", q, x.device, keep=(x, w, bias, dy, dx, dw, db, ws))
    xb = b * L * D * 2
    res = {}
    for name, plan, nbytes in (("fwd", fwd, 2 * xb), ("bwd", bwd, 3 * xb)):
        _, ev = time_plans([plan], steps, warmup)
        t = ev * 1e-3
        res[name] = dict(us_per_step=ev * 1e3, alg_bytes=nbytes, hbm_GBs=nbytes / t / 1e9,
                         roofline_frac=nbytes / PEAK_HBM / t)
    return res


def bench_kda_ref(cfg, steps, warmup):
    """Reference-mode KDA scan (phi = elu + 1, normaliser, fused differential output) at the kda5 shape:
    q1, q2, k, v read and the output written (bf16)."""
    import mamformer_amd as mh
    from mamformer_amd import workloads as W
    inp = W.kda_inputs(cfg, device="cuda")
    lam = mh.diff_lambda(torch.linspace(-2.0, 3.0, cfg.nheads, device="cuda"))
    plan = mh.plan_linear_attn_scan(inp["q1"], inp["q2"], inp["k"], inp["v"], mode="reference", kernel_dim=cfg.dk,
                                    lam=lam)
    _, ev = time_plans([plan], steps, warmup)
    nbytes = cfg.batch * cfg.nheads * cfg.seqlen * (4 * cfg.dk * 2 + cfg.dv * 2)
    t = ev * 1e-3
    res = dict(mtok_s=cfg.batch * cfg.seqlen / t / 1e6, us_per_step=ev * 1e3, alg_bytes=nbytes,
               hbm_GBs=nbytes / t / 1e9, roofline_frac=nbytes / PEAK_HBM / t)
    del plan, inp
    torch.cuda.empty_cache()
    return res


def bench_kda_step(steps, warmup, batch=64, nheads=32, dk=128, dv=128):
    """KDA decode: one reference-mode recurrent step (phi applied in the kernel) for `batch` sequences of `nheads`
    heads: the fp32 state and normaliser read and written in place, q1, q2, k, v, o per head."""
    import mamformer_amd as mh
    g = torch.Generator(device="cuda").manual_seed(5)
    state = 0.1 * torch.randn(batch, nheads, dk, dv, device="cuda", generator=g)
    z = torch.rand(batch, nheads, dk, device="cuda", generator=g) + 1.0
    mk = lambda d: (torch.randn(batch, nheads, d, device="cuda", generator=g) / d ** 0.5).to(torch.bfloat16)
    q1, q2, k, v = mk(dk), mk(dk), mk(dk), mk(dv)
    plan = mh.plan_linear_attn_step(state, z, q1, q2, k, v, lam=0.8, kernel_dim=dk)
    _, ev = time_plans([plan], steps, warmup)
    nbytes = batch * nheads * (2 * dk * dv * 4 + 2 * dk * 4 + 3 * dk * 2 + 2 * dv * 2)
    t = ev * 1e-3
    return dict(us_per_step=ev * 1e3, alg_bytes=nbytes, hbm_GBs=nbytes / t / 1e9, roofline_frac=nbytes / PEAK_HBM / t)


def bench_decode(cfg, steps, warmup, nsets):
    import mamformer_amd as mh
    from mamformer_amd import workloads as W

    plans = []
    for i in range(nsets):
        inp = W.decode_inputs(cfg.scaled(seed=cfg.seed + 1000 * i), device="cuda")
        plans.append(mh.plan_selective_state_update(inp["state"], inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                                                    inp["D"], dt_bias=inp["dt_bias"], dt_softplus=True))
    wall, ev = time_plans(plans, steps, warmup)
    nbytes = decode_alg(cfg)
    t = ev * 1e-3
    res = dict(us_per_step=ev * 1e3, alg_bytes=nbytes, hbm_GBs=nbytes / t / 1e9, roofline_frac=nbytes / PEAK_HBM / t,
               wall_us_per_step=wall * 1e3)
    del plans
    torch.cuda.empty_cache()
    return res


PEAK_EXP = 256 * 4 * 4 * 2.4e9   # exponentials/s: the transcendental unit at a quarter of the 16-lane VALU rate
PEAK_VALU = 256 * 4 * 16 * 2.4e9  # fp32 lane operations/s without packed math (16-lane SIMDs, 4 per CU)


def bench_ref_scan(steps, warmup, batch=2, seqlen=4096, d_inner=2048, dstate=128):
    """The reference-parameterised prefill (``selective_scan_reference``: A per state, dt and D per channel,
    mamba2.py:70-130) at the reference's 1b preset width (d_inner 2048, N 128; config.py:833-843), bf16, with and
    without h_states.  Bound by one exponential per (token, channel, state): ``exp_roofline_us`` is that count at
    the transcendental rate, ``valu_roofline_us`` adds the four fp32 operations per element (decay argument,
    B dt x, the state update and the C read-out) at the VALU rate, sharing the same issue slots.  ``us_train`` is a
    forward + backward through autograd (the backward recomputes the states from checkpoints twice, so it costs
    about three forward passes of exponentials)."""
    import mamformer_amd as mh

    g = torch.Generator(device="cuda").manual_seed(21)
    plans, plans_hs = [], []
    for _ in range(3):
        x = torch.randn(batch, seqlen, d_inner, device="cuda", generator=g).to(torch.bfloat16)
        dt = torch.nn.functional.softplus(torch.randn(batch, seqlen, d_inner, device="cuda", generator=g) - 2.0)
        A_log = torch.log(torch.linspace(0.5, 8.0, dstate, device="cuda"))
        B = torch.randn(batch, seqlen, dstate, device="cuda", generator=g).to(torch.bfloat16)
        C = torch.randn(batch, seqlen, dstate, device="cuda", generator=g).to(torch.bfloat16)
        D = torch.ones(d_inner, device="cuda")
        plans.append(mh.plan_selective_scan_reference(x, dt, A_log, B, C, D, return_final_state=True))
        plans_hs.append(mh.plan_selective_scan_reference(x, dt, A_log, B, C, D, True, True))
    _, ev = time_plans(plans, steps, warmup)
    _, ev_hs = time_plans(plans_hs, steps, warmup)
    # training: forward + backward of <gy, y> through autograd (mh_ssd_ref_scan_fwd, then mh_ssd_ref_scan_bwd:
    # a checkpointing forward pass and two recomputing gradient kernels)
    leaves = [x.clone().requires_grad_(), dt.clone().requires_grad_(), A_log.clone().requires_grad_(),
              B.clone().requires_grad_(), C.clone().requires_grad_(), D.clone().requires_grad_()]
    gy = torch.randn_like(x)

    def train():
        y = mh.selective_scan_reference(*leaves)
        torch.autograd.grad(y, leaves, gy)

    _, ev_tr = time_plans([train], max(3, steps // 10), 1)
    elems = batch * seqlen * d_inner * dstate
    t_exp = elems / PEAK_EXP
    t_valu = elems * (4 + 4) / PEAK_VALU
    nbytes = batch * seqlen * (d_inner * (2 + 4 + 2) + 2 * dstate * 2) + batch * d_inner * dstate * 4
    t = ev * 1e-3
    res = dict(us_per_step=ev * 1e3, us_with_h_states=ev_hs * 1e3, us_train=ev_tr * 1e3,
               mtok_s=batch * seqlen / t / 1e6,
               exp_roofline_us=t_exp * 1e6, valu_roofline_us=t_valu * 1e6, exp_frac=t_exp / t, valu_frac=t_valu / t,
               alg_bytes=nbytes, hbm_frac=nbytes / PEAK_HBM / t,
               shape=f"b{batch} L{seqlen} d_inner{d_inner} N{dstate} bf16")
    del plans, plans_hs, leaves
    torch.cuda.empty_cache()
    return res


def bench_kda(cfg, steps, warmup):
    import mamformer_amd as mh
    from mamformer_amd import workloads as W

    inp = W.kda_inputs(cfg, device="cuda")
    plan = mh.plan_linear_attn_scan(inp["q1"], inp["q2"], inp["k"], inp["v"], g=inp["g"], lam=inp["lam"],
                                    return_final_state=True)
    wall, ev = time_plans([plan], steps, warmup)
    nbytes, flops = kda_alg(cfg)
    t = ev * 1e-3
    res = dict(mtok_s=cfg.batch * cfg.seqlen / t / 1e6, us_per_step=ev * 1e3, alg_bytes=nbytes, alg_flops=flops,
               hbm_GBs=nbytes / t / 1e9, roofline_frac=max(nbytes / PEAK_HBM, flops / PEAK_BF16) / t)
    del plan, inp
    torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------------- CPU baseline (reference algorithm on the host)

def _cpu_info():
    """CPU model, logical CPU counts and the thread count the CPU legs use: the smallest of os.cpu_count(), the
    process's affinity set and OMP_NUM_THREADS (the host share a GPU box grants one GPU)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(nproc, affinity, int(omp) if omp and omp.isdigit() and int(omp) > 0 else nproc)
    return dict(cpu_model=model, nproc=nproc, affinity=affinity, omp_num_threads=omp, threads=threads)


def _median_time(fn, runs):
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline(cfg, sample_len, kda_sample=512):
    """The reference's pure-PyTorch CPU path (oracle/baseline.py restates it at its cost structure) on the host:
    the ssd2 prefill (headline comparator), the c3 decode step at B = 64 and 256, and the reference-mode KDA
    operator at the kda5 shape on a leading slice of ``kda_sample`` tokens (fixed work per token)."""
    from mamformer_amd import workloads as W
    from oracle import baseline as BL

    info = _cpu_info()
    torch.set_num_threads(info["threads"])
    inp = W.ssd_inputs(cfg.scaled(seqlen=sample_len))
    x4, dt, A, B, C, D = (inp[k] for k in ("x", "dt", "A", "B", "C", "D"))
    BL.ssd_prefill_sample(x4[:, :16], dt[:, :16], A, B[:, :16], C[:, :16], D)      # warm-up
    t = _median_time(lambda: BL.ssd_prefill_sample(x4, dt, A, B, C, D), 3)
    del inp, x4, B, C
    res = dict(value=cfg.batch * sample_len / t / 1e6, unit="Mtok/s", cores=info["threads"], kind="port",
               sample=(f"{cfg.name} full width (b{cfg.batch} d_inner {cfg.nheads * cfg.headdim} N{cfg.dstate}), "
                       f"first {sample_len} of {cfg.seqlen} tokens, fp32, median of 3 runs ({t:.2f} s each); "
                       f"torch {torch.__version__} threads={torch.get_num_threads()}"),
               cpu_model=info["cpu_model"], nproc=info["nproc"], affinity=info["affinity"],
               omp_num_threads=info["omp_num_threads"], torch_threads=torch.get_num_threads())
    extra = {}
    # c3 decode: one _recurrent_step (mamba2.py:431-458) at d_inner = H*P, fp32 state (b, d_inner, N)
    for bsz in (64, 256):
        c = W.DEC3.scaled(batch=bsz)
        d_inner, N = c.nheads * c.headdim, c.dstate
        g = torch.Generator().manual_seed(c.seed)
        h = 0.1 * torch.randn(bsz, d_inner, N, generator=g)
        x_t, dt_t = torch.randn(bsz, d_inner, generator=g), torch.rand(bsz, d_inner, generator=g) * 0.1
        B_t, C_t = torch.randn(bsz, N, generator=g), torch.randn(bsz, N, generator=g)
        A_log, Dv = torch.zeros(N), torch.ones(d_inner)
        BL.recurrent_step_cpu(x_t, dt_t, B_t, C_t, h, A_log, Dv)
        td = _median_time(lambda: BL.recurrent_step_cpu(x_t, dt_t, B_t, C_t, h, A_log, Dv), 5)
        nbytes = decode_alg(c)
        extra[f"decode_B{bsz}"] = dict(us_per_step=round(td * 1e6, 1), GBs=round(nbytes / td / 1e9, 2),
                                       sample=f"dec3 B={bsz} one step, fp32, median of 5")
        del h
    # c5: LinearDiffAttention._linear_attention_scan (kda_diff.py:357-478) at the kda5 shape, leading slice
    c = W.KDA5.scaled(seqlen=kda_sample)
    q = W.kda_inputs(c)
    lr = torch.full((c.nheads,), 1.386)                 # sigmoid(1.386) = 0.8, the workload's lambda
    BL.linear_attention_scan_cpu(q["q1"][:, :, :64], q["q2"][:, :, :64], q["k"][:, :, :64], q["v"][:, :, :64],
                                 c.dk, lr)
    tk = _median_time(lambda: BL.linear_attention_scan_cpu(q["q1"], q["q2"], q["k"], q["v"], c.dk, lr), 3)
    extra["kda5"] = dict(mtok_s=c.batch * kda_sample / tk / 1e6, s_per_run=round(tk, 2),
                         sample=(f"kda5 full width (B{c.batch} H{c.nheads} D{c.dk}), first {kda_sample} of "
                                 f"{W.KDA5.seqlen} tokens, the reference's ungated normalised operator, bf16, "
                                 f"median of 3"))
    res["other"] = extra
    return res


# ----------------------------------------------------------------- HBM traffic calibration

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def copy_calibration(nbytes, reps=5):
    """A plain device copy of `nbytes` (read nbytes + write nbytes), run `reps` times.

    Run under ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` next to the scan
    kernels, its counters give the KiB-per-byte scale used to turn the scan
    kernels' counter readings into HBM bytes.
    """
    n = nbytes // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: {reps} x {nbytes} bytes")


def measured_traffic(workload="ssd2"):
    """HBM bytes per launch of a workload's op from the committed PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t.get(workload)
    except (OSError, ValueError):
        return None


# ----------------------------------------------------------------- main

LEGS = ("ssd2", "decode", "ssd4", "kda5", "ssd2_bwd", "kda5_bwd", "conv1d", "kda5_ref", "kda_step", "ssd1", "ref1b",
        "ssd2_hstates", "cpu")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only (no decode / ssd4 / kda5 / cpu legs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None,
                    help=f"comma-separated legs to run, of {','.join(LEGS)} (profiling); the JSON line then carries "
                         "only those")
    ap.add_argument("--cpu-sample", type=int, default=4096,
                    help="tokens per sequence of the CPU baseline sample (ssd2 has 4096: the whole workload)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="first run a plain device copy of BYTES (HBM counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (--gpus {args.gpus} requested); the scan path has no "
              "multi-GPU mode here (each GPU would take its own share of heads or batch).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.only:
        legs = set(args.only.split(","))
        bad = legs - set(LEGS)
        if bad:
            ap.error(f"unknown legs {sorted(bad)}")
    elif args.quick:
        legs = {"ssd2"}
    else:
        legs = set(LEGS) - ({"cpu"} if args.no_cpu else set())

    from mamformer_amd import workloads as W

    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
    cfg = W.SSD2
    out = {
        "metric": METRIC,
        "value": None,
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded recipes of mamformer_amd/workloads.py, drawn on the GPU)",
        "config": {"workload": "ssd2: 1b-shape SSD chunked-scan prefill, b2 L4096 nheads64 headdim64 dstate128 "
                               "ngroups1, bf16 x/B/C/y, fp32 dt/A/D and final state",
                   "batch": cfg.batch, "seqlen": cfg.seqlen, "nheads": cfg.nheads, "headdim": cfg.headdim,
                   "dstate": cfg.dstate, "ngroups": cfg.ngroups, "parallelism": "single GPU"},
    }
    if "ssd2" in legs:
        log(f"ssd2 headline: {args.steps} steps after {args.warmup} warmup, 3 rotating buffer sets")
        head, wall, ev = bench_ssd(cfg, args.steps, args.warmup, nsets=3)
        log(f"ssd2: {head['mtok_s']:.1f} Mtok/s, {head['us_per_step']:.1f} us/step, "
            f"roofline {head['roofline_frac']:.3f}")
        out["value"] = round(head["mtok_s"], 3)
        out["ms_per_step"] = round(wall, 5)
        out["config"]["chunk_len"] = head["chunk_len"]
        out["config"]["chunk_len_note"] = (
            "state-passing chunk of the kernels, chosen by mh_ssd_chunk_len: 512 gives one 8-wave workgroup per CU "
            "(2 x 8 chunks x 16 head blocks = 256); chunk 256 doubles the chunk-state traffic and the look-back "
            "length and measured slower. The workload's chunk 256 is the chunk of the reference's Triton kernels; "
            "the outputs do not depend on the chunk length")
        tr = measured_traffic()
        out["roofline"] = {
            "bound": "hbm", "achieved": round(head["hbm_GBs"], 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(head["hbm_GBs"] / (PEAK_HBM / 1e9), 4),
            "traffic": None if tr is None else tr["bytes_per_launch"],
            "kernel": "mh_ssd_chunk_scan_fwd (ssd_lb_state_kernel + ssd_lb_scan_kernel)",
            "alg_bytes_per_launch": head["alg_bytes"], "alg_flops_per_launch": head["alg_flops"],
            "launch_us": round(head["us_per_step"], 2),
            # algorithmic FLOPs / time / dense bf16 peak (not a counter; the MFMA-busy counters of the two kernels
            # are in profiles/sq_counters_ssd2_prefill.md)
            "alg_flop_frac": round(head["alg_flops"] / (head["us_per_step"] * 1e-6) / PEAK_BF16, 4),
        }
        if tr is not None:
            out["roofline"]["traffic_source"] = tr.get("source")
    if "decode" in legs:
        dec = {}
        for b in (64, 256):
            c = W.DEC3.scaled(batch=b)
            r = bench_decode(c, max(args.steps, 50), args.warmup, nsets=3 if b == 64 else 2)
            log(f"decode B={b}: {r['hbm_GBs']:.0f} GB/s ({r['roofline_frac']:.3f} of 8 TB/s), {r['us_per_step']:.1f} us")
            dec[f"dec3_b{b}"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        out["decode"] = dec
    other = {}
    if "ssd2" in legs:
        r, _, _ = bench_ssd(cfg, args.steps, args.warmup, nsets=3, gated=True)
        log(f"ssd2 gated (y * silu(z) fused): {r['mtok_s']:.1f} Mtok/s, {r['us_per_step']:.1f} us, "
            f"roofline {r['roofline_frac']:.3f}")
        other["ssd2_gated"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "ssd4" in legs:
        r, _, _ = bench_ssd(W.SSD4, max(5, args.steps // 10), 3, nsets=1)
        log(f"ssd4: {r['mtok_s']:.1f} Mtok/s, {r['us_per_step']:.0f} us, roofline {r['roofline_frac']:.3f}")
        other["ssd4"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "kda5" in legs:
        r = bench_kda(W.KDA5, max(5, args.steps // 5), 3)
        log(f"kda5: {r['mtok_s']:.1f} Mtok/s, {r['us_per_step']:.0f} us, roofline {r['roofline_frac']:.3f}")
        other["kda5"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "ssd2_bwd" in legs:
        r = bench_ssd_bwd(cfg, max(10, args.steps // 2), 5, nsets=3)
        log(f"ssd2 backward: {r['us_per_step']:.1f} us, {r['tflops']:.0f} TFLOP/s, roofline {r['roofline_frac']:.3f}")
        other["ssd2_bwd"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "kda5_bwd" in legs:
        r = bench_kda_bwd(W.KDA5, max(5, args.steps // 10), 2)
        log(f"kda5 backward (reference mode, differential output): {r['us_per_step']:.0f} us, "
            f"{r['tflops']:.0f} TFLOP/s, roofline {r['roofline_frac']:.3f}")
        other["kda5_bwd"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "conv1d" in legs:
        r = bench_conv1d(args.steps, args.warmup)
        log(f"conv1d+SiLU (b2 L4096 D4096 K4 bf16): forward {r['fwd']['us_per_step']:.1f} us "
            f"({r['fwd']['roofline_frac']:.3f} of 8 TB/s), backward {r['bwd']['us_per_step']:.1f} us "
            f"({r['bwd']['roofline_frac']:.3f})")
        other["conv1d"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                           for k, v in r.items()}
    if "kda5_ref" in legs:
        r = bench_kda_ref(W.KDA5, max(5, args.steps // 5), 3)
        log(f"kda5 reference mode (differential output): {r['us_per_step']:.0f} us, roofline {r['roofline_frac']:.3f}")
        other["kda5_ref"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "kda_step" in legs:
        r = bench_kda_step(args.steps, args.warmup)
        log(f"KDA decode step B=64 H=32: {r['us_per_step']:.1f} us, {r['hbm_GBs']:.0f} GB/s "
            f"({r['roofline_frac']:.3f} of 8 TB/s)")
        other["kda_step"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "ssd2_hstates" in legs:
        r = bench_ssd_hstates(cfg, max(10, args.steps // 5), 3)
        log(f"ssd2 return_h_states: {r['us_with_h_states']:.1f} us with h_states vs {r['us_plain']:.1f} us without "
            f"(h_states alone {r['us_h_states']:.1f} us, x{r['overhead']:.2f}); forward + backward "
            f"{r['us_train_with_h_states']:.0f} us with vs {r['us_train_plain']:.0f} us without")
        other["ssd2_hstates"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "ref1b" in legs:
        r = bench_ref_scan(max(5, args.steps // 10), 3)
        log(f"reference-form prefill ({r['shape']}): {r['us_per_step']:.0f} us ({r['us_with_h_states']:.0f} us with "
            f"h_states), exp roofline {r['exp_roofline_us']:.0f} us -> {r['exp_frac']:.3f}, VALU {r['valu_frac']:.3f}")
        other["ref1b"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    if "ssd1" in legs:
        r, _, _ = bench_ssd(W.SSD1, args.steps, args.warmup, nsets=1, chunk=64)
        other["ssd1"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
    # measured HBM bytes per launch (PMC, copy-calibrated) next to each leg's algorithmic bytes
    for key, entry in [(k, v) for k, v in other.items() if k not in ("conv1d", "ssd1")] + \
            [(f"conv1d_{k}", v) for k, v in other.get("conv1d", {}).items()] + \
            [(k, v) for k, v in out.get("decode", {}).items()]:
        tr = measured_traffic(key)
        if tr is not None:
            entry["traffic"] = tr["bytes_per_launch"]
    if other:
        out["other"] = other
    if "cpu" in legs:
        log(f"cpu baseline: reference prefill on {args.cpu_sample} tokens of ssd2")
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_sample)
        cb = out["cpu_baseline"]
        log(f"cpu ({cb['cpu_model']}, {cb['cores']} threads of nproc {cb['nproc']}): ssd2 {cb['value']:.4f} Mtok/s; "
            f"decode B=64 {cb['other']['decode_B64']['GBs']} GB/s, B=256 {cb['other']['decode_B256']['GBs']} GB/s; "
            f"kda5 {cb['other']['kda5']['mtok_s']:.4f} Mtok/s")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
