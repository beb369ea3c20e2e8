"""GPU parity of the reference-mode KDA backward (mh_kda_chunk_scan_bwd) against the float64 oracle
(oracle/kda_bwd.py, the adjoint recurrence pinned against autograd of the attention-matrix form).

Tolerance: relative L2 <= 1e-2 on every gradient (bf16 I/O; the kernels run bf16 MFMA operands with
fp32 accumulation), per head where the differential output scales the heads by 1 / (1 - lambda).  Cases: the pair outputs (triton_linear_attn_scan's contract), the fused differential
output with the lambda gradient through sigmoid and the 0.99 clamp (LinearDiffAttention._linear_attention_scan),
a single query stream, kernel_dim below head_dim, an initial state and normaliser with their gradients,
final-state gradients, ragged last chunks (S = 1, 70, 130, 200), S = 0, and S = 600 / 700 where the reverse
walk is split into segments that run side by side.  A longer sequence (S = 2048) is
checked through a leading slice: with the output gradient zero after T0 every gradient past T0 is exactly zero
and the earlier ones equal the truncated problem's.  No float atomics: two calls agree bit for bit.
"""

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from oracle import kda as okda
from oracle import kda_bwd as obwd
from tests.gpu_helpers import check_lambda_bound, check_per_head, check, dev, host, lambda_term_scale, say

pytestmark = pytest.mark.gpu
TOL = 1e-2


def inputs(seed, B, H, S, D=128, scale=4.0):
    g = torch.Generator().manual_seed(seed)
    mk = lambda s: (torch.randn(B, H, S, D, generator=g) * s / D ** 0.5).to(torch.bfloat16)
    return [mk(scale) for _ in range(3)] + [mk(1.0)] + [mk(1.0), mk(1.0)]


@pytest.mark.parametrize("B,H,S,kd,init,dfin", [
    (1, 2, 64, 128, False, False), (2, 2, 130, 128, True, True), (1, 1, 1, 128, False, False),
    (1, 3, 200, 100, True, False), (2, 1, 70, 37, False, True),
    (1, 2, 600, 128, True, True),      # 10 chunks: the reverse walk runs as two segments side by side
])
def test_pair_backward_vs_oracle(B, H, S, kd, init, dfin):
    q1, q2, k, v, do1, do2 = inputs(S + 7 * H + kd, B, H, S)
    g = torch.Generator().manual_seed(99)
    s0 = (torch.randn(B, H, 128, 128, generator=g) * 0.1) if init else None
    z0 = (torch.rand(B, H, 128, generator=g) * 2 + 0.5) if init else None
    dF = (torch.randn(B, H, 128, 128, generator=g) * 0.1) if dfin else None
    dFz = (torch.randn(B, H, 128, generator=g) * 0.1) if dfin else None
    say(f"kda bwd pair B={B} H={H} S={S} kd={kd} init={init} dfin={dfin}")
    r = mh.linear_attn_scan_bwd(dev(q1, torch.bfloat16), dev(q2, torch.bfloat16), dev(k, torch.bfloat16),
                                dev(v, torch.bfloat16), kernel_dim=kd, do1=dev(do1, torch.bfloat16),
                                do2=dev(do2, torch.bfloat16), pair=True, initial_state=dev(s0), initial_z=dev(z0),
                                d_final_state=dev(dF), d_final_z=dev(dFz))
    torch.cuda.synchronize()
    f64 = lambda t: None if t is None else t.double().numpy()
    ref = obwd.ref_scan_pair_backward(f64(q1), f64(q2), f64(k), f64(v), kd, f64(do1), f64(do2),
                                      initial_state=None if s0 is None else f64(s0)[:, :, :kd],
                                      initial_z=None if z0 is None else f64(z0)[:, :, :kd],
                                      d_final_state=None if dF is None else f64(dF)[:, :, :kd],
                                      d_final_z=None if dFz is None else f64(dFz)[:, :, :kd])
    if S == 1 and not init:
        # one token, zero state: o = v exactly, so dq and dk vanish (the oracle's are rounding noise)
        for name in ("dq1", "dq2", "dk"):
            assert r[name].abs().max().item() <= 1e-3 * r["dv"].abs().max().item(), name
        check("dv", r["dv"], ref["dv"], TOL)
    else:
        for name in ("dq1", "dq2", "dk", "dv"):
            check(name, r[name], ref[name], TOL)
    check("d_initial_state", r["d_initial_state"][:, :, :kd], ref["dS0"], TOL)
    check("d_initial_z", r["d_initial_z"][:, :, :kd], ref["dz0"], TOL)
    assert torch.all(r["dq1"][..., kd:] == 0) and torch.all(r["dk"][..., kd:] == 0)


@pytest.mark.parametrize("S", [96, 257, 700])
def test_diff_output_autograd_vs_oracle(S):
    B, H = 2, 4
    q1, q2, k, v, dout, _ = inputs(S, B, H, S)
    lr = torch.tensor([-1.0, 0.4, 2.5, 5.5])       # sigmoid(5.5) > 0.99: clamped, zero gradient
    say(f"kda bwd diff autograd S={S}")
    tq1, tq2, tk, tv = (dev(t, torch.bfloat16).requires_grad_() for t in (q1, q2, k, v))
    tl = dev(lr).requires_grad_()
    out = mh.linear_attention_scan(tq1, tq2, tk, tv, 128, tl)
    out.backward(dev(dout, torch.bfloat16))
    torch.cuda.synchronize()
    f64 = lambda t: t.double().numpy()
    ref = obwd.ref_attention_scan_backward(f64(q1), f64(q2), f64(k), f64(v), 128, lr.double().numpy(), f64(dout))
    # per head: the gradients scale by 1 / (1 - lam), up to 100x on the clamped head
    for name, t in (("dq1", tq1), ("dq2", tq2), ("dk", tk), ("dv", tv)):
        check_per_head(name, t.grad, ref[name], TOL)
    # d lam_h = c^2 sum dout . (o1 - o2): with random dout the sum cancels down to about 1/sqrt(B S D) of its
    # terms, and o1 - o2 (o1 ~ o2 in reference mode) carries the bf16-operand rounding of the recomputed
    # outputs, so one head's value is not a meaningful 1e-2 target.  Checked three ways: the vector over heads
    # to 1e-2; every head within 4e-3 (about the bf16 unit roundoff) of the summed magnitude of its terms; and
    # every head to 1e-2 with a coherent dout (test_diff_lambda_gradient_per_head)
    check("d_lambda_raw", tl.grad, ref["d_lambda_raw"], TOL)
    scale = lambda_term_scale(dout.double().numpy(), ref["o1"], ref["o2"], lr.double().numpy())
    check_lambda_bound("d_lambda_raw", tl.grad, ref["d_lambda_raw"], scale, 4e-3)
    assert tl.grad[3].item() == 0.0


def test_diff_lambda_gradient_per_head():
    """The lambda gradient of every head, with dout along o1 - o2 (from the oracle's forward), so each head's
    sum c^2 sum dout . (o1 - o2) is coherent rather than a cancelling random sum; a wrong term or sign in the
    lambda chain moves it by O(1)."""
    B, H, S = 2, 4, 160
    q1, q2, k, v, _, _ = inputs(23, B, H, S)
    lr = torch.tensor([-1.0, 0.4, 2.5, 3.5])
    f64 = lambda t: t.double().numpy()
    o1, o2, _, _ = okda.ref_scan_pair(f64(q1), f64(q2), f64(k), f64(v), 128)
    dout = torch.tensor(o1 - o2).to(torch.bfloat16)
    say("kda bwd lambda gradient per head (coherent dout)")
    tq1, tq2, tk, tv = (dev(t, torch.bfloat16).requires_grad_() for t in (q1, q2, k, v))
    tl = dev(lr).requires_grad_()
    out = mh.linear_attention_scan(tq1, tq2, tk, tv, 128, tl)
    out.backward(dev(dout, torch.bfloat16))
    torch.cuda.synchronize()
    ref = obwd.ref_attention_scan_backward(f64(q1), f64(q2), f64(k), f64(v), 128, lr.double().numpy(), f64(dout))
    check_per_head("d_lambda_raw", tl.grad, ref["d_lambda_raw"], TOL, axis=0)


def test_single_query_autograd_vs_oracle():
    B, H, S = 1, 2, 150
    q1, _, k, v, do1, _ = inputs(5, B, H, S)
    say("kda bwd single query")
    tq, tk, tv = (dev(t, torch.bfloat16).requires_grad_() for t in (q1, k, v))
    o = mh.linear_attn_scan_single(tq, tk, tv, 128)
    o.backward(dev(do1, torch.bfloat16))
    torch.cuda.synchronize()
    f64 = lambda t: t.double().numpy()
    ref = obwd.ref_scan_pair_backward(f64(q1), None, f64(k), f64(v), 128, f64(do1))
    for name, t in (("dq1", tq), ("dk", tk), ("dv", tv)):
        check(name, t.grad, ref[name], TOL)


def test_empty_sequence_passes_final_state_gradient():
    B, H = 2, 3
    z = torch.zeros(B, H, 0, 128, dtype=torch.bfloat16, device="cuda")
    dF = torch.randn(B, H, 128, 128, device="cuda")
    dFz = torch.randn(B, H, 128, device="cuda")
    say("kda bwd S=0")
    r = mh.linear_attn_scan_bwd(z, z, z, z, kernel_dim=128, do1=z, pair=True, d_final_state=dF, d_final_z=dFz)
    torch.cuda.synchronize()
    assert torch.equal(r["d_initial_state"], dF) and torch.equal(r["d_initial_z"], dFz)
    assert r["dq1"].shape == (B, H, 0, 128)


def test_leading_slice_of_long_sequence_and_determinism():
    B, H, S, T0 = 1, 4, 2048, 320
    q1, q2, k, v, do1, do2 = inputs(11, B, H, S)
    do1[:, :, T0:] = 0
    do2[:, :, T0:] = 0
    args = [dev(t, torch.bfloat16) for t in (q1, q2, k, v)]
    say(f"kda bwd leading slice S={S} T0={T0}")
    r1 = mh.linear_attn_scan_bwd(*args, kernel_dim=128, do1=dev(do1, torch.bfloat16), do2=dev(do2, torch.bfloat16),
                                 pair=True)
    r2 = mh.linear_attn_scan_bwd(*args, kernel_dim=128, do1=dev(do1, torch.bfloat16), do2=dev(do2, torch.bfloat16),
                                 pair=True)
    short = mh.linear_attn_scan_bwd(*(a[:, :, :T0].contiguous() for a in args), kernel_dim=128,
                                    do1=dev(do1[:, :, :T0], torch.bfloat16), do2=dev(do2[:, :, :T0], torch.bfloat16),
                                    pair=True)
    torch.cuda.synchronize()
    for name in ("dq1", "dq2", "dk", "dv", "d_initial_state", "d_initial_z"):
        assert torch.equal(r1[name], r2[name]), name
    for name in ("dq1", "dq2", "dk", "dv"):
        assert torch.all(r1[name][:, :, T0:] == 0), name
        check(name + " slice", r1[name][:, :, :T0], host(short[name]), 2e-3)
    f64 = lambda t: t.double().numpy()
    ref = obwd.ref_scan_pair_backward(f64(q1[:, :, :T0]), f64(q2[:, :, :T0]), f64(k[:, :, :T0]), f64(v[:, :, :T0]),
                                      128, f64(do1[:, :, :T0]), f64(do2[:, :, :T0]))
    for name in ("dq1", "dq2", "dk", "dv"):
        check(name + " oracle", r1[name][:, :, :T0], ref[name], TOL)
