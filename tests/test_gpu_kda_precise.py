"""GPU parity of the fp32-arithmetic KDA kernels (kda_precise.hip) against the float64 oracle: fp32 I/O at
every supported head size, and bf16 I/O at head sizes other than dk = dv = 128 (the reference's 300m and debug
presets use head_dim 64, mamformer/config.py:836-838, so kernel_dim = min(kernel_dim, head_dim) = 64,
kda_diff.py:154).

Tolerance: global relative L2 <= 1e-4 for fp32 I/O and <= 1e-2 for bf16 I/O (bf16 inputs are rounded before
the oracle sees them), on outputs, final states and every gradient.  Cases: the gated operator (oracle
``gated_recurrent``) with and without q2, g and an initial state, decays steep enough to cut the factorisation
windows; the reference scan (``ref_scan_pair``) as a pair, fused differential output with per-head lambda and
single query, kernel_dim below the head size, initial state and normaliser; its backward
(``oracle.kda_bwd``) as a pair with initial / final-state gradients and through autograd of the differential
output including the lambda gradient; ragged chunk ends (S = 1, 33, 65, 70, 130).
"""

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from oracle import kda as okda
from oracle import kda_bwd as obwd
from tests.gpu_helpers import (TOL, check, check_lambda_bound, check_per_head, dev, host, lambda_term_scale,
                               say)

pytestmark = pytest.mark.gpu
F32, BF = torch.float32, torch.bfloat16


def rnd(g, shape, dtype, scale=1.0):
    """Random values exactly representable in `dtype` (float64 copy for the oracle, device copy for the kernels)."""
    t = (torch.randn(*shape, generator=g) * scale).to(dtype)
    return t.double().numpy(), dev(t, dtype)


def ids(v):
    return str(v).replace("torch.", "")


@pytest.mark.parametrize("dtype,dk,dv,S,two_q,gate,init", [
    (F32, 128, 128, 100, True, True, True),
    (F32, 64, 64, 33, True, True, False),
    (F32, 64, 128, 65, False, True, True),
    (F32, 128, 64, 1, True, False, False),
    (BF, 64, 64, 130, True, True, True),
    (BF, 128, 64, 70, True, True, False),
], ids=ids)
def test_gated_vs_recurrence(dtype, dk, dv, S, two_q, gate, init):
    B, H = 2, 3
    g = torch.Generator().manual_seed(S + dk + dv)
    q1, tq1 = rnd(g, (B, H, S, dk), dtype, dk ** -0.5)
    q2, tq2 = rnd(g, (B, H, S, dk), dtype, dk ** -0.5) if two_q else (np.zeros_like(q1), None)
    k, tk = rnd(g, (B, H, S, dk), dtype, dk ** -0.5)
    v, tv = rnd(g, (B, H, S, dv), dtype)
    gl = torch.nn.functional.logsigmoid(torch.randn(B, H, S, dk, generator=g)) / 16 if gate else None
    s0 = torch.randn(B, H, dk, dv, generator=g) * 0.1 if init else None
    say(f"precise gated {dtype} dk={dk} dv={dv} S={S} q2={two_q} g={gate} s0={init}")
    o, fin = mh.linear_attn_scan(tq1, tq2, tk, tv, g=dev(gl), lam=0.8, initial_state=dev(s0),
                                 return_final_state=True)
    torch.cuda.synchronize()
    ro, rf = okda.gated_recurrent(q1, q2, k, v, None if gl is None else gl.double().numpy(), 0.8,
                                  None if s0 is None else s0.double().numpy())
    assert o.dtype == dtype and o.shape == (B, H, S, dv) and fin.shape == (B, H, dk, dv)
    check("o", o, ro, TOL[dtype])
    check("final", fin, rf, TOL[dtype])


def test_gated_steep_decay_cuts_windows_fp32():
    """log-decays down to -40 per token: a 32-token chunk spans far more than the factorisation range, so the
    chunk is cut into windows; the outputs still match the recurrence to fp32 accuracy."""
    B, H, S, D = 1, 2, 70, 64
    g = torch.Generator().manual_seed(5)
    q1, tq1 = rnd(g, (B, H, S, D), F32, 0.2)
    q2, tq2 = rnd(g, (B, H, S, D), F32, 0.2)
    k, tk = rnd(g, (B, H, S, D), F32, 0.2)
    v, tv = rnd(g, (B, H, S, D), F32)
    gl = -40.0 * torch.rand(B, H, S, D, generator=g) * (torch.rand(B, H, S, D, generator=g) < 0.2)
    say("precise gated steep decay fp32")
    o, fin = mh.linear_attn_scan(tq1, tq2, tk, tv, g=dev(gl), lam=0.5, return_final_state=True)
    torch.cuda.synchronize()
    ro, rf = okda.gated_recurrent(q1, q2, k, v, gl.double().numpy(), 0.5)
    check("o", o, ro, 1e-4)
    check("final", fin, rf, 1e-4)


@pytest.mark.parametrize("dtype,dk,dv,S,kd,state", [
    (F32, 128, 128, 97, 128, True),
    (F32, 64, 64, 64, 64, True),
    (F32, 64, 128, 33, 40, False),
    (F32, 128, 64, 1, 128, False),
    (BF, 64, 64, 130, 64, True),
    (BF, 64, 128, 65, 48, False),
], ids=ids)
def test_ref_pair_vs_oracle(dtype, dk, dv, S, kd, state):
    B, H = 2, 3
    g = torch.Generator().manual_seed(3 * S + kd)
    q1, tq1 = rnd(g, (B, H, S, dk), dtype)
    q2, tq2 = rnd(g, (B, H, S, dk), dtype)
    k, tk = rnd(g, (B, H, S, dk), dtype)
    v, tv = rnd(g, (B, H, S, dv), dtype)
    S0 = z0 = None
    if state:
        S0 = torch.rand(B, H, dk, dv, generator=g) * 2.0
        z0 = torch.rand(B, H, dk, generator=g) * 3.0
        S0[:, :, kd:] = 0
        z0[:, :, kd:] = 0
    say(f"precise ref pair {dtype} dk={dk} dv={dv} S={S} kd={kd} state={state}")
    o1, o2, fin, finz = mh.linear_attn_scan(tq1, tq2, tk, tv, mode="reference", kernel_dim=kd, pair=True,
                                            return_final_state=True, initial_state=dev(S0), initial_z=dev(z0))
    torch.cuda.synchronize()
    r1, r2, rs, rz = okda.ref_scan_pair(q1, q2, k, v, kd,
                                        initial_state=None if S0 is None else S0.double().numpy()[:, :, :kd],
                                        initial_z=None if z0 is None else z0.double().numpy()[:, :, :kd])
    tol = TOL[dtype]
    check("o1", o1, r1, tol)
    check("o2", o2, r2, tol)
    check("final S", host(fin)[:, :, :kd], rs, tol)
    check("final z", host(finz)[:, :, :kd], rz, tol)
    assert torch.count_nonzero(fin[:, :, kd:]) == 0 and torch.count_nonzero(finz[:, :, kd:]) == 0


@pytest.mark.parametrize("dtype,D", [(F32, 64), (F32, 128), (BF, 64)], ids=ids)
def test_ref_fused_diff_and_single_vs_oracle(dtype, D):
    """LinearDiffAttention._linear_attention_scan (differential output, lam per head from lambda_raw, the
    0.99 clamp) and the single-query scan."""
    B, H, S = 2, 4, 77
    g = torch.Generator().manual_seed(D)
    q1, tq1 = rnd(g, (B, H, S, D), dtype)
    q2, tq2 = rnd(g, (B, H, S, D), dtype)
    k, tk = rnd(g, (B, H, S, D), dtype)
    v, tv = rnd(g, (B, H, S, D), dtype)
    lr = torch.tensor([-1.0, 0.4, 2.0, 5.5])
    say(f"precise ref fused diff {dtype} D={D}")
    out = mh.linear_attention_scan(tq1, tq2, tk, tv, D, dev(lr))
    single = mh.linear_attn_scan_single(tq1, tk, tv, D)
    torch.cuda.synchronize()
    # per head: the differential output scales the heads by 1 / (1 - lambda), up to 100 at the clamp
    check_per_head("fused diff", out, okda.ref_attention_scan(q1, q2, k, v, D, lr.double().numpy()), TOL[dtype])
    r1, _, _, _ = okda.ref_scan_pair(q1, q1, k, v, D)
    check("single", single, r1, TOL[dtype])


@pytest.mark.parametrize("dtype,dk,dv,S,kd,init,dfin", [
    (F32, 128, 128, 70, 128, True, True),
    (F32, 64, 64, 100, 64, False, True),
    (F32, 64, 128, 33, 50, True, False),
    (F32, 64, 64, 1, 64, True, True),
    (BF, 64, 64, 130, 64, True, True),
], ids=ids)
def test_ref_pair_backward_vs_oracle(dtype, dk, dv, S, kd, init, dfin):
    B, H = 2, 2
    g = torch.Generator().manual_seed(S + dk + kd)
    q1, tq1 = rnd(g, (B, H, S, dk), dtype, 4.0 / dk ** 0.5)
    q2, tq2 = rnd(g, (B, H, S, dk), dtype, 4.0 / dk ** 0.5)
    k, tk = rnd(g, (B, H, S, dk), dtype, 4.0 / dk ** 0.5)
    v, tv = rnd(g, (B, H, S, dv), dtype)
    do1, tdo1 = rnd(g, (B, H, S, dv), dtype)
    do2, tdo2 = rnd(g, (B, H, S, dv), dtype)
    s0 = torch.randn(B, H, dk, dv, generator=g) * 0.1 if init else None
    z0 = torch.rand(B, H, dk, generator=g) * 2 + 0.5 if init else None
    dF = torch.randn(B, H, dk, dv, generator=g) * 0.1 if dfin else None
    dFz = torch.randn(B, H, dk, generator=g) * 0.1 if dfin else None
    say(f"precise ref bwd pair {dtype} dk={dk} dv={dv} S={S} kd={kd} init={init} dfin={dfin}")
    r = mh.linear_attn_scan_bwd(tq1, tq2, tk, tv, kernel_dim=kd, do1=tdo1, do2=tdo2, pair=True,
                                initial_state=dev(s0), initial_z=dev(z0), d_final_state=dev(dF), d_final_z=dev(dFz))
    torch.cuda.synchronize()
    f64 = lambda t: None if t is None else t.double().numpy()[:, :, :kd]
    ref = obwd.ref_scan_pair_backward(q1, q2, k, v, kd, do1, do2, initial_state=f64(s0), initial_z=f64(z0),
                                      d_final_state=f64(dF), d_final_z=f64(dFz))
    tol = TOL[dtype]
    names = ("dq1", "dq2", "dk", "dv") if S > 1 or init else ("dv",)
    for name in names:
        assert r[name].dtype == dtype
        check(name, r[name], ref[name], tol)
    check("d_initial_state", r["d_initial_state"][:, :, :kd], ref["dS0"], tol)
    check("d_initial_z", r["d_initial_z"][:, :, :kd], ref["dz0"], tol)
    assert torch.all(r["dq1"][..., kd:] == 0) and torch.all(r["dk"][..., kd:] == 0)


@pytest.mark.parametrize("dtype,D", [(F32, 64), (F32, 128), (BF, 64)], ids=ids)
def test_diff_output_autograd_vs_oracle(dtype, D):
    B, H, S = 2, 4, 97
    g = torch.Generator().manual_seed(7 * D)
    q1, tq1 = rnd(g, (B, H, S, D), dtype, 4.0 / D ** 0.5)
    q2, tq2 = rnd(g, (B, H, S, D), dtype, 4.0 / D ** 0.5)
    k, tk = rnd(g, (B, H, S, D), dtype, 4.0 / D ** 0.5)
    v, tv = rnd(g, (B, H, S, D), dtype)
    dout, tdout = rnd(g, (B, H, S, D), dtype)
    lr = torch.tensor([-1.0, 0.4, 2.5, 5.5])       # sigmoid(5.5) > 0.99: clamped, zero gradient
    say(f"precise diff autograd {dtype} D={D}")
    leaves = [t.clone().requires_grad_() for t in (tq1, tq2, tk, tv)]
    tl = dev(lr).requires_grad_()
    out = mh.linear_attention_scan(*leaves, D, tl)
    out.backward(tdout)
    torch.cuda.synchronize()
    ref = obwd.ref_attention_scan_backward(q1, q2, k, v, D, lr.double().numpy(), dout)
    for name, t in zip(("dq1", "dq2", "dk", "dv"), leaves):
        check_per_head(name, t.grad, ref[name], TOL[dtype])
    check("d_lambda_raw", tl.grad, ref["d_lambda_raw"], TOL[dtype])
    # every head against the summed magnitude of its (cancelling) terms; fp32 arithmetic throughout
    scale = lambda_term_scale(dout, ref["o1"], ref["o2"], lr.double().numpy())
    check_lambda_bound("d_lambda_raw", tl.grad, ref["d_lambda_raw"], scale, 1e-4 if dtype == F32 else 4e-3)
    assert tl.grad[3].item() == 0.0


@pytest.mark.parametrize("dtype,D,S", [(F32, 64, 160), (F32, 128, 160), (BF, 64, 160), (F32, 64, 2048),
                                       (BF, 64, 2048)], ids=ids)
def test_diff_lambda_gradient_per_head(dtype, D, S):
    """The lambda gradient of every head with dout along o1 - o2 (from the oracle's forward), so each head's sum
    c^2 sum dout . (o1 - o2) is coherent rather than a cancelling random sum: a wrong term or sign in the lambda
    chain moves it by O(1).  S = 2048 runs 64 chunks through the centred partial sums."""
    B, H = 2, 4
    g = torch.Generator().manual_seed(3 * D + S)
    q1, tq1 = rnd(g, (B, H, S, D), dtype, 4.0 / D ** 0.5)
    q2, tq2 = rnd(g, (B, H, S, D), dtype, 4.0 / D ** 0.5)
    k, tk = rnd(g, (B, H, S, D), dtype, 4.0 / D ** 0.5)
    v, tv = rnd(g, (B, H, S, D), dtype)
    lr = torch.tensor([-1.0, 0.4, 2.5, 3.5])
    o1, o2, _, _ = okda.ref_scan_pair(q1, q2, k, v, D)
    dout_t = torch.tensor(o1 - o2).to(dtype)
    dout = dout_t.double().numpy()
    say(f"precise lambda gradient per head (coherent dout) {dtype} D={D} S={S}")
    leaves = [t.clone().requires_grad_() for t in (tq1, tq2, tk, tv)]
    tl = dev(lr).requires_grad_()
    out = mh.linear_attention_scan(*leaves, D, tl)
    out.backward(dev(dout_t, dtype))
    torch.cuda.synchronize()
    ref = obwd.ref_attention_scan_backward(q1, q2, k, v, D, lr.double().numpy(), dout)
    check_per_head("d_lambda_raw", tl.grad, ref["d_lambda_raw"], TOL[dtype], axis=0)


def test_empty_sequence_head64():
    """S = 0 at dk = dv = 64: final state = initial, and the backward passes the final-state gradients through."""
    B, H, D = 1, 2, 64
    s0 = torch.randn(B, H, D, D, device="cuda")
    z0 = torch.rand(B, H, D, device="cuda")
    x = torch.zeros(B, H, 0, D, device="cuda")
    o1, o2, fin, finz = mh.linear_attn_scan(x, x, x, x, mode="reference", pair=True, return_final_state=True,
                                            initial_state=s0, initial_z=z0)
    assert o1.shape == (B, H, 0, D) and torch.equal(fin, s0) and torch.equal(finz, z0)
    dF = torch.randn(B, H, D, D, device="cuda")
    r = mh.linear_attn_scan_bwd(x, x, x, x, pair=True, do1=x, do2=x, d_final_state=dF)
    torch.cuda.synchronize()
    assert torch.equal(r["d_initial_state"], dF) and float(r["d_initial_z"].abs().max()) == 0.0


def test_layer_head64_prefill_and_cache_vs_oracle():
    """kda_linear_attention (LinearDiffAttention.forward's recurrent-state semantics, kda_diff.py:286-338) at the
    300m preset's head size 64 in bf16: the prefill output, and the cached S / z it hands to the next step."""
    from mamformer_amd.layers import kda_linear_attention
    B, H, S, D = 2, 4, 90, 64
    g = torch.Generator().manual_seed(64)
    q1, tq1 = rnd(g, (B, H, S, D), BF)
    q2, tq2 = rnd(g, (B, H, S, D), BF)
    k, tk = rnd(g, (B, H, S, D), BF)
    v, tv = rnd(g, (B, H, S, D), BF)
    lr = torch.tensor([-1.0, 0.4, 2.0, 0.0])
    say("kda layer head 64 prefill + cache")
    out, cache = kda_linear_attention(tq1, tq2, tk, tv, dev(lr), 64, use_cache=True)
    torch.cuda.synchronize()
    check("prefill", out, okda.ref_attention_scan(q1, q2, k, v, 64, lr.double().numpy()), 1e-2)
    _, _, rs, rz = okda.ref_scan_pair(q1, q2, k, v, 64)
    check("cache S", cache["S"], rs, 1e-2)
    check("cache z", cache["z"][..., 0], rz, 1e-2)
