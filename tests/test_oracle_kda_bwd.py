"""Pins of the KDA backward oracle (oracle/kda_bwd.py) on the CPU.

The oracle is an adjoint recurrence; it is checked against torch autograd of a different formulation of
the same forward -- the attention-matrix form o_i = (W_i V + phi(q_i) S0) / (rowsum W_i + phi(q_i) z0 + 1e-8),
W_i = causal(phi(q_i) phi(k)^T), with torch's own elu -- in float64, including kernel_dim < head_dim, an
initial state and normaliser, and the differential combination with lam = clamp(sigmoid(lambda_raw), 0.99)
on both sides of the clamp.  Planted mistakes (the normaliser's gradient dropped, an exclusive state) move
the gradients far outside the tolerance.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kda as okda
from oracle import kda_bwd as obwd


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return np.linalg.norm(a - b) / den if den > 0 else np.linalg.norm(a)


def matrix_form(q, k, v, K, S0=None, z0=None, exclusive=False, detach_norm=False):
    """o = (causal(phi(q) phi(k)^T) v + phi(q) S0) / (row sums + phi(q) z0 + 1e-8), torch float64."""
    pq = F.elu(q[..., :K]) + 1.0
    pk = F.elu(k[..., :K]) + 1.0
    S = q.shape[2]
    mask = torch.ones(S, S, dtype=torch.bool).tril(-1 if exclusive else 0)
    W = (pq @ pk.transpose(-1, -2)).masked_fill(~mask, 0.0)
    num = W @ v
    den = W.sum(-1)
    if S0 is not None:
        num = num + pq @ S0
        den = den + (pq * z0[:, :, None, :]).sum(-1)
    den = den + 1e-8
    if detach_norm:
        den = den.detach()
    return num / den[..., None]


def make(rng, B=2, H=3, S=11, Dk=8, D=6, scale=1.0):
    t = lambda *s: rng.standard_normal(s) * scale
    return t(B, H, S, Dk), t(B, H, S, Dk), t(B, H, S, Dk), t(B, H, S, D)


@pytest.mark.parametrize("K,init", [(8, False), (5, True), (8, True)])
def test_pair_backward_matches_autograd_of_matrix_form(K, init):
    rng = np.random.default_rng(3 + K)
    q1, q2, k, v = make(rng)
    B, H, S, Dk = q1.shape
    D = v.shape[-1]
    do1, do2 = rng.standard_normal((B, H, S, D)), rng.standard_normal((B, H, S, D))
    S0 = rng.standard_normal((B, H, K, D)) * 0.5 if init else None
    z0 = rng.uniform(0.5, 2.0, (B, H, K)) if init else None
    r = obwd.ref_scan_pair_backward(q1, q2, k, v, K, do1, do2, initial_state=S0, initial_z=z0)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tq1, tq2, tk, tv = map(T, (q1, q2, k, v))
    tS0, tz0 = (T(S0), T(z0)) if init else (None, None)
    o1 = matrix_form(tq1, tk, tv, K, tS0, tz0)
    o2 = matrix_form(tq2, tk, tv, K, tS0, tz0)
    ((o1 * torch.tensor(do1)).sum() + (o2 * torch.tensor(do2)).sum()).backward()
    assert rel_l2(r["o1"], o1.detach().numpy()) < 1e-12
    for name, t in (("dq1", tq1), ("dq2", tq2), ("dk", tk), ("dv", tv)):
        assert rel_l2(r[name], t.grad.numpy()) < 1e-10, name
    assert np.all(r["dq1"][..., K:] == 0) and np.all(r["dk"][..., K:] == 0)
    if init:
        assert rel_l2(r["dS0"], tS0.grad.numpy()) < 1e-10
        assert rel_l2(r["dz0"], tz0.grad.numpy()) < 1e-10


def test_final_state_gradients_match_autograd():
    rng = np.random.default_rng(41)
    q1, q2, k, v = make(rng, S=8)
    B, H, S, Dk = q1.shape
    D = v.shape[-1]
    S0, z0 = rng.standard_normal((B, H, Dk, D)) * 0.5, rng.uniform(0.5, 2.0, (B, H, Dk))
    dF, dFz = rng.standard_normal((B, H, Dk, D)), rng.standard_normal((B, H, Dk))
    do1 = rng.standard_normal((B, H, S, D))
    r = obwd.ref_scan_pair_backward(q1, q2, k, v, Dk, do1, None, initial_state=S0, initial_z=z0,
                                    d_final_state=dF, d_final_z=dFz)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tq1, tq2, tk, tv, tS0, tz0 = map(T, (q1, q2, k, v, S0, z0))
    o1 = matrix_form(tq1, tk, tv, Dk, tS0, tz0)
    pk = F.elu(tk) + 1.0
    SL = tS0 + pk.transpose(-1, -2) @ tv
    zL = tz0 + pk.sum(2)
    ((o1 * torch.tensor(do1)).sum() + (SL * torch.tensor(dF)).sum() + (zL * torch.tensor(dFz)).sum()).backward()
    for name, t in (("dq1", tq1), ("dk", tk), ("dv", tv), ("dS0", tS0), ("dz0", tz0)):
        assert rel_l2(r[name], t.grad.numpy()) < 1e-10, name
    assert np.all(r["dq2"] == 0)


def test_single_query_backward_matches_autograd():
    rng = np.random.default_rng(9)
    q1, _, k, v = make(rng, S=7)
    do1 = rng.standard_normal(v.shape)
    r = obwd.ref_scan_pair_backward(q1, None, k, v, 8, do1)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tq, tk, tv = map(T, (q1, k, v))
    (matrix_form(tq, tk, tv, 8) * torch.tensor(do1)).sum().backward()
    assert "dq2" not in r
    for name, t in (("dq1", tq), ("dk", tk), ("dv", tv)):
        assert rel_l2(r[name], t.grad.numpy()) < 1e-10, name


def test_diff_backward_matches_autograd_including_lambda_clamp():
    rng = np.random.default_rng(17)
    q1, q2, k, v = make(rng, H=4, S=9)
    lr = np.array([-1.0, 0.3, 2.0, 5.5])            # sigmoid(5.5) = 0.9959 > 0.99: clamped, no gradient
    dout = rng.standard_normal(v.shape)
    r = obwd.ref_attention_scan_backward(q1, q2, k, v, 8, lr, dout)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tq1, tq2, tk, tv, tl = map(T, (q1, q2, k, v, lr))
    lam = torch.clamp(torch.sigmoid(tl), max=0.99).view(1, -1, 1, 1)
    out = (matrix_form(tq1, tk, tv, 8) - lam * matrix_form(tq2, tk, tv, 8)) / (1.0 - lam + 1e-8)
    assert rel_l2(okda.ref_attention_scan(q1, q2, k, v, 8, lr), out.detach().numpy()) < 1e-12
    (out * torch.tensor(dout)).sum().backward()
    for name, t in (("dq1", tq1), ("dq2", tq2), ("dk", tk), ("dv", tv), ("d_lambda_raw", tl)):
        assert rel_l2(r[name], t.grad.numpy()) < 1e-10, name
    assert r["d_lambda_raw"][3] == 0.0 and abs(r["d_lambda_raw"][0]) > 0


def test_central_differences():
    rng = np.random.default_rng(23)
    q1, q2, k, v = make(rng, B=1, H=1, S=6, Dk=4, D=3)
    do1, do2 = rng.standard_normal(v.shape), rng.standard_normal(v.shape)
    r = obwd.ref_scan_pair_backward(q1, q2, k, v, 4, do1, do2)

    def loss(q1_, q2_, k_, v_):
        o1, o2, _, _ = okda.ref_scan_pair(q1_, q2_, k_, v_, 4)
        return (o1 * do1).sum() + (o2 * do2).sum()

    eps = 1e-6
    for name, idx in (("dq1", (0, 0, 3, 1)), ("dq2", (0, 0, 5, 2)), ("dk", (0, 0, 0, 3)), ("dk", (0, 0, 4, 0)),
                      ("dv", (0, 0, 1, 2))):
        args = [q1.copy(), q2.copy(), k.copy(), v.copy()]
        j = {"dq1": 0, "dq2": 1, "dk": 2, "dv": 3}[name]
        args[j][idx] += eps
        up = loss(*args)
        args[j][idx] -= 2 * eps
        dn = loss(*args)
        assert abs((up - dn) / (2 * eps) - r[name][idx]) < 1e-6 * max(1.0, abs(r[name][idx])), (name, idx)


@pytest.mark.parametrize("mistake", ["detach_norm", "exclusive"])
def test_planted_mistakes_are_caught(mistake):
    """Gradients of a plausible wrong forward (normaliser treated as constant; state exclusive of the current
    token) are far from the oracle's, so the pins above have the power to see such mistakes."""
    rng = np.random.default_rng(31)
    q1, _, k, v = make(rng, S=10)
    do1 = rng.standard_normal(v.shape)
    do1[:, :, 0] = 0.0                                   # token 0 has no exclusive history
    r = obwd.ref_scan_pair_backward(q1, None, k, v, 8, do1)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tq, tk, tv = map(T, (q1, k, v))
    kw = {"detach_norm": True} if mistake == "detach_norm" else {"exclusive": True}
    (matrix_form(tq, tk, tv, 8, **kw) * torch.tensor(do1)).sum().backward()
    assert max(rel_l2(r["dq1"], tq.grad.numpy()), rel_l2(r["dk"], tk.grad.numpy())) > 1e-2
