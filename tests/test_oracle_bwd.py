"""Pins of the SSD backward oracle (oracle/ssd_bwd.py) -- CPU only.

Each check compares the adjoint recurrence with an independent construction of the same gradient:
torch autograd through the reference's own scan (``oracle.baseline.selective_scan_cpu``, the
restatement of mamba2.py:84-126) over the SSD bridge, torch autograd through an SSD-form recurrence
with an initial state and the dt prologue, central finite differences, and closed forms.  The
``test_planted_*`` tests plant mistakes in the oracle's output and check that the pins catch them.
"""

import numpy as np
import pytest
import torch

from oracle import ssd, ssd_bwd
from oracle.baseline import selective_scan_cpu
from tests.conftest import rel_l2

GRADS = ("dx", "ddt", "dA", "dB", "dC", "dD")


def case(rng, b=2, L=19, H=4, P=3, N=5, G=2, D_per_channel=False):
    x = rng.standard_normal((b, L, H, P))
    dt = rng.standard_normal((b, L, H)) - 1.0                 # raw: softplus in the prologue
    A = -np.exp(rng.uniform(0, np.log(4), H))
    B = rng.standard_normal((b, L, G, N))
    C = rng.standard_normal((b, L, G, N))
    D = rng.standard_normal((H, P)) if D_per_channel else rng.standard_normal(H)
    dy = rng.standard_normal((b, L, H, P))
    dfin = rng.standard_normal((b, H, P, N))
    return x, dt, A, B, C, D, dy, dfin


def autograd_reference(x, dt_p, A, B, C, D, dy, dfin):
    """Gradients by torch autograd through the reference scan, one call per group over the SSD bridge
    (A_log = 0, dt_ref = -A dt, x_ref = x / -A, D_ref = -A D); dt_p is the processed dt."""
    t = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    xs, dts, As, Bs, Cs, Ds = map(t, (x, dt_p, A, B, C, D))
    b, L, H, P = x.shape
    G = B.shape[2]
    hpg = H // G
    N = B.shape[-1]
    loss = 0.0
    for g in range(G):
        hs = slice(g * hpg, (g + 1) * hpg)
        a = -As[hs]
        dt_ref = (dts[:, :, hs] * a).unsqueeze(-1).expand(b, L, hpg, P).reshape(b, L, hpg * P)
        x_ref = (xs[:, :, hs] / a[None, None, :, None]).reshape(b, L, hpg * P)
        Dv = Ds[hs] if Ds.dim() == 1 else Ds[hs]
        D_ref = ((Dv * a).unsqueeze(-1).expand(hpg, P) if Dv.dim() == 1 else Dv * a[:, None]).reshape(hpg * P)
        y, hT = selective_scan_cpu(x_ref, dt_ref, torch.zeros(N, dtype=torch.float64), Bs[:, :, g], Cs[:, :, g], D_ref)
        loss = loss + (y.reshape(b, L, hpg, P) * torch.tensor(dy[:, :, hs])).sum()
        loss = loss + (hT.reshape(b, hpg, P, N) * torch.tensor(dfin[:, hs])).sum()
    loss.backward()
    return {"dx": xs.grad.numpy(), "ddt": dts.grad.numpy(), "dA": As.grad.numpy(), "dB": Bs.grad.numpy(),
            "dC": Cs.grad.numpy(), "dD": Ds.grad.numpy()}


def autograd_ssd_form(x, dt_raw, A, B, C, D, dy, dfin, h0, dt_bias, dt_limit):
    """Gradients by torch autograd through the SSD recurrence with h0 and the raw-dt prologue."""
    t = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    xs, dts, As, Bs, Cs, Ds, h0s, bs = map(t, (x, dt_raw, A, B, C, D, h0, dt_bias))
    b, L, H, P = x.shape
    G = B.shape[2]
    gidx = torch.arange(H) // (H // G)
    d = torch.nn.functional.softplus(dts + bs)
    d = torch.clamp(d, dt_limit[0], dt_limit[1])
    h = h0s
    loss = 0.0
    for i in range(L):
        a = torch.exp(As[None, :] * d[:, i])
        Bt, Ct = Bs[:, i][:, gidx], Cs[:, i][:, gidx]
        h = a[:, :, None, None] * h + (d[:, i, :, None, None] * xs[:, i, :, :, None]) * Bt[:, :, None, :]
        y = torch.einsum("bhpn,bhn->bhp", h, Ct) + Ds[None, :, None] * xs[:, i]
        loss = loss + (y * torch.tensor(dy[:, i])).sum()
    loss = loss + (h * torch.tensor(dfin)).sum()
    loss.backward()
    return {"dx": xs.grad.numpy(), "ddt": dts.grad.numpy(), "dA": As.grad.numpy(), "dB": Bs.grad.numpy(),
            "dC": Cs.grad.numpy(), "dD": Ds.grad.numpy(), "dh0": h0s.grad.numpy(), "ddt_bias": bs.grad.numpy()}


@pytest.mark.parametrize("G,dpc,ck", [(1, False, 64), (2, True, 5), (4, False, 7)])
def test_backward_matches_autograd_of_reference_scan(rng, G, dpc, ck):
    x, dt, A, B, C, D, dy, dfin = case(rng, G=G, D_per_channel=dpc)
    dtp = ssd.process_dt(dt, dt_softplus=True)
    ref = autograd_reference(x, dtp, A, B, C, D, dy, dfin)
    got = ssd_bwd.ssd_backward(x, dtp, A, B, C, D, dy, d_final=dfin, checkpoint=ck)
    for k in GRADS:
        assert rel_l2(got[k], ref[k]) < 1e-12, k


def test_backward_matches_autograd_with_h0_and_dt_prologue(rng):
    x, dt, A, B, C, D, dy, dfin = case(rng, L=23, G=2)
    h0 = 0.5 * rng.standard_normal(dfin.shape)
    bias = 0.3 * rng.standard_normal(A.shape)
    lim = (0.12, 0.6)                                          # some dt land on each side of the clamp
    ref = autograd_ssd_form(x, dt, A, B, C, D, dy, dfin, h0, bias, lim)
    got = ssd_bwd.ssd_backward(x, dt, A, B, C, D, dy, d_final=dfin, initial_state=h0, dt_bias=bias,
                               dt_softplus=True, dt_limit=lim, checkpoint=8)
    dtp = ssd.process_dt(dt, bias, True, lim)
    assert np.any(dtp == lim[0]) and np.any(dtp == lim[1]) and np.any((dtp > lim[0]) & (dtp < lim[1]))
    for k in GRADS + ("dh0", "ddt_bias"):
        assert rel_l2(got[k], ref[k]) < 1e-12, k


def test_backward_matches_finite_differences(rng):
    x, dt, A, B, C, D, dy, dfin = case(rng, b=1, L=6, H=2, P=2, N=3, G=1)
    h0 = 0.5 * rng.standard_normal(dfin.shape)
    bias = 0.2 * rng.standard_normal(A.shape)

    def loss(x_, dt_, A_, B_, C_, D_, h0_, bias_):
        dtp = ssd.process_dt(dt_, bias_, True)
        y, hT = ssd.ssd_direct(x_, dtp, A_, B_, C_, D_, initial_state=h0_)
        return float((y * dy).sum() + (hT * dfin).sum())

    args = [x, dt, A, B, C, D, h0, bias]
    got = ssd_bwd.ssd_backward(x, dt, A, B, C, D, dy, d_final=dfin, initial_state=h0, dt_bias=bias, dt_softplus=True)
    names = ["dx", "ddt", "dA", "dB", "dC", "dD", "dh0", "ddt_bias"]
    eps = 1e-6
    for i, name in enumerate(names):
        fd = np.zeros_like(args[i])
        for idx in np.ndindex(args[i].shape):
            hi = [a.copy() for a in args]
            lo = [a.copy() for a in args]
            hi[i][idx] += eps
            lo[i][idx] -= eps
            fd[idx] = (loss(*hi) - loss(*lo)) / (2 * eps)
        assert rel_l2(got[name], fd) < 1e-7, name


def test_backward_closed_forms(rng):
    """dy = 0: only the final-state gradient flows, dh0 = exp(A sum dt) d_final and dC = 0;
    d_final = 0, L = 1, h0 = 0: dx = dt (C.B) dy + D dy, dB = dt (x.dy) C, dD = x.dy."""
    x, dt, A, B, C, D, dy, dfin = case(rng, L=9, G=1)
    dtp = ssd.process_dt(dt, dt_softplus=True)
    r = ssd_bwd.ssd_backward(x, dtp, A, B, C, D, np.zeros_like(dy), d_final=dfin)
    decay = np.exp(A[None, :] * dtp.sum(axis=1))
    assert rel_l2(r["dh0"], decay[:, :, None, None] * dfin) < 1e-13
    assert np.abs(r["dC"]).max() == 0.0
    r = ssd_bwd.ssd_backward(x[:, :1], dtp[:, :1], A, B[:, :1], C[:, :1], D, dy[:, :1])
    cb = np.einsum("bgn,bgn->bg", B[:, 0], C[:, 0])[:, 0]
    xdy = np.einsum("bhp,bhp->bh", x[:, 0], dy[:, 0])
    assert rel_l2(r["dx"][:, 0], (dtp[:, 0] * cb[:, None])[..., None] * dy[:, 0] + D[None, :, None] * dy[:, 0]) < 1e-13
    assert rel_l2(r["dB"][:, 0, 0], np.einsum("bh,bn->bn", dtp[:, 0] * xdy, C[:, 0, 0])) < 1e-13
    assert rel_l2(r["dD"], xdy.sum(axis=0)) < 1e-13


@pytest.mark.parametrize("plant", ["drop_dA_term", "sign_dx", "transpose_dC_head", "exclusive_adjoint"])
def test_planted_mistakes_are_caught(rng, plant):
    x, dt, A, B, C, D, dy, dfin = case(rng, G=2)
    dtp = ssd.process_dt(dt, dt_softplus=True)
    ref = autograd_reference(x, dtp, A, B, C, D, dy, dfin)
    got = ssd_bwd.ssd_backward(x, dtp, A, B, C, D, dy, d_final=dfin)
    if plant == "drop_dA_term":
        got["dA"] = np.zeros_like(got["dA"])
    elif plant == "sign_dx":
        got["dx"] = got["dx"] - 2 * D[None, None, :, None] * dy
    elif plant == "transpose_dC_head":
        got["dC"] = got["dC"][:, :, ::-1]
    else:   # adjoint that omits the current token's own readout (dy_t C_t added after use)
        got = ssd_bwd.ssd_backward(x, dtp, A, B, C, D, dy, d_final=dfin)
        got["dx"] = got["dx"] - dtp[..., None] * np.einsum("blgn,blgn->blg", B, C).repeat(2, axis=2)[..., None] * dy
    assert max(rel_l2(got[k], ref[k]) for k in GRADS) > 1e-3


@pytest.mark.parametrize("silu,K,S", [(True, 4, 0), (False, 3, 2), (True, 2, 1), (True, 1, 0)])
def test_conv1d_backward_matches_autograd(rng, silu, K, S):
    """Against torch autograd of F.conv1d (depthwise, left padding K-1, cached rows prepended) + SiLU, float64."""
    b, L, D = 2, 9, 5
    x = rng.standard_normal((b, L, D))
    w = rng.standard_normal((D, K))
    bias = rng.standard_normal(D)
    dy = rng.standard_normal((b, L, D))
    cs = rng.standard_normal((b, S, D)) if S else None
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    bt = torch.tensor(bias, requires_grad=True)
    cst = torch.tensor(cs, requires_grad=True) if S else None
    xin = xt if cs is None else torch.cat([cst, xt], dim=1)
    u = torch.nn.functional.conv1d(torch.nn.functional.pad(xin.transpose(1, 2), (K - 1, 0)), wt[:, None, :], bt,
                                   groups=D).transpose(1, 2)[:, -L:]
    y = torch.nn.functional.silu(u) if silu else u
    (y * torch.tensor(dy)).sum().backward()
    dx, dw, db, dcs = ssd_bwd.causal_conv1d_backward(x, w, bias, dy, conv_state=cs, silu=silu, with_state_grad=True)
    assert rel_l2(dx, xt.grad.numpy()) < 1e-12
    assert rel_l2(dw, wt.grad.numpy()) < 1e-12
    assert rel_l2(db, bt.grad.numpy()) < 1e-12
    assert dcs.shape == (b, S, D)
    if S:
        assert rel_l2(dcs, cst.grad.numpy()) < 1e-12


def test_conv1d_backward_planted_mistake_is_caught(rng):
    """A reversed kernel (convolution instead of the reference's cross-correlation) in the oracle's dx fails."""
    b, L, D, K = 1, 7, 3, 4
    x, w, bias, dy = rng.standard_normal((b, L, D)), rng.standard_normal((D, K)), rng.standard_normal(D), \
        rng.standard_normal((b, L, D))
    dx, _, _ = ssd_bwd.causal_conv1d_backward(x, w, bias, dy, silu=True)
    dx_flip, _, _ = ssd_bwd.causal_conv1d_backward(x, w[:, ::-1], bias, dy, silu=True)
    xt = torch.tensor(x, requires_grad=True)
    u = torch.nn.functional.conv1d(torch.nn.functional.pad(xt.transpose(1, 2), (K - 1, 0)),
                                   torch.tensor(w)[:, None, :], torch.tensor(bias), groups=D).transpose(1, 2)
    (torch.nn.functional.silu(u) * torch.tensor(dy)).sum().backward()
    assert rel_l2(dx, xt.grad.numpy()) < 1e-12 and rel_l2(dx_flip, xt.grad.numpy()) > 1e-2
