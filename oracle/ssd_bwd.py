"""Float64 oracle for the gradient of the Mamba-2 selective scan (SSD prefill backward).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference trains through ``selective_scan`` by PyTorch autograd of ``_selective_scan_impl``
(R/mamformer/layers/mamba2.py:70-130; exercised by R/tests/test_mamba2.py:56-71).  This module states
that gradient as the adjoint recurrence of the SSD-form scan (the same recurrence as ``oracle.ssd.ssd_direct``):

    forward   h_t = a_t h_{t-1} + dt_t x_t B_t^T,  a_t = exp(A dt_t),   y_t = h_t C_t + D x_t
    adjoint   lam_t = a_{t+1} lam_{t+1} + dy_t C_t^T,   lam_{L-1} = dy_{L-1} C_{L-1}^T + d_final
    grads     dx_t  = dt_t lam_t B_t + D dy_t
              dB_t  = dt_t lam_t^T x_t            (summed over the heads of B's group)
              dC_t  = h_t^T dy_t                  (summed over the heads of C's group)
              ddt_t = <lam_t, x_t B_t^T> + A a_t <lam_t, h_{t-1}>      (w.r.t. the processed dt)
              dA    = sum_t dt_t a_t <lam_t, h_{t-1}>
              dD    = sum_t dy_t . x_t  (per head, or per channel)
              dh0   = a_0 lam_0

and carries the raw-dt chain rule of ``process_dt``: softplus'(u) = sigmoid(u) below PyTorch's threshold
20 (identity above, as torch's softplus backward), clamp passing the gradient where lo <= dt <= hi (as
torch.clamp's backward).  Pinned in ``tests/test_oracle_bwd.py`` against torch autograd through
``oracle.baseline.selective_scan_cpu`` (the reference's own scan, restated) over the SSD bridge, against
autograd through an SSD-form recurrence with an initial state and the dt prologue, and against central
finite differences.
"""

from __future__ import annotations

import numpy as np

from .ssd import _expand_D, _groups_of, process_dt, softplus

__all__ = ["ssd_backward", "dt_chain", "causal_conv1d_backward"]


def dt_chain(dt_raw, dt_bias=None, dt_softplus=False, dt_limit=None):
    """d(processed dt) / d(raw dt) elementwise (float64), matching torch's softplus / clamp backward."""
    u = np.asarray(dt_raw, np.float64)
    if dt_bias is not None:
        u = u + np.asarray(dt_bias, np.float64)
    g = np.ones_like(u)
    v = u
    if dt_softplus:
        g = np.where(u > 20.0, 1.0, 1.0 / (1.0 + np.exp(-np.minimum(u, 20.0))))
        v = softplus(u)
    if dt_limit is not None:
        lo, hi = dt_limit
        g = g * ((v >= lo) & (v <= hi))
    return g


def ssd_backward(x, dt_raw, A, B, C, D, dy, d_final=None, initial_state=None, dt_bias=None, dt_softplus=False,
                 dt_limit=None, checkpoint=64):
    """Gradients of L = <dy, y> + <d_final, h_L> for the SSD scan y, h_L = scan(x, dt, A, B, C, D, h0).

    x (b,L,H,P); dt_raw (b,L,H) before bias/softplus/clamp; A (H,); B, C (b,L,N) or (b,L,G,N);
    D None, (H,) or (H,P); dy (b,L,H,P); d_final, initial_state (b,H,P,N) or None.
    Returns a dict of float64 arrays: dx, ddt (w.r.t. dt_raw), dA, dB, dC (shaped like B, C), dD (shaped like
    D, absent for D None), dh0 (b,H,P,N), ddt_bias (H,).  States are checkpointed every ``checkpoint``
    tokens and recomputed per span, so memory stays at O(L/checkpoint) states.
    """
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    A = np.asarray(A, np.float64)
    b, L, H, P = x.shape
    B_in = np.asarray(B)
    Bg, G = _groups_of(B, H)
    Cg, _ = _groups_of(C, H)
    N = Bg.shape[-1]
    gidx = np.arange(H) // (H // G)
    Dhp = _expand_D(D, H, P)
    dt = process_dt(dt_raw, dt_bias, dt_softplus, dt_limit)                 # (b,L,H)
    dA_t = np.exp(A[None, None, :] * dt)                                     # (b,L,H)

    h = np.zeros((b, H, P, N)) if initial_state is None else np.array(initial_state, np.float64)
    ckpt = {}
    for t in range(L):
        if t % checkpoint == 0:
            ckpt[t] = h.copy()
        Bt = Bg[:, t][:, gidx]
        h = dA_t[:, t, :, None, None] * h + (dt[:, t, :, None, None] * x[:, t, :, :, None]) * Bt[:, :, None, :]

    dx = np.zeros_like(x)
    ddt = np.zeros((b, L, H))
    dA = np.zeros(H)
    dBh = np.zeros((b, L, H, N))
    dCh = np.zeros((b, L, H, N))
    dDhp = np.zeros((H, P))
    lam = np.zeros((b, H, P, N)) if d_final is None else np.array(d_final, np.float64)
    for t0 in reversed(range(0, L, checkpoint)):
        t1 = min(t0 + checkpoint, L)
        hs = [ckpt[t0]]                                                      # hs[i] = state before token t0 + i
        for t in range(t0, t1):
            Bt = Bg[:, t][:, gidx]
            hs.append(dA_t[:, t, :, None, None] * hs[-1]
                      + (dt[:, t, :, None, None] * x[:, t, :, :, None]) * Bt[:, :, None, :])
        for t in reversed(range(t0, t1)):
            Bt = Bg[:, t][:, gidx]
            Ct = Cg[:, t][:, gidx]
            h_prev, h_t = hs[t - t0], hs[t - t0 + 1]
            lam = lam + dy[:, t, :, :, None] * Ct[:, :, None, :]            # full adjoint of h_t
            lB = np.einsum("bhpn,bhn->bhp", lam, Bt)
            dx[:, t] = dt[:, t, :, None] * lB + Dhp[None] * dy[:, t]
            dBh[:, t] = dt[:, t, :, None] * np.einsum("bhpn,bhp->bhn", lam, x[:, t])
            dCh[:, t] = np.einsum("bhpn,bhp->bhn", h_t, dy[:, t])
            lh = np.einsum("bhpn,bhpn->bh", lam, h_prev)
            ddt[:, t] = np.einsum("bhp,bhp->bh", lB, x[:, t]) + A[None, :] * dA_t[:, t] * lh
            dA += np.einsum("bh,bh->h", dt[:, t] * dA_t[:, t], lh)
            dDhp += np.einsum("bhp,bhp->hp", dy[:, t], x[:, t])
            lam = dA_t[:, t, :, None, None] * lam                             # adjoint of h_{t-1}
    ddt_raw = ddt * dt_chain(dt_raw, dt_bias, dt_softplus, dt_limit)

    def group_sum(v):
        out = np.zeros((b, L, G, N))
        for gg in range(G):
            out[:, :, gg] = v[:, :, gidx == gg].sum(axis=2)
        return out.reshape(B_in.shape) if B_in.ndim == 3 else out

    res = {"dx": dx, "ddt": ddt_raw, "dA": dA, "dB": group_sum(dBh), "dC": group_sum(dCh), "dh0": lam,
           "ddt_bias": ddt_raw.sum(axis=(0, 1))}
    if D is not None:
        Dn = np.asarray(D)
        res["dD"] = dDhp.sum(axis=1) if Dn.shape == (H,) else dDhp.reshape(Dn.shape)
    return res


def causal_conv1d_backward(x, weight, bias, dy, conv_state=None, silu=False, with_state_grad=False):
    """Gradients of <dy, y> for y = act(conv(x)), the causal depthwise conv of ``oracle.ssd.ref_causal_conv1d``
    (R/mamformer/layers/mamba2.py:370-405) followed, when ``silu``, by the SiLU of mamba2.py:282-283.

    With xin = [conv_state; x] (S cached rows first), u[t] = bias + sum_j w[:, j] xin[S + t - (K-1) + j] and
    du = dy * act'(u) (act'(u) = s (1 + u (1 - s)), s = sigmoid(u), for the SiLU):
        dxin[i] = sum_j w[:, j] du[i - S + (K-1) - j]   (du = 0 outside 0..L-1),
        dw[:, j] = sum_{b,t} du[t] xin[S + t - (K-1) + j],   dbias = sum_{b,t} du[t].
    Returns dx = dxin[:, S:] (b, L, D), dweight (D, K), dbias (D,) in float64, and with ``with_state_grad``
    also d_conv_state = dxin[:, :S] (b, S, D).
    """
    from .ssd import ref_causal_conv1d

    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    b, L, D = x.shape
    w = np.asarray(weight, np.float64).reshape(D, -1)
    K = w.shape[1]
    u = ref_causal_conv1d(x, w, bias, conv_state)
    if silu:
        sg = 1.0 / (1.0 + np.exp(-u))
        du = dy * sg * (1.0 + u * (1.0 - sg))
    else:
        du = dy
    S = 0 if conv_state is None else np.asarray(conv_state).shape[1]
    xin = x if conv_state is None else np.concatenate([np.asarray(conv_state, np.float64), x], axis=1)
    pad = np.concatenate([np.zeros((b, K - 1, D)), xin], axis=1)          # pad[:, i] = xin[i - (K-1)]
    dxin = np.zeros((b, S + L, D))
    dw = np.zeros((D, K))
    for j in range(K):
        # y_t uses pad[S + t + j] = xin[S + t + j - (K-1)]  (t = 0..L-1)
        dw[:, j] = np.einsum("btd,btd->d", du, pad[:, S + j:S + j + L])
        for t in range(L):
            i = S + t + j - (K - 1)
            if i >= 0:
                dxin[:, i] += w[None, :, j] * du[:, t]
    res = (dxin[:, S:], dw, du.sum(axis=(0, 1)))
    return res + (dxin[:, :S],) if with_state_grad else res
