"""Float64 oracle for the Mamba-2 selective scan, its decode step and the SSD convention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference algorithm (``R`` = ``/root/reference/mamformer 671b/``):

* ``ref_selective_scan``  restates ``_selective_scan_impl``  R/mamformer/layers/mamba2.py:70-130
* ``ref_recurrent_step``  restates ``Mamba2Block._recurrent_step`` R/mamformer/layers/mamba2.py:407-458
* ``softplus``            restates ``F.softplus`` (beta=1, threshold=20) as used at mamba2.py:293/304
* ``ref_causal_conv1d``   restates ``Mamba2Block._causal_conv1d`` R/mamformer/layers/mamba2.py:370-405

SSD (Mamba-2) convention -- nheads H, headdim P, scalar A_h < 0 per head, dt per
head, ngroups G sharing B/C -- is reduced to the reference formula by the exact
"bridge" (per head h with a_h = -A_h > 0):

    A_log := 0 (A_par = exp(clamp(0)) = 1),  dt_ref[c] = a_h * dt_h,
    x_ref[c] = x[c] / a_h,                  D_ref[c] = a_h * D_h,      c = h*P + p

so that exp(-A_par*dt_ref) = exp(A_h*dt_h), B*dt_ref*x_ref = B*dt_h*x and
D_ref*x_ref = D_h*x.  ngroups > 1 is one reference call per group; an initial
state is handled by stepping the reference decode recurrence from ``h0``
(mamba2.py:447-450 seeds the recurrence with ``h_prev``).

``ssd_direct`` (a second, independent statement in SSD form) and
``ssd_semiseparable`` (explicit L x L matrix, tiny sizes) pin the bridge.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "softplus",
    "ref_selective_scan",
    "ref_recurrent_step",
    "ref_causal_conv1d",
    "ssd_h_states",
    "process_dt",
    "ssd_via_reference",
    "ssd_direct",
    "ssd_chunked",
    "ssd_semiseparable",
    "state_update_via_reference",
    "state_update_direct",
]


def softplus(x):
    """F.softplus(x, beta=1, threshold=20): x where x > 20, else log1p(exp(x))."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


# ---------------------------------------------------------------------------
# Reference algorithm, restated
# ---------------------------------------------------------------------------

def ref_selective_scan(x, dt, A_log, B, C, D, return_h_states=False, return_final_state=False):
    """Restates ``_selective_scan_impl`` (R/mamformer/layers/mamba2.py:70-130) in float64.

    x, dt (b, L, d_inner); A_log (N,); B, C (b, L, N); D (d_inner,).
    * A_par = exp(clamp(A_log, -5, 5))                          (mamba2.py:87-88)
    * A_disc[b,t,c,n] = exp(-A_par[n] * dt[b,t,c])              (:90)
    * h = A_disc[:,t] * h + B[:,t,None,:] * dt[:,t,:,None] * x  (:94-97, :111)
    * y[:,t] = sum_n C[:,t,n] * h[:,:,n]                         (:113)
    * h_states[:,t] = mean over d_inner of h                     (:115-116)
    * y += D * x                                                 (:119)
    Returns y, or a tuple in the order (y, h_states, final_h)    (:121-130).
    The (b,L,d_inner,N) tensors of the reference are streamed one timestep at
    a time here; the arithmetic per element is unchanged.
    """
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A_log = np.asarray(A_log, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    D = np.asarray(D, np.float64)
    b, L, d_inner = x.shape
    N = A_log.shape[0]
    A_par = np.exp(np.clip(A_log, -5.0, 5.0))
    h = np.zeros((b, d_inner, N))
    y = np.zeros((b, L, d_inner))
    hs = np.zeros((b, L, N)) if return_h_states else None
    for t in range(L):
        dtt = dt[:, t, :, None]                       # (b, d_inner, 1)
        a_disc = np.exp(-A_par[None, None, :] * dtt)  # (b, d_inner, N)
        h = a_disc * h + (B[:, t, None, :] * dtt) * x[:, t, :, None]
        y[:, t] = np.sum(C[:, t, None, :] * h, axis=-1)
        if return_h_states:
            hs[:, t] = h.mean(axis=1)
    y = y + D[None, None, :] * x
    out = [y]
    if return_h_states:
        out.append(hs)
    if return_final_state:
        out.append(h)
    return out[0] if len(out) == 1 else tuple(out)


def ref_recurrent_step(x, dt, B, C, h_prev, A_log, D):
    """Restates ``Mamba2Block._recurrent_step`` (R/mamformer/layers/mamba2.py:407-458).

    Only the last token is used (:435-438).  No clamp on A_log (:441-443).
    h_prev None -> zeros (:448-449).  Returns (y_t (b,1,d_inner), h_t (b,d_inner,N)).
    """
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    A_log = np.asarray(A_log, np.float64)
    D = np.asarray(D, np.float64)
    b, _, d_inner = x.shape
    N = A_log.shape[0]
    x_t, dt_t, B_t, C_t = x[:, -1], dt[:, -1], B[:, -1], C[:, -1]
    a_disc = np.exp(-np.exp(A_log)[None, None, :] * dt_t[:, :, None])
    b_disc = B_t[:, None, :] * dt_t[:, :, None]
    if h_prev is None:
        h_prev = np.zeros((b, d_inner, N))
    h_t = a_disc * np.asarray(h_prev, np.float64) + b_disc * x_t[:, :, None]
    y_t = np.sum(C_t[:, None, :] * h_t, axis=-1) + D[None, :] * x_t
    return y_t[:, None, :], h_t


def ref_causal_conv1d(x, weight, bias=None, conv_state=None):
    """Restates ``Mamba2Block._causal_conv1d`` (R/mamformer/layers/mamba2.py:370-405) in float64.

    x (b, L, D); weight (D, 1, K) or (D, K) (depthwise ``nn.Conv1d``); bias (D,) or None; conv_state
    (b, S_c, D) cached raw inputs or None.  With a cache the input is cat(conv_state, x) (:388-390); the
    sequence is left-padded with K-1 zeros (:393), cross-correlated with the per-channel kernel
    (``F.conv1d``, :397) and, with a cache, only the last L outputs are kept (:401-402).
    """
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64).reshape(x.shape[2], -1)
    K = w.shape[1]
    L = x.shape[1]
    xin = x if conv_state is None else np.concatenate([np.asarray(conv_state, np.float64), x], axis=1)
    pad = np.concatenate([np.zeros((x.shape[0], K - 1, x.shape[2])), xin], axis=1)
    n_out = xin.shape[1]
    out = np.zeros((x.shape[0], n_out, x.shape[2]))
    for j in range(K):
        out += w[None, None, :, j] * pad[:, j:j + n_out, :]
    if bias is not None:
        out += np.asarray(bias, np.float64)[None, None, :]
    return out[:, -L:] if L else out[:, :0]


# ---------------------------------------------------------------------------
# SSD convention helpers
# ---------------------------------------------------------------------------

def process_dt(dt, dt_bias=None, dt_softplus=False, dt_limit=None):
    """dt' = clamp(softplus?(dt + dt_bias), *dt_limit) per head (float64).

    The bias + softplus order follows mamba2.py:293 (softplus of the
    projection); the clamp is the Mamba-2 ``dt_limit`` option used by the
    CPU-plumbing workload (dt clamped to [1e-3, 0.1]).
    """
    d = np.asarray(dt, np.float64)
    if dt_bias is not None:
        d = d + np.asarray(dt_bias, np.float64)
    if dt_softplus:
        d = softplus(d)
    if dt_limit is not None:
        lo, hi = dt_limit
        d = np.clip(d, lo, hi)
    return d


def _groups_of(B, H):
    B = np.asarray(B, np.float64)
    if B.ndim == 3:
        B = B[:, :, None, :]
    G = B.shape[2]
    if H % G:
        raise ValueError(f"nheads {H} not divisible by ngroups {G}")
    return B, G


def _expand_D(D, H, P):
    if D is None:
        return np.zeros((H, P))
    D = np.asarray(D, np.float64)
    if D.shape == (H,):
        return np.repeat(D[:, None], P, axis=1)
    return D.reshape(H, P)


def ssd_via_reference(x, dt, A, B, C, D=None, initial_state=None, return_h_states=False):
    """SSD-convention scan computed *by the reference algorithm* through the bridge.

    x (b,L,H,P); dt (b,L,H) already processed (positive); A (H,) with A < 0;
    B, C (b,L,N) or (b,L,G,N); D None, (H,) or (H,P); initial_state (b,H,P,N) or None.
    Returns (y (b,L,H,P), final_state (b,H,P,N)), float64; with ``return_h_states`` (zero initial
    state) also h_states (b,L,N) = the reference's per-token mean of the state over all H*P channels
    (mamba2.py:114-116), combined over the per-group calls weighted by their channel counts.

    Zero initial state: one ``ref_selective_scan`` call per group (heads
    h with h // (H//G) == g share B[:,:,g], C[:,:,g]).  Nonzero initial state:
    the reference decode recurrence ``ref_recurrent_step`` is stepped token by
    token from h_prev = initial_state (mamba2.py:447-450), which is the
    reference's own state-carry semantics.
    """
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    b, L, H, P = x.shape
    Bg, G = _groups_of(B, H)
    Cg, _ = _groups_of(C, H)
    N = Bg.shape[-1]
    if np.any(A >= 0):
        raise ValueError("bridge needs A < 0 (a_h = -A_h > 0)")
    a = -A                                         # (H,)
    Dhp = _expand_D(D, H, P)
    hpg = H // G
    y = np.zeros((b, L, H, P))
    final = np.zeros((b, H, P, N))
    if return_h_states and initial_state is not None:
        raise ValueError("ssd_via_reference: h_states through the bridge needs a zero initial state")
    hs_all = np.zeros((b, L, N)) if return_h_states else None
    for g in range(G):
        hs = slice(g * hpg, (g + 1) * hpg)
        ag = a[hs]                                               # (hpg,)
        dt_ref = np.repeat((dt[:, :, hs] * ag[None, None, :])[..., None], P, axis=-1)
        x_ref = x[:, :, hs, :] / ag[None, None, :, None]
        D_ref = (Dhp[hs] * ag[:, None]).reshape(-1)
        dt_ref = dt_ref.reshape(b, L, hpg * P)
        x_ref = x_ref.reshape(b, L, hpg * P)
        A_log = np.zeros(N)
        if initial_state is None and return_h_states:
            yg, hsg, hg = ref_selective_scan(x_ref, dt_ref, A_log, Bg[:, :, g], Cg[:, :, g], D_ref,
                                             return_h_states=True, return_final_state=True)
            hs_all += hsg * (hpg * P) / (H * P)
        elif initial_state is None:
            yg, hg = ref_selective_scan(x_ref, dt_ref, A_log, Bg[:, :, g], Cg[:, :, g], D_ref,
                                        return_final_state=True)
        else:
            h = np.asarray(initial_state, np.float64)[:, hs].reshape(b, hpg * P, N)
            yg = np.zeros((b, L, hpg * P))
            for t in range(L):
                yt, h = ref_recurrent_step(x_ref[:, t:t + 1], dt_ref[:, t:t + 1],
                                           Bg[:, t:t + 1, g], Cg[:, t:t + 1, g], h, A_log, D_ref)
                yg[:, t] = yt[:, 0]
            hg = h
        y[:, :, hs, :] = yg.reshape(b, L, hpg, P)
        final[:, hs] = hg.reshape(b, hpg, P, N)
    if return_h_states:
        return y, final, hs_all
    return y, final


def ssd_h_states(x, dt, A, B, C=None, initial_state=None):
    """h_states[b,t,n] = mean over (h, p) of the SSD state after token t, in direct SSD form (any initial
    state); the quantity ``selective_scan(..., return_h_states=True)`` returns (mamba2.py:114-116)."""
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    b, L, H, P = x.shape
    Bg, G = _groups_of(B, H)
    N = Bg.shape[-1]
    gidx = np.arange(H) // (H // G)
    h = np.zeros((b, H, P, N)) if initial_state is None else np.array(initial_state, np.float64)
    hs = np.zeros((b, L, N))
    for t in range(L):
        dA = np.exp(A[None, :] * dt[:, t, :])
        Bt = Bg[:, t][:, gidx]
        h = dA[:, :, None, None] * h + (dt[:, t, :, None, None] * x[:, t, :, :, None]) * Bt[:, :, None, :]
        hs[:, t] = h.mean(axis=(1, 2))
    return hs


def ssd_direct(x, dt, A, B, C, D=None, initial_state=None):
    """SSD recurrence written directly in SSD form (independent of the bridge).

    h[b,h,p,n] <- exp(A_h dt[b,t,h]) h + dt[b,t,h] x[b,t,h,p] B[b,t,g(h),n]
    y[b,t,h,p]  = sum_n C[b,t,g(h),n] h[b,h,p,n] + D[h,p] x[b,t,h,p]
    Works for any real A (including A = 0).
    """
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    b, L, H, P = x.shape
    Bg, G = _groups_of(B, H)
    Cg, _ = _groups_of(C, H)
    N = Bg.shape[-1]
    gidx = np.arange(H) // (H // G)
    Dhp = _expand_D(D, H, P)
    h = np.zeros((b, H, P, N)) if initial_state is None else np.array(initial_state, np.float64)
    y = np.zeros((b, L, H, P))
    for t in range(L):
        dA = np.exp(A[None, :] * dt[:, t, :])                     # (b,H)
        Bt = Bg[:, t][:, gidx]                                     # (b,H,N)
        Ct = Cg[:, t][:, gidx]
        h = dA[:, :, None, None] * h + (dt[:, t, :, None, None] * x[:, t, :, :, None]) * Bt[:, :, None, :]
        y[:, t] = np.einsum("bhpn,bhn->bhp", h, Ct) + Dhp[None] * x[:, t]
    return y, h


def ssd_chunked(x, dt, A, B, C, D=None, initial_state=None, chunk_size=64):
    """Chunked SSD (the four-step decomposition) in float64 -- the blueprint of the HIP path.

    Per chunk: cs = cumsum(A*dt); intra-chunk Y = (C B^T o L) (dt x) with
    L[t,s] = exp(cs_t - cs_s) for s <= t; chunk state S = B^T (exp(cs_end - cs) dt x);
    state passing H_{c+1} = exp(cs_end) H_c + S_c; readout Y += exp(cs_t) C H_c^T; D skip.
    Must equal ``ssd_direct`` for any chunk size (including L % chunk_size != 0).
    """
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    b, L, H, P = x.shape
    Bg, G = _groups_of(B, H)
    Cg, _ = _groups_of(C, H)
    N = Bg.shape[-1]
    gidx = np.arange(H) // (H // G)
    Dhp = _expand_D(D, H, P)
    Hs = np.zeros((b, H, P, N)) if initial_state is None else np.array(initial_state, np.float64)
    y = np.zeros((b, L, H, P))
    for c0 in range(0, L, chunk_size):
        c1 = min(L, c0 + chunk_size)
        xc = x[:, c0:c1]                         # (b,Q,H,P)
        dtc = dt[:, c0:c1]                       # (b,Q,H)
        Bc = Bg[:, c0:c1][:, :, gidx]            # (b,Q,H,N)
        Cc = Cg[:, c0:c1][:, :, gidx]
        cs = np.cumsum(A[None, None, :] * dtc, axis=1)           # (b,Q,H)
        seg = cs[:, :, None, :] - cs[:, None, :, :]              # (b,t,s,H)
        Q = c1 - c0
        mask = np.tril(np.ones((Q, Q), bool))[None, :, :, None]
        Lm = np.where(mask, np.exp(np.where(mask, seg, 0.0)), 0.0)
        CB = np.einsum("bthn,bshn->btsh", Cc, Bc)
        M = CB * Lm * dtc[:, None, :, :]
        y_diag = np.einsum("btsh,bshp->bthp", M, xc)
        y_off = np.einsum("bthn,bhpn->bthp", Cc, Hs) * np.exp(cs)[..., None]
        y[:, c0:c1] = y_diag + y_off + Dhp[None, None] * xc
        w = np.exp(cs[:, -1:, :] - cs) * dtc                     # (b,Q,H)
        S = np.einsum("bsh,bshp,bshn->bhpn", w, xc, Bc)
        Hs = np.exp(cs[:, -1, :])[:, :, None, None] * Hs + S
    return y, Hs


def ssd_semiseparable(x, dt, A, B, C, D=None):
    """Brute force (tiny sizes): y = M x with the explicit semiseparable matrix.

    M[b,h][t,s] = C_t . B_s * exp(A_h * sum_{s<tau<=t} dt_tau) * dt_s   for s <= t.
    Zero initial state only.  Built from cumulative products of exp(A dt)
    (not from differences of a cumsum) so it is an independent construction.
    """
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    b, L, H, P = x.shape
    Bg, G = _groups_of(B, H)
    Cg, _ = _groups_of(C, H)
    gidx = np.arange(H) // (H // G)
    Dhp = _expand_D(D, H, P)
    y = np.zeros((b, L, H, P))
    for bi in range(b):
        for h in range(H):
            g = gidx[h]
            dec = np.exp(A[h] * dt[bi, :, h])        # per-step decay
            M = np.zeros((L, L))
            for t in range(L):
                prod = 1.0
                for s in range(t, -1, -1):
                    M[t, s] = np.dot(Cg[bi, t, g], Bg[bi, s, g]) * prod * dt[bi, s, h]
                    prod *= dec[s]
            y[bi, :, h, :] = M @ x[bi, :, h, :] + Dhp[h][None, :] * x[bi, :, h, :]
    return y


# ---------------------------------------------------------------------------
# Decode (selective state update)
# ---------------------------------------------------------------------------

def state_update_via_reference(state, x, dt, A, B, C, D=None, dt_bias=None, dt_softplus=True,
                               dt_limit=None):
    """One-token SSD state update computed by ``ref_recurrent_step`` through the bridge.

    state (b,H,P,N); x (b,H,P); dt (b,H) raw; A (H,) < 0; B, C (b,N) or (b,G,N);
    D None/(H,)/(H,P).  dt is processed first (bias, softplus, clamp) as the
    decode path of mamba2.py:293 does before calling _recurrent_step.
    Returns (y (b,H,P), new_state (b,H,P,N)) -- the reference returns a new
    tensor (mamba2.py:450, 458); the HIP op may update in place.
    """
    x = np.asarray(x, np.float64)
    b, H, P = x.shape
    d = process_dt(dt, dt_bias, dt_softplus, dt_limit)           # (b,H)
    Bn = np.asarray(B, np.float64)
    Cn = np.asarray(C, np.float64)
    if Bn.ndim == 2:
        Bn = Bn[:, None, :]
        Cn = Cn[:, None, :]
    G = Bn.shape[1]
    N = Bn.shape[-1]
    hpg = H // G
    A = np.asarray(A, np.float64)
    a = -A
    Dhp = _expand_D(D, H, P)
    y = np.zeros((b, H, P))
    new = np.zeros((b, H, P, N))
    for g in range(G):
        hs = slice(g * hpg, (g + 1) * hpg)
        ag = a[hs]
        dt_ref = np.repeat((d[:, hs] * ag[None, :])[..., None], P, axis=-1).reshape(b, 1, hpg * P)
        x_ref = (x[:, hs, :] / ag[None, :, None]).reshape(b, 1, hpg * P)
        D_ref = (Dhp[hs] * ag[:, None]).reshape(-1)
        h_prev = np.asarray(state, np.float64)[:, hs].reshape(b, hpg * P, N)
        yt, ht = ref_recurrent_step(x_ref, dt_ref, Bn[:, None, g], Cn[:, None, g], h_prev,
                                    np.zeros(N), D_ref)
        y[:, hs] = yt[:, 0].reshape(b, hpg, P)
        new[:, hs] = ht.reshape(b, hpg, P, N)
    return y, new


def state_update_direct(state, x, dt, A, B, C, D=None, dt_bias=None, dt_softplus=True, dt_limit=None):
    """Same update written directly: s <- exp(A dt) s + dt x B ; y = s.C + D x."""
    x = np.asarray(x, np.float64)
    b, H, P = x.shape
    d = process_dt(dt, dt_bias, dt_softplus, dt_limit)
    Bn = np.asarray(B, np.float64)
    Cn = np.asarray(C, np.float64)
    if Bn.ndim == 2:
        Bn = Bn[:, None, :]
        Cn = Cn[:, None, :]
    G = Bn.shape[1]
    gidx = np.arange(H) // (H // G)
    Dhp = _expand_D(D, H, P)
    A = np.asarray(A, np.float64)
    s = np.asarray(state, np.float64)
    dA = np.exp(A[None, :] * d)
    s = dA[:, :, None, None] * s + (d[:, :, None, None] * x[:, :, :, None]) * Bn[:, gidx][:, :, None, :]
    y = np.einsum("bhpn,bhn->bhp", s, Cn[:, gidx]) + Dhp[None] * x
    return y, s
