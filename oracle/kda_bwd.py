"""Float64 oracle for the gradient of the reference's normalised linear-attention scan (KDA backward).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference trains LinearDiffAttention through PyTorch autograd of its eager chunked scan
``_linear_attention_scan`` (R/mamformer/layers/kda_diff.py:357-478; the Triton scan it prefers,
triton_ssd.py:260-350, returns plain tensors with no autograd node).  That scan computes, per head,

    phi(x) = elu(x[..., :K]) + 1                                  (kda_diff.py:67-89)
    S_t = S_{t-1} + phi(k_t)^T v_t,   z_t = z_{t-1} + phi(k_t)     (inclusive of token t)
    num_i,t = phi(q_i,t) S_t,   n_i,t = phi(q_i,t) . z_t + 1e-8,   o_i,t = num_i,t / n_i,t
    out = (o_1 - lam o_2) / (1 - lam + 1e-8),  lam = min(sigmoid(lambda_raw), 0.99)   (:473-478)

and this module states its gradient as the adjoint recurrence, token by token:

    dnum_i,t = do_i,t / n_i,t,            dn_i,t = -(do_i,t . num_i,t) / n_i,t^2
    dphi(q_i,t) = S_t dnum_i,t + dn_i,t z_t
    Lam_t = Lam_{t+1} + sum_i phi(q_i,t)^T dnum_i,t,   zeta_t = zeta_{t+1} + sum_i dn_i,t phi(q_i,t)
    dphi(k_t) = Lam_t v_t + zeta_t,       dv_t = Lam_t^T phi(k_t)
    dS_0 = Lam_0,  dz_0 = zeta_0          (gradients of the initial state and normaliser)

starting from Lam_L = d_final_state, zeta_L = d_final_z (zero unless the final state enters the loss).

with dq = dphi(q) * phi'(q) (phi' = 1 above 0, e^x at or below, 0 beyond channel K) and the same for dk.
Pinned in ``tests/test_oracle_kda_bwd.py`` against torch autograd of the attention-matrix form
(row-normalised causal phi(q) phi(k)^T weights), against finite differences, and by planted mistakes.
"""

from __future__ import annotations

import numpy as np

from .kda import diff_lambda, feature_map

__all__ = ["phi_grad", "ref_scan_pair_backward", "ref_attention_scan_backward"]


def phi_grad(x, K):
    """d phi / d x elementwise on the first K channels (elu'(x) = 1 for x > 0, e^x otherwise)."""
    x = np.asarray(x, np.float64)[..., :K]
    return np.where(x > 0, 1.0, np.exp(np.minimum(x, 0.0)))


def ref_scan_pair_backward(q1, q2, k, v, kernel_dim, do1, do2=None, initial_state=None, initial_z=None,
                           d_final_state=None, d_final_z=None):
    """Gradients of <do1, o1> + <do2, o2> (+ <d_final_state, S_L> + <d_final_z, z_L>) for (o1, o2, S_L, z_L) =
    the reference-mode scan (``oracle.kda.ref_scan_pair``).

    q1, q2, k (B, H, S, Dk); v, do1, do2 (B, H, S, D); q2 / do2 None for a single query stream.
    Returns a dict of float64 arrays: dq1, dq2 (absent without q2), dk shaped like q1 (zero beyond channel
    K = min(kernel_dim, Dk)), dv like v, dS0 (B, H, K, D), dz0 (B, H, K), and o1, o2 (the forward outputs).
    """
    v = np.asarray(v, np.float64)
    Bb, H, S, D = v.shape
    Dk = np.asarray(q1).shape[-1]
    K = min(kernel_dim, Dk)
    qs = [q1] if q2 is None else [q1, q2]
    dos = [np.asarray(do1, np.float64)] + ([] if q2 is None else
                                           [np.zeros_like(v) if do2 is None else np.asarray(do2, np.float64)])
    ps = [feature_map(q, K) for q in qs]
    pk = feature_map(k, K)
    st = np.zeros((Bb, H, K, D)) if initial_state is None else np.array(initial_state, np.float64)
    z = np.zeros((Bb, H, K)) if initial_z is None else np.array(initial_z, np.float64).reshape(Bb, H, K)
    Ss, zs = [], []
    for t in range(S):
        st = st + pk[:, :, t, :, None] * v[:, :, t, None, :]
        z = z + pk[:, :, t]
        Ss.append(st)
        zs.append(z)
    dps = [np.zeros((Bb, H, S, K)) for _ in qs]
    os_ = [np.zeros((Bb, H, S, D)) for _ in qs]
    dpk = np.zeros((Bb, H, S, K))
    dv = np.zeros_like(v)
    lam_ = np.zeros((Bb, H, K, D)) if d_final_state is None else np.array(d_final_state, np.float64)
    zeta = np.zeros((Bb, H, K)) if d_final_z is None else np.array(d_final_z, np.float64).reshape(Bb, H, K)
    for t in reversed(range(S)):
        for i, p in enumerate(ps):
            num = np.einsum("bhk,bhkd->bhd", p[:, :, t], Ss[t])
            n = np.einsum("bhk,bhk->bh", p[:, :, t], zs[t]) + 1e-8
            os_[i][:, :, t] = num / n[..., None]
            dnum = dos[i][:, :, t] / n[..., None]
            dn = -np.einsum("bhd,bhd->bh", dos[i][:, :, t], num) / n ** 2
            dps[i][:, :, t] = np.einsum("bhkd,bhd->bhk", Ss[t], dnum) + dn[..., None] * zs[t]
            lam_ = lam_ + p[:, :, t, :, None] * dnum[:, :, None, :]
            zeta = zeta + dn[..., None] * p[:, :, t]
        dpk[:, :, t] = np.einsum("bhkd,bhd->bhk", lam_, v[:, :, t]) + zeta
        dv[:, :, t] = np.einsum("bhkd,bhk->bhd", lam_, pk[:, :, t])

    def pad(g):
        out = np.zeros(g.shape[:-1] + (Dk,))
        out[..., :K] = g
        return out

    res = {"dq1": pad(dps[0] * phi_grad(q1, K)), "dk": pad(dpk * phi_grad(k, K)), "dv": dv,
           "dS0": lam_, "dz0": zeta, "o1": os_[0]}
    if q2 is not None:
        res["dq2"] = pad(dps[1] * phi_grad(q2, K))
        res["o2"] = os_[1]
    return res


def ref_attention_scan_backward(q1, q2, k, v, kernel_dim, lambda_raw, dout):
    """Gradients of <dout, out> for out = ``oracle.kda.ref_attention_scan`` (the differential combination of
    kda_diff.py:473-478 over the scan pair, zero initial state).  Returns dq1, dq2, dk, dv and d_lambda_raw
    (H,), the last through lam = min(sigmoid(lambda_raw), 0.99) with torch's clamp backward (gradient passes
    where sigmoid(lambda_raw) <= 0.99)."""
    lam = diff_lambda(lambda_raw)                                   # (H,)
    c = 1.0 / (1.0 - lam + 1e-8)
    dout = np.asarray(dout, np.float64)
    do1 = dout * c[None, :, None, None]
    do2 = -dout * (lam * c)[None, :, None, None]
    r = ref_scan_pair_backward(q1, q2, k, v, kernel_dim, do1, do2)
    o1, o2 = r["o1"], r["o2"]
    # d out / d lam = (-o2 (1 - lam + eps) + (o1 - lam o2)) / (1 - lam + eps)^2 = c^2 (o1 - (1 + eps) o2)
    c2 = (c ** 2)[None, :, None, None]
    dlam = np.einsum("bhsd,bhsd->h", dout, c2 * (o1 - (1.0 + 1e-8) * o2))
    lr = np.asarray(lambda_raw, np.float64)
    sg = 1.0 / (1.0 + np.exp(-lr))
    dlr = dlam * sg * (1.0 - sg) * (sg <= 0.99)
    # o1, o2 ride along so that a check can scale d_lambda_raw by the magnitude of the terms it sums
    return {"dq1": r["dq1"], "dq2": r["dq2"], "dk": r["dk"], "dv": r["dv"], "d_lambda_raw": dlr, "o1": o1, "o2": o2}
