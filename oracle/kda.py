"""Float64 oracle for the KDA-Diff linear-attention scans.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Two operators share one kernel in the HIP path:

1. **Reference mode** -- the reference's normalised differential linear
   attention.  Restated from (``R`` = ``/root/reference/mamformer 671b/``):
     * ``kernel_feature_map``            R/mamformer/layers/kda_diff.py:67-89   phi(x) = elu(x[..., :K]) + 1
     * ``_linear_attention_scan``        R/mamformer/layers/kda_diff.py:357-478 S += phi(k)^T v, z += phi(k),
                                         o_i = phi(q_i) S / (phi(q_i) z + 1e-8), (o1 - lam o2)/(1 - lam + 1e-8)
     * ``triton_linear_attn_scan``       R/mamformer/kernels/triton_ssd.py:121-181 (same math, returns (o1, o2))
     * ``_linear_attention_recurrent``   R/mamformer/layers/kda_diff.py:564-605 (one token, phi already applied)
     * lambda = min(sigmoid(lambda_raw_h), 0.99)                                  kda_diff.py:473-474
   The update is *inclusive*: token t is added to the state before it is read
   out (triton_ssd.py:139-169; cumsum inclusive at kda_diff.py:433).

2. **Gated mode** -- the decay-gated, un-normalised recurrence of the KDA
   benchmark configuration, which no reference function computes:
     S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,   o_t = q1_t S_t - lam * q2_t S_t
   (identity feature map, no normaliser, no (1 - lam) division).  With g == 0
   it is the causal linear attention sum_{s<=t} (q_t . k_s) v_s.

Layout everywhere: (batch, heads, seq, dim) as in the reference (kda_diff.py:270-273).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "sigmoid",
    "feature_map",
    "diff_lambda",
    "gated_recurrent",
    "gated_closed_form",
    "gated_chunked",
    "ref_scan_pair",
    "ref_attention_scan",
    "ref_attention_recurrent",
    "ref_attention_matrix",
]


def sigmoid(x):
    x = np.asarray(x, np.float64)
    return 1.0 / (1.0 + np.exp(-x))


def feature_map(x, kernel_dim):
    """phi(x) = elu(x[..., :K]) + 1 (kda_diff.py:87-89); elu(x) = x if x > 0 else exp(x) - 1."""
    xs = np.asarray(x, np.float64)[..., :kernel_dim]
    return np.where(xs > 0.0, xs + 1.0, np.exp(np.minimum(xs, 0.0)))


def diff_lambda(lambda_raw):
    """lambda = clamp(sigmoid(lambda_raw), max=0.99) per head (kda_diff.py:473-474)."""
    return np.minimum(sigmoid(lambda_raw), 0.99)


# ---------------------------------------------------------------------------
# Gated mode (benchmark configuration; no reference function)
# ---------------------------------------------------------------------------

def gated_recurrent(q1, q2, k, v, g, lam, initial_state=None):
    """Token-by-token recurrence.  q1,q2,k,g (B,H,S,K); v (B,H,S,V); lam scalar or (H,).

    Returns (o (B,H,S,V), final_state (B,H,K,V)).
    """
    q1 = np.asarray(q1, np.float64)
    q2 = np.asarray(q2, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.zeros_like(k) if g is None else np.asarray(g, np.float64)
    Bb, H, S, K = k.shape
    V = v.shape[-1]
    lam = np.broadcast_to(np.asarray(lam, np.float64), (H,))
    st = np.zeros((Bb, H, K, V)) if initial_state is None else np.array(initial_state, np.float64)
    o = np.zeros((Bb, H, S, V))
    for t in range(S):
        st = np.exp(g[:, :, t, :, None]) * st + k[:, :, t, :, None] * v[:, :, t, None, :]
        o1 = np.einsum("bhk,bhkv->bhv", q1[:, :, t], st)
        o2 = np.einsum("bhk,bhkv->bhv", q2[:, :, t], st)
        o[:, :, t] = o1 - lam[None, :, None] * o2
    return o, st


def gated_closed_form(q1, q2, k, v, g, lam, initial_state=None):
    """Brute force: o_t = sum_{s<=t} sum_k qe_t[k] exp(G_t[k]-G_s[k]) k_s[k] v_s + sum_k qe_t[k] exp(G_t[k]) S0[k,:].

    G = inclusive cumsum of g over time, qe = q1 - lam q2.  Final state
    S_T[k,:] = exp(G_T[k]) S0[k,:] + sum_s exp(G_T[k]-G_s[k]) k_s[k] v_s.
    """
    q1 = np.asarray(q1, np.float64)
    q2 = np.asarray(q2, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.zeros_like(k) if g is None else np.asarray(g, np.float64)
    Bb, H, S, K = k.shape
    V = v.shape[-1]
    lam = np.broadcast_to(np.asarray(lam, np.float64), (H,))
    qe = q1 - lam[None, :, None, None] * q2
    G = np.cumsum(g, axis=2)
    S0 = np.zeros((Bb, H, K, V)) if initial_state is None else np.asarray(initial_state, np.float64)
    o = np.zeros((Bb, H, S, V))
    for t in range(S):
        dec = np.exp(G[:, :, t:t + 1, :] - G[:, :, :t + 1, :])          # (B,H,t+1,K)
        w = np.einsum("bhk,bhsk,bhsk->bhs", qe[:, :, t], dec, k[:, :, :t + 1])
        o[:, :, t] = np.einsum("bhs,bhsv->bhv", w, v[:, :, :t + 1])
        o[:, :, t] += np.einsum("bhk,bhk,bhkv->bhv", qe[:, :, t], np.exp(G[:, :, t]), S0)
    decT = np.exp(G[:, :, -1:, :] - G)                                  # (B,H,S,K)
    ST = np.exp(G[:, :, -1, :, None]) * S0 + np.einsum("bhsk,bhsk,bhsv->bhkv", decT, k, v)
    return o, ST


def gated_chunked(q1, q2, k, v, g, lam, initial_state=None, chunk_size=64):
    """Chunked form of the gated recurrence (the blueprint of the HIP kernel), float64.

    Per chunk with in-chunk cumulative log-decay G (B,H,Q,K):
      A[t,s] = sum_k qe_t[k] k_s[k] exp(G_t[k]-G_s[k])  (s <= t)
      o = A v + (qe * exp(G)) S ;  S <- exp(G_end) S + sum_s (k_s exp(G_end-G_s))^T v_s
    """
    q1 = np.asarray(q1, np.float64)
    q2 = np.asarray(q2, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.zeros_like(k) if g is None else np.asarray(g, np.float64)
    Bb, H, S, K = k.shape
    V = v.shape[-1]
    lam = np.broadcast_to(np.asarray(lam, np.float64), (H,))
    qe = q1 - lam[None, :, None, None] * q2
    st = np.zeros((Bb, H, K, V)) if initial_state is None else np.array(initial_state, np.float64)
    o = np.zeros((Bb, H, S, V))
    for c0 in range(0, S, chunk_size):
        c1 = min(S, c0 + chunk_size)
        Q = c1 - c0
        G = np.cumsum(g[:, :, c0:c1], axis=2)
        qc, kc, vc = qe[:, :, c0:c1], k[:, :, c0:c1], v[:, :, c0:c1]
        mask = np.tril(np.ones((Q, Q), bool))
        dec = G[:, :, :, None, :] - G[:, :, None, :, :]                  # (B,H,t,s,K)
        dec = np.where(mask[None, None, :, :, None], np.exp(np.where(mask[None, None, :, :, None], dec, 0.0)), 0.0)
        A = np.einsum("bhtk,bhsk,bhtsk->bhts", qc, kc, dec)
        o[:, :, c0:c1] = np.einsum("bhts,bhsv->bhtv", A, vc) + np.einsum("bhtk,bhkv->bhtv", qc * np.exp(G), st)
        wk = kc * np.exp(G[:, :, -1:, :] - G)
        st = np.exp(G[:, :, -1, :, None]) * st + np.einsum("bhsk,bhsv->bhkv", wk, vc)
    return o, st


# ---------------------------------------------------------------------------
# Reference mode (the reference's own operator)
# ---------------------------------------------------------------------------

def ref_scan_pair(q1, q2, k, v, kernel_dim, initial_state=None, initial_z=None):
    """Restates ``_linear_attn_scan_kernel`` (triton_ssd.py:121-181): returns (o1, o2, S, z).

    Per token (inclusive): S += phi(k)^T v (K x D), z += phi(k) (K);
    o_i = phi(q_i) S / (phi(q_i) z + 1e-8).  K = min(kernel_dim, head_dim).
    ``initial_state``/``initial_z`` default to zero (the reference scan always
    starts from zero: kda_diff.py:407-408, triton_ssd.py:112-113).
    """
    v = np.asarray(v, np.float64)
    Bb, H, S, Dd = v.shape
    K = min(kernel_dim, np.asarray(q1).shape[-1])
    p1 = feature_map(q1, K)
    p2 = feature_map(q2, K)
    pk = feature_map(k, K)
    st = np.zeros((Bb, H, K, Dd)) if initial_state is None else np.array(initial_state, np.float64)
    z = np.zeros((Bb, H, K)) if initial_z is None else np.array(initial_z, np.float64).reshape(Bb, H, K)
    o1 = np.zeros((Bb, H, S, Dd))
    o2 = np.zeros((Bb, H, S, Dd))
    for t in range(S):
        st = st + pk[:, :, t, :, None] * v[:, :, t, None, :]
        z = z + pk[:, :, t]
        n1 = np.einsum("bhk,bhkd->bhd", p1[:, :, t], st)
        d1 = np.einsum("bhk,bhk->bh", p1[:, :, t], z) + 1e-8
        n2 = np.einsum("bhk,bhkd->bhd", p2[:, :, t], st)
        d2 = np.einsum("bhk,bhk->bh", p2[:, :, t], z) + 1e-8
        o1[:, :, t] = n1 / d1[..., None]
        o2[:, :, t] = n2 / d2[..., None]
    return o1, o2, st, z


def ref_attention_scan(q1, q2, k, v, kernel_dim, lambda_raw):
    """Restates ``LinearDiffAttention._linear_attention_scan`` (kda_diff.py:357-478) in float64.

    The chunking of the reference (kda_diff.py:413-466) does not change the
    exact result; it is evaluated token by token here.  Returns (B,H,S,D).
    """
    o1, o2, _, _ = ref_scan_pair(q1, q2, k, v, kernel_dim)
    lam = diff_lambda(lambda_raw)[None, :, None, None]
    return (o1 - lam * o2) / (1.0 - lam + 1e-8)


def ref_attention_recurrent(q1_phi, q2_phi, k_phi, v, S, z, lambda_raw):
    """Restates ``_linear_attention_recurrent`` (kda_diff.py:564-605); inputs already feature-mapped.

    q*_phi, k_phi (B,H,1,K); v (B,H,1,D); S (B,H,K,D); z (B,H,K,1).
    Returns (diff_output (B,H,1,D), S_new, z_new) -- S_new/z_new are the
    values the reference's cache update (kda_diff.py:329-338) stores for a
    one-token step.
    """
    q1p = np.asarray(q1_phi, np.float64)
    q2p = np.asarray(q2_phi, np.float64)
    kp = np.asarray(k_phi, np.float64)
    v = np.asarray(v, np.float64)
    kt = np.swapaxes(kp, -2, -1)                        # (B,H,K,1)
    S = np.asarray(S, np.float64) + kt @ v
    z = np.asarray(z, np.float64) + kt
    out1 = (q1p @ S) / ((q1p @ z) + 1e-8)
    out2 = (q2p @ S) / ((q2p @ z) + 1e-8)
    lam = diff_lambda(lambda_raw)[None, :, None, None]
    return (out1 - lam * out2) / (1.0 - lam + 1e-8), S, z


def ref_attention_matrix(q, k, v, kernel_dim):
    """Brute force for one query stream: causal row-normalised phi(q) phi(k)^T attention.

    o_t = sum_{s<=t} a_ts v_s / (sum_{s<=t} a_ts + 1e-8),  a_ts = phi(q_t) . phi(k_s).
    """
    K = min(kernel_dim, np.asarray(q).shape[-1])
    pq = feature_map(q, K)
    pk = feature_map(k, K)
    v = np.asarray(v, np.float64)
    S = v.shape[2]
    a = np.einsum("bhtk,bhsk->bhts", pq, pk) * np.tril(np.ones((S, S)))[None, None]
    return np.einsum("bhts,bhsd->bhtd", a, v) / (a.sum(-1)[..., None] + 1e-8)
