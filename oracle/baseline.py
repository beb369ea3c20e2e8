"""Torch-CPU restatement of the reference's scan path, kept at the reference's cost structure.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): timed by ``bench.py``'s
``cpu_baseline`` leg as "the reference's pure-PyTorch CPU path".  The reference
code itself cannot travel to the GPU box, so this module re-expresses its
algorithm with the same materialisations and loop structure:

* ``selective_scan_cpu`` -- ``_selective_scan_impl`` (R/mamformer/layers/mamba2.py:84-126):
  A_disc / B_disc / Bx materialised at (b, L, d_inner, N), then one torch
  step per timestep (decay-multiply, add, C-contract) and the D skip.
* ``recurrent_step_cpu`` -- ``Mamba2Block._recurrent_step`` (mamba2.py:431-458).
* ``linear_attention_scan_cpu`` -- ``LinearDiffAttention._linear_attention_scan``
  (R/mamformer/layers/kda_diff.py:390-478) with its bf16 intermediates and
  per-chunk (B,H,C,K,D) outer-product tensors.

Inputs reach the reference form through the SSD bridge (A_log = 0,
dt_ref = a_h dt, x_ref = x / a_h, D_ref = a_h D) so the work per token is the
reference's.  ``R`` = ``/root/reference/mamformer 671b/``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def bridge(x4, dt, A, D):
    """SSD (b,L,H,P)/(b,L,H)/(H,)/(H,) -> reference (b,L,d_inner) dt/x, A_log (zeros), D (d_inner)."""
    b, L, H, P = x4.shape
    a = -A.to(torch.float32)
    dt_ref = (dt.to(torch.float32) * a).unsqueeze(-1).expand(b, L, H, P).reshape(b, L, H * P)
    x_ref = (x4.to(torch.float32) / a[None, None, :, None]).reshape(b, L, H * P)
    D_ref = (D.to(torch.float32) * a).unsqueeze(-1).expand(H, P).reshape(H * P)
    return x_ref, dt_ref, D_ref


def selective_scan_cpu(x, dt, A_log, B, C, D):
    """``_selective_scan_impl`` (mamba2.py:84-126) in fp32 on the CPU, same materialisation and loop."""
    batch, seqlen, d_inner = x.shape
    d_state = A_log.shape[0]
    A_param = torch.exp(torch.clamp(A_log, min=-5.0, max=5.0))
    dt_e = dt.unsqueeze(-1)
    A_disc = torch.exp(-A_param.view(1, 1, 1, d_state) * dt_e)
    B_disc = B.unsqueeze(2) * dt_e
    Bx = B_disc * x.unsqueeze(-1)
    h = torch.zeros(batch, d_inner, d_state, dtype=x.dtype)
    y = torch.zeros(batch, seqlen, d_inner, dtype=x.dtype)
    for t in range(seqlen):
        h = A_disc[:, t] * h + Bx[:, t]
        y[:, t] = torch.sum(C[:, t].unsqueeze(1) * h, dim=-1)
    return y + D.view(1, 1, d_inner) * x, h


def recurrent_step_cpu(x_t, dt_t, B_t, C_t, h_prev, A_log, D):
    """``_recurrent_step`` body (mamba2.py:441-456) for one token, fp32 on the CPU."""
    A_disc = torch.exp(-torch.exp(A_log).unsqueeze(0) * dt_t.unsqueeze(-1))
    B_disc = B_t.unsqueeze(1) * dt_t.unsqueeze(-1)
    h_t = A_disc * h_prev + B_disc * x_t.unsqueeze(-1)
    y_t = (C_t.unsqueeze(1) * h_t).sum(dim=-1) + D * x_t
    return y_t, h_t


def linear_attention_scan_cpu(q1, q2, k, v, kernel_dim, lambda_raw, chunk_size=64):
    """``_linear_attention_scan`` (kda_diff.py:390-478) on the CPU with the reference's chunk tensors."""
    B, H, S, D_full = q1.shape
    K_dim = kernel_dim
    compute_dtype = torch.bfloat16 if q1.dtype == torch.float32 else q1.dtype
    q1_phi = (F.elu(q1[..., :K_dim]) + 1.0).to(compute_dtype)
    q2_phi = (F.elu(q2[..., :K_dim]) + 1.0).to(compute_dtype)
    k_phi = (F.elu(k[..., :K_dim]) + 1.0).to(compute_dtype)
    S_state = torch.zeros(B, H, K_dim, D_full, dtype=torch.float32)
    z_state = torch.zeros(B, H, K_dim, 1, dtype=torch.float32)
    o1s, o2s = [], []
    for start in range(0, S, chunk_size):
        end = min(start + chunk_size, S)
        c = end - start
        k_c = k_phi[:, :, start:end]
        v_c = v[:, :, start:end].to(compute_dtype)
        q1_c = q1_phi[:, :, start:end]
        q2_c = q2_phi[:, :, start:end]
        kv_c = torch.bmm(k_c.reshape(B * H * c, K_dim, 1), v_c.reshape(B * H * c, 1, D_full))
        kv_c = kv_c.reshape(B, H, c, K_dim, D_full)
        kv_cum = torch.cumsum(kv_c, dim=2) + S_state.unsqueeze(2).to(compute_dtype)
        k_cum = torch.cumsum(k_c, dim=2) + z_state.squeeze(-1).unsqueeze(2).to(compute_dtype)
        kv_f = kv_cum.reshape(B * H * c, K_dim, D_full)
        q1_f = q1_c.reshape(B * H * c, 1, K_dim)
        q2_f = q2_c.reshape(B * H * c, 1, K_dim)
        o1 = torch.bmm(q1_f, kv_f).reshape(B, H, c, D_full)
        o2 = torch.bmm(q2_f, kv_f).reshape(B, H, c, D_full)
        kc_f = k_cum.reshape(B * H * c, K_dim, 1)
        n1 = torch.bmm(q1_f, kc_f).reshape(B, H, c)
        n2 = torch.bmm(q2_f, kc_f).reshape(B, H, c)
        o1s.append((o1 / (n1.unsqueeze(-1) + 1e-8)).to(q1.dtype))
        o2s.append((o2 / (n2.unsqueeze(-1) + 1e-8)).to(q1.dtype))
        S_state = S_state + kv_c.sum(dim=2).to(torch.float32)
        z_state = z_state + k_c.sum(dim=2).unsqueeze(-1).to(torch.float32)
    o1 = torch.cat(o1s, 2)
    o2 = torch.cat(o2s, 2)
    lam = torch.clamp(torch.sigmoid(lambda_raw).view(1, H, 1, 1), max=0.99)
    return (o1 - lam * o2) / (1.0 - lam + 1e-8)


def ssd_prefill_sample(x4, dt, A, B, C, D):
    """Run the reference prefill on an SSD-convention sample (group 0); returns y (b, L, d_inner)."""
    x_ref, dt_ref, D_ref = bridge(x4, dt, A, D)
    N = B.shape[-1]
    return selective_scan_cpu(x_ref, dt_ref, torch.zeros(N), B[:, :, 0].float(), C[:, :, 0].float(), D_ref)[0]

