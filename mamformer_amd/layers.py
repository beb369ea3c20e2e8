"""Layer-level counterparts of the reference's scan call sites.

``Mamba2Layer`` mirrors ``Mamba2Block`` (R/mamformer/layers/mamba2.py:153-364) around the
SSD scan: in_proj -> causal depthwise conv1d -> SiLU -> dt/B/C projections -> scan (full
prefill, or the one-token recurrent step when a cache holds an SSM state) -> SiLU(z) gate
-> out_proj, with the reference's cache dict ``{"conv_state", "ssm_state"}``.  The conv,
SiLU, scan, z-gate and decode step run the HIP kernels of ``mamformer_amd.ops`` (conv and
SiLU fused; the gate applied by the scan / step kernels as y is stored); the projections are
plain library GEMMs.

Recorded deviation (per-head SSD convention): the reference parameterises dt per channel
(``dt_proj: d_inner -> d_inner``) and A per state (``A_log (d_state,)``), which is a
Mamba-1-style diagonal decay that is not MFMA-factorable.  Here ``dt_proj`` ends in
``nheads`` outputs, ``A_log``, ``D`` and ``dt_bias`` are per head, and B/C have ``ngroups``
groups; dt = softplus(dt_proj(x) + dt_bias) inside the kernel.

``kda_linear_attention`` mirrors the recurrent-state handling of
``LinearDiffAttention.forward`` (R/mamformer/layers/kda_diff.py:286-338) on already
projected, rotated and GQA-expanded q1, q2, k, v (B, H, S, D).
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from . import ops

__all__ = ["Mamba2Layer", "kda_linear_attention"]


class Mamba2Layer(nn.Module):
    """Head-structured Mamba-2 layer; forward/cache semantics of ``Mamba2Block.forward`` (mamba2.py:249-364)."""

    def __init__(self, d_model: int, d_state: int = 128, d_conv: int = 4, expand: int = 1, headdim: int = 64,
                 ngroups: int = 1, dt_rank: Optional[int] = None, bias: bool = False, device=None, dtype=None):
        super().__init__()
        fk = {"device": device, "dtype": dtype}
        self.d_model = d_model
        self.d_inner = d_model * expand
        if self.d_inner % headdim:
            raise ValueError("Mamba2Layer: d_model * expand must be a multiple of headdim")
        self.headdim = headdim
        self.nheads = self.d_inner // headdim
        if self.nheads % ngroups:
            raise ValueError("Mamba2Layer: nheads must be a multiple of ngroups")
        self.ngroups = ngroups
        self.d_state = d_state
        self.d_conv = d_conv
        self.dt_rank = dt_rank if dt_rank is not None else math.ceil(d_model / 32)       # mamba2.py:191
        self.in_proj = nn.Linear(d_model, 2 * self.d_inner, bias=bias, **fk)
        self.conv_weight = nn.Parameter(torch.empty(self.d_inner, 1, d_conv, **fk))      # nn.Conv1d depthwise layout
        self.conv_bias = nn.Parameter(torch.zeros(self.d_inner, **fk)) if bias else None
        self.dt_proj = nn.Sequential(nn.Linear(self.d_inner, self.dt_rank, bias=bias, **fk),
                                     nn.Linear(self.dt_rank, self.nheads, bias=bias, **fk))
        self.B_proj = nn.Linear(self.d_inner, ngroups * d_state, bias=bias, **fk)
        self.C_proj = nn.Linear(self.d_inner, ngroups * d_state, bias=bias, **fk)
        self.A_log = nn.Parameter(torch.log(torch.linspace(1.0, 16.0, self.nheads, device=device)))
        self.dt_bias = nn.Parameter(torch.zeros(self.nheads, device=device))
        self.D = nn.Parameter(torch.ones(self.nheads, device=device))
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=bias, **fk)
        self._init_weights()

    def _init_weights(self):
        """Initialisation of mamba2.py:229-247 (normal, std 0.02; dt projection std 0.001)."""
        nn.init.normal_(self.in_proj.weight, std=0.02)
        nn.init.normal_(self.out_proj.weight, std=0.02)
        for layer in self.dt_proj:
            nn.init.normal_(layer.weight, std=0.001)
        nn.init.normal_(self.B_proj.weight, std=0.02)
        nn.init.normal_(self.C_proj.weight, std=0.02)
        nn.init.normal_(self.conv_weight, std=0.02)

    def forward(self, u: torch.Tensor, use_cache: bool = False, cache: Optional[dict] = None,
                return_h_states: bool = False):
        """u (b, L, d_model) -> (out, cache) or (out, cache, h_states), as mamba2.py:249-364.

        Path choice of mamba2.py:285-334: an incremental one-token step (only the last token's SSM
        output, :296 / :435-438) when ``use_cache`` and ``cache["ssm_state"]`` is set; otherwise the full
        chunked scan.  The cache is ``{"conv_state": last d_conv-1 raw x rows, "ssm_state": (b, d_inner, N)
        fp32}`` (:343-364).
        """
        b, L, _ = u.shape
        x, z = self.in_proj(u).chunk(2, dim=-1)                 # mamba2.py:272-273
        raw_x = x
        conv_state = cache.get("conv_state") if (use_cache and cache is not None) else None
        x_act = ops.causal_conv1d(x, self.conv_weight, self.conv_bias, conv_state, silu=True)   # :279-283
        incremental = use_cache and cache is not None and cache.get("ssm_state") is not None    # :289
        dt = self.dt_proj(x_act)                                 # (b, L, H); softplus(+ dt_bias) in the kernel
        Bm = self.B_proj(x_act).view(b, L, self.ngroups, self.d_state)
        Cm = self.C_proj(x_act).view(b, L, self.ngroups, self.d_state)
        # A_log is clamped to [-5, 5] on the prefill path only, as the reference does (clamp in the scan,
        # mamba2.py:87; none in the decode step, :441-443)
        A_log = self.A_log.float()
        A = -torch.exp(A_log if incremental else A_log.clamp(-5.0, 5.0))
        D = self.D.float()
        h_states = None
        # the z-gate y * silu(z) (:337-338) is applied by the kernels as y is stored
        if incremental:
            y, final = ops.recurrent_step(x_act, dt, Bm, Cm, cache["ssm_state"], A, D,
                                          dt_bias=self.dt_bias, dt_softplus=True, z=z)
        else:
            res = ops.selective_scan(x_act, dt, A, Bm, Cm, D, return_h_states=return_h_states,
                                     return_final_state=use_cache, dt_bias=self.dt_bias, dt_softplus=True, z=z)
            res = res if isinstance(res, tuple) else (res,)
            y = res[0]
            h_states = res[1] if return_h_states else None
            final = res[-1] if use_cache else None
        out = self.out_proj(y)
        new_cache = None
        if use_cache:
            k = self.d_conv - 1
            conv_x = raw_x[:, -k:] if raw_x.shape[1] >= self.d_conv else raw_x   # :355
            if cache is not None and "conv_state" in cache:
                conv_x = torch.cat([cache["conv_state"], conv_x], dim=1)[:, -k:]
            new_cache = {"conv_state": conv_x, "ssm_state": final}
        if return_h_states:
            return out, new_cache, h_states
        return out, new_cache


def kda_linear_attention(q1, q2, k, v, lambda_raw, kernel_dim, use_cache=False, cache=None):
    """Recurrent-state semantics of ``LinearDiffAttention.forward`` (R/mamformer/layers/kda_diff.py:286-338).

    q1, q2, k, v (B, H, S, D) after projection, RoPE and GQA expansion; lambda_raw (H,); kernel_dim K.
    * seq_len == 1 with ``use_cache``: one recurrent step from the cached (S, z) (:301-308, :564-605).
    * otherwise the normalised chunked scan from a zero state -- a cached state is *not* used for the
      outputs of a multi-token forward (:309-325, reference quirk, kept).
    * with ``use_cache`` the new cache is S = S_prev + phi(K)^T V, z = z_prev + sum_t phi(k_t) (:327-338),
      S (B, H, K, D) and z (B, H, K, 1) in float32.
    Returns (attn_output (B, H, S, D), new_cache or None).
    """
    Bb, H, S, Dh = q1.shape
    K = min(int(kernel_dim), Dh)
    if use_cache and cache is not None and cache.get("attn_type") == "linear":
        S_prev = cache["S"].to(torch.float32)
        z_prev = cache["z"].to(torch.float32)
    else:
        S_prev = torch.zeros((Bb, H, K, Dh), device=q1.device, dtype=torch.float32)
        z_prev = torch.zeros((Bb, H, K, 1), device=q1.device, dtype=torch.float32)
    lam = ops.diff_lambda(lambda_raw)
    if S == 1 and use_cache:
        # one in-place step (dk = K) on fp32 copies of the cache, which become the new cache (the reference
        # returns new tensors): the state has K rows, so only the first K channels of q and k enter
        St = S_prev.clone(memory_format=torch.contiguous_format)
        zt = z_prev.clone(memory_format=torch.contiguous_format)
        out = ops.linear_attn_step(St, zt, q1[..., :K], q2[..., :K], k[..., :K], v, lam=lam, kernel_dim=K,
                                   apply_phi=True)
        out = out.reshape(Bb, H, 1, Dh)
        return out, {"S": St, "z": zt, "attn_type": "linear"}
    if not use_cache:
        return ops.linear_attention_scan(q1, q2, k, v, K, lambda_raw), None
    out, S_new, z_new = ops.linear_attn_scan(q1, q2, k, v, mode="reference", kernel_dim=K, lam=lam,
                                             return_final_state=True)
    new_cache = {"S": S_prev + S_new[:, :, :K], "z": z_prev + z_new[:, :, :K, None], "attn_type": "linear"}
    return out, new_cache
