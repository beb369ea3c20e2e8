"""Seeded synthetic inputs for the five benchmark workloads of the scan path.

Every recipe draws its tensors from one ``torch.Generator`` seeded with the
workload's seed, in a fixed order (x, B, C, dt_raw, A_u, D, h0 for the SSD
workloads; q1, q2, k, v, g for KDA), so that the same (seed, shape) gives the
same tensors on every machine.  Drawn on the CPU by default; ``device`` may
name a GPU for full-size benchmark inputs (then the values differ from the
CPU draw but follow the same distributions).

Workloads (shapes of the reference's Mamba-2 / KDA-Diff layers):

====  ===========================================================================
ssd1  CPU plumbing: b1 L512 H8 P64 N64 G1 chunk 64, fp32; dt = clamp(softplus(N(0,1)-4.6), 1e-3, 0.1)
ssd2  1b-shape prefill: b2 L4096 H64 P64 N128 G1 chunk 256, bf16 x/B/C, fp32 dt = softplus(N(0,1)-4.6)
dec3  decode state update: B in {64, 256}, H64 P64 N128 G1, fp32 state ~N(0,0.1), dt_raw ~N(0,1), dt_bias -4.6
ssd4  128K prefill: b1 L131072 H128 P64 N128 G8 chunk 256, bf16, fp32 initial state ~N(0,0.1)
kda5  gated KDA: B4 S8192 H32 K=V=128 chunk 64, bf16 q/k/v ~N(0,1)/sqrt(128), g = logsigmoid(N(0,1))/16, lam 0.8
====  ===========================================================================

A = -exp(U(0, ln 16)) per head everywhere.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace
from typing import Optional

import torch
import torch.nn.functional as F

__all__ = ["SSDConfig", "DecodeConfig", "KDAConfig", "SSD1", "SSD2", "SSD4", "DEC3", "KDA5",
           "ssd_inputs", "decode_inputs", "kda_inputs"]


@dataclass(frozen=True)
class SSDConfig:
    name: str
    batch: int
    seqlen: int
    nheads: int
    headdim: int
    dstate: int
    ngroups: int
    chunk: int
    dtype: torch.dtype
    seed: int
    dt_clamp: Optional[tuple] = None     # clamp after softplus (ssd1)
    D_ones: bool = False                 # D = 1 (ssd1) else N(1, 0.1)
    init_state: bool = False             # nonzero initial state (ssd4)

    def scaled(self, **kw):
        return replace(self, **kw)


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    nheads: int
    headdim: int
    dstate: int
    ngroups: int
    dtype: torch.dtype
    seed: int

    def scaled(self, **kw):
        return replace(self, **kw)


@dataclass(frozen=True)
class KDAConfig:
    name: str
    batch: int
    seqlen: int
    nheads: int
    dk: int
    dv: int
    chunk: int
    lam: float
    dtype: torch.dtype
    seed: int

    def scaled(self, **kw):
        return replace(self, **kw)


SSD1 = SSDConfig("ssd1", 1, 512, 8, 64, 64, 1, 64, torch.float32, 0, dt_clamp=(1e-3, 0.1), D_ones=True)
SSD2 = SSDConfig("ssd2", 2, 4096, 64, 64, 128, 1, 256, torch.bfloat16, 1)
DEC3 = DecodeConfig("dec3", 64, 64, 64, 128, 1, torch.bfloat16, 2)
SSD4 = SSDConfig("ssd4", 1, 131072, 128, 64, 128, 8, 256, torch.bfloat16, 3, init_state=True)
KDA5 = KDAConfig("kda5", 4, 8192, 32, 128, 128, 64, 0.8, torch.bfloat16, 4)

DT_BIAS = -4.6


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, g, device):
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32)


def ssd_inputs(cfg: SSDConfig, device="cpu"):
    """Inputs of an SSD prefill workload.

    Returns a dict with x (b,L,H,P), B, C (b,L,G,N) in ``cfg.dtype``; dt (b,L,H)
    fp32 (already softplus'ed and clamped); A (H,) fp32; D (H,) fp32;
    initial_state (b,H,P,N) fp32 or None.
    """
    g = _gen(cfg.seed, device)
    b, L, H, P, N, G = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    x = _randn((b, L, H, P), g, device).to(cfg.dtype)
    B = _randn((b, L, G, N), g, device).to(cfg.dtype)
    C = _randn((b, L, G, N), g, device).to(cfg.dtype)
    dt_raw = _randn((b, L, H), g, device)
    A_u = torch.rand((H,), generator=g, device=device, dtype=torch.float32)
    D_n = _randn((H,), g, device)
    h0 = _randn((b, H, P, N), g, device) * 0.1 if cfg.init_state else None
    dt = F.softplus(dt_raw + DT_BIAS)
    if cfg.dt_clamp is not None:
        dt = dt.clamp(cfg.dt_clamp[0], cfg.dt_clamp[1])
    A = -torch.exp(A_u * math.log(16.0))
    D = torch.ones(H, device=device) if cfg.D_ones else 1.0 + 0.1 * D_n
    return dict(x=x, dt=dt.contiguous(), A=A, B=B, C=C, D=D, initial_state=h0)


def decode_inputs(cfg: DecodeConfig, device="cpu"):
    """Inputs of a decode (selective state update) workload.

    state (B,H,P,N) fp32 ~N(0, 0.1); x (B,H,P), B, C (B,G,N) in ``cfg.dtype``;
    dt (B,H) fp32 raw ~N(0,1); dt_bias (H,) = -4.6 (applied with softplus by
    the op); A (H,) fp32; D (H,) = 1.
    """
    g = _gen(cfg.seed, device)
    b, H, P, N, G = cfg.batch, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    x = _randn((b, H, P), g, device).to(cfg.dtype)
    B = _randn((b, G, N), g, device).to(cfg.dtype)
    C = _randn((b, G, N), g, device).to(cfg.dtype)
    dt = _randn((b, H), g, device)
    A_u = torch.rand((H,), generator=g, device=device, dtype=torch.float32)
    _ = _randn((H,), g, device)                   # D draw kept for a fixed order; D = 1
    state = _randn((b, H, P, N), g, device) * 0.1
    A = -torch.exp(A_u * math.log(16.0))
    return dict(state=state, x=x, dt=dt, A=A, B=B, C=C, D=torch.ones(H, device=device),
                dt_bias=torch.full((H,), DT_BIAS, device=device))


def kda_inputs(cfg: KDAConfig, device="cpu"):
    """Inputs of the gated KDA workload: q1, q2, k (B,H,S,K), v (B,H,S,V) in ``cfg.dtype``; g fp32."""
    gen = _gen(cfg.seed, device)
    b, H, S, K, V = cfg.batch, cfg.nheads, cfg.seqlen, cfg.dk, cfg.dv
    s = 1.0 / math.sqrt(K)
    q1 = (_randn((b, H, S, K), gen, device) * s).to(cfg.dtype)
    q2 = (_randn((b, H, S, K), gen, device) * s).to(cfg.dtype)
    k = (_randn((b, H, S, K), gen, device) * s).to(cfg.dtype)
    v = (_randn((b, H, S, V), gen, device) * (1.0 / math.sqrt(V))).to(cfg.dtype)
    g = F.logsigmoid(_randn((b, H, S, K), gen, device)) / 16.0
    return dict(q1=q1, q2=q2, k=k, v=v, g=g.contiguous(), lam=cfg.lam)
