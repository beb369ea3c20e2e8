"""Write the committed golden fixtures of the scan path (inputs + float64-oracle outputs).

The reference ships no numeric vectors for this path (its tests check shapes
and finiteness only), so the fixtures come from the float64 CPU oracle
(``oracle.ssd`` / ``oracle.kda``), which ``tests/test_oracle.py`` pins with
closed forms, brute-force matrices and invariants.  Inputs are drawn with the
seeded recipes of ``mamformer_amd.workloads`` (bf16 inputs are stored after
rounding, as float32).  Expected outputs are stored as float32.

Run:  python tests/golden/make_golden.py    (rewrites tests/golden/*.npz)
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from mamformer_amd import workloads as W  # noqa: E402
from oracle import kda, ssd  # noqa: E402


def f32(t):
    return t.detach().to(torch.float32).cpu().numpy() if torch.is_tensor(t) else np.asarray(t, np.float32)


def ssd1():
    inp = W.ssd_inputs(W.SSD1)
    x, dt, A, B, C, D = (f32(inp[k]) for k in ("x", "dt", "A", "B", "C", "D"))
    y, fin = ssd.ssd_via_reference(x, dt, A, B, C, D)
    np.savez_compressed(HERE / "ssd1.npz", x=x, dt=dt, A=A, B=B, C=C, D=D, y=y.astype(np.float32),
             final=fin.astype(np.float32))


# (name, b, L, H, N, G, dtype, h0, seed)
SSD_EDGE = [
    ("L1", 2, 1, 2, 64, 2, torch.bfloat16, True, 11),
    ("L7", 1, 7, 4, 128, 1, torch.bfloat16, False, 12),
    ("L33", 1, 33, 4, 128, 2, torch.bfloat16, True, 13),
    ("L64", 1, 64, 2, 64, 1, torch.float32, True, 14),
    ("L100", 2, 100, 8, 64, 4, torch.bfloat16, False, 15),
    ("L300", 1, 300, 2, 128, 2, torch.float32, True, 16),
]


def ssd_edge():
    out = {}
    for name, b, L, H, N, G, dtype, h0, seed in SSD_EDGE:
        cfg = W.SSDConfig(name, b, L, H, 64, N, G, 64, dtype, seed, init_state=h0)
        inp = W.ssd_inputs(cfg)
        arrs = {k: f32(inp[k]) for k in ("x", "dt", "A", "B", "C", "D")}
        s0 = f32(inp["initial_state"]) if h0 else None
        y, fin = ssd.ssd_via_reference(arrs["x"], arrs["dt"], arrs["A"], arrs["B"], arrs["C"], arrs["D"],
                                       initial_state=s0)
        for k, v in arrs.items():
            out[f"{name}/{k}"] = v
        if s0 is not None:
            out[f"{name}/initial_state"] = s0
        out[f"{name}/y"] = y.astype(np.float32)
        out[f"{name}/final"] = fin.astype(np.float32)
        out[f"{name}/bf16"] = np.array(dtype == torch.bfloat16)
    np.savez_compressed(HERE / "ssd_edge.npz", **out)


def decode_small():
    """Three consecutive decode steps, b=3 H=4 P=64 N=128 G=2, bf16, dt_bias + softplus."""
    g = torch.Generator().manual_seed(21)
    b, H, P, N, G, steps = 3, 4, 64, 128, 2, 3
    state = (torch.randn(b, H, P, N, generator=g) * 0.1)
    A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
    D = torch.randn(H, generator=g) * 0.1 + 1.0
    bias = torch.full((H,), -4.6)
    xs = torch.randn(steps, b, H, P, generator=g).to(torch.bfloat16)
    Bs = torch.randn(steps, b, G, N, generator=g).to(torch.bfloat16)
    Cs = torch.randn(steps, b, G, N, generator=g).to(torch.bfloat16)
    dts = torch.randn(steps, b, H, generator=g)
    out = dict(state0=f32(state), A=f32(A), D=f32(D), dt_bias=f32(bias), x=f32(xs), B=f32(Bs), C=f32(Cs),
               dt=f32(dts))
    s = f32(state).astype(np.float64)
    ys = []
    for i in range(steps):
        y, s = ssd.state_update_via_reference(s, out["x"][i], out["dt"][i], out["A"], out["B"][i], out["C"][i],
                                              out["D"], dt_bias=out["dt_bias"], dt_softplus=True)
        ys.append(y)
    out["y"] = np.stack(ys).astype(np.float32)
    out["state"] = s.astype(np.float32)
    np.savez_compressed(HERE / "decode_small.npz", **out)


def kda_small():
    """Gated KDA, B=1 H=2 S=100 dk=dv=128, bf16, nonzero initial state."""
    cfg = W.KDAConfig("kda_small", 1, 100, 2, 128, 128, 64, 0.8, torch.bfloat16, 31)
    inp = W.kda_inputs(cfg)
    arr = {k: f32(inp[k]) for k in ("q1", "q2", "k", "v", "g")}
    S0 = (torch.randn(1, 2, 128, 128, generator=torch.Generator().manual_seed(32)) * 0.1).numpy()
    o, ST = kda.gated_recurrent(arr["q1"], arr["q2"], arr["k"], arr["v"], arr["g"], cfg.lam, S0)
    np.savez_compressed(HERE / "kda_small.npz", **arr, S0=S0.astype(np.float32), lam=np.float32(cfg.lam),
             o=o.astype(np.float32), final=ST.astype(np.float32))


if __name__ == "__main__":
    ssd1()
    ssd_edge()
    decode_small()
    kda_small()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
