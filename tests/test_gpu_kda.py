"""GPU parity of the gated KDA linear-attention scan against the float64 oracle (oracle/kda.py)."""

from pathlib import Path

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from mamformer_amd import workloads as W
from oracle import kda as ref
from tests.gpu_helpers import check_per_head, check, dev, host, say

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
BF = torch.bfloat16


def run(inp, lam, s0=None, **kw):
    o, fin = mh.linear_attn_scan(dev(inp["q1"], BF), dev(inp["q2"], BF), dev(inp["k"], BF), dev(inp["v"], BF),
                                 g=dev(inp["g"]) if inp.get("g") is not None else None, lam=lam,
                                 initial_state=dev(s0) if s0 is not None else None, return_final_state=True, **kw)
    torch.cuda.synchronize()
    return o, fin


def test_kda_golden():
    z = np.load(GOLD / "kda_small.npz")
    say("kda golden B1 H2 S100")
    o, fin = run({k: z[k] for k in ("q1", "q2", "k", "v", "g")}, float(z["lam"]), z["S0"])
    check("o", o, z["o"], 1e-2)
    check("final", fin, z["final"], 1e-2)


@pytest.mark.parametrize("S,gate,s0", [(1, True, False), (63, True, True), (64, False, False),
                                       (65, True, False), (257, True, True)])
def test_kda_small_vs_recurrence(S, gate, s0):
    cfg = W.KDA5.scaled(batch=2, nheads=4, seqlen=S, seed=50 + S)
    inp = W.kda_inputs(cfg)
    if not gate:
        inp["g"] = None
    S0 = (torch.randn(2, 4, 128, 128, generator=torch.Generator().manual_seed(S)) * 0.1).numpy() if s0 else None
    say(f"kda S={S} gate={gate} s0={s0}")
    o, fin = run(inp, 0.8, S0)
    arr = {k: (None if v is None or not torch.is_tensor(v) else v.double().numpy()) for k, v in inp.items()}
    o_ref, f_ref = ref.gated_chunked(arr["q1"], arr["q2"], arr["k"], arr["v"], arr["g"], 0.8, S0, chunk_size=32)
    check("o", o, o_ref, 1e-2)
    check("final", fin, f_ref, 1e-2)


def test_kda_per_head_lambda_and_single_query():
    cfg = W.KDA5.scaled(batch=1, nheads=8, seqlen=130, seed=77)
    inp = W.kda_inputs(cfg)
    lam = torch.linspace(0.0, 0.99, 8)
    say("kda per-head lambda")
    o, _ = run(inp, lam.cuda())
    arr = {k: v.double().numpy() for k, v in inp.items() if torch.is_tensor(v)}
    o_ref, _ = ref.gated_recurrent(arr["q1"], arr["q2"], arr["k"], arr["v"], arr["g"], lam.double().numpy())
    check_per_head("o", o, o_ref, 1e-2)          # per head: lambda differs by head
    o1 = mh.linear_attn_scan(dev(inp["q1"], BF), None, dev(inp["k"], BF), dev(inp["v"], BF), g=dev(inp["g"]),
                             lam=0.5)
    o_ref1, _ = ref.gated_recurrent(arr["q1"], np.zeros_like(arr["q1"]), arr["k"], arr["v"], arr["g"], 0.5)
    check("o single query", o1, o_ref1, 1e-2)


def test_kda_extreme_decay_cuts_segments():
    cfg = W.KDA5.scaled(batch=1, nheads=2, seqlen=150, seed=88)
    inp = W.kda_inputs(cfg)
    g = inp["g"].clone()
    g[..., :8] = -30.0 * torch.rand(g[..., :8].shape, generator=torch.Generator().manual_seed(3))
    inp["g"] = g
    say("kda extreme decay")
    o, fin = run(inp, 0.8)
    arr = {k: v.double().numpy() for k, v in inp.items() if torch.is_tensor(v)}
    o_ref, f_ref = ref.gated_recurrent(arr["q1"], arr["q2"], arr["k"], arr["v"], arr["g"], 0.8)
    check("o", o, o_ref, 1e-2)
    check("final", fin, f_ref, 1e-2)


def test_kda5_full_size_properties():
    """Benchmark shape kda5 (B4 S8192 H32 K=V=128, bf16)."""
    inp = W.kda_inputs(W.KDA5, device="cuda")
    say("kda5 full: run")
    o, fin = mh.linear_attn_scan(inp["q1"], inp["q2"], inp["k"], inp["v"], g=inp["g"], lam=inp["lam"],
                                 return_final_state=True)
    o2, fin2 = mh.linear_attn_scan(inp["q1"], inp["q2"], inp["k"], inp["v"] * 2, g=inp["g"], lam=inp["lam"],
                                   return_final_state=True)
    torch.cuda.synchronize()
    say("kda5 full: linearity in v")
    assert torch.equal(o2, o * 2) and torch.equal(fin2, fin * 2)
    n = 256
    arr = {k: host(v[:, :4, :n]) for k, v in inp.items() if torch.is_tensor(v)}
    o_ref, _ = ref.gated_chunked(arr["q1"], arr["q2"], arr["k"], arr["v"], arr["g"], inp["lam"], chunk_size=64)
    check("kda5 o[:, :4, :256] vs oracle", o[:, :4, :n], o_ref, 1e-2)
    S = W.KDA5.seqlen
    oa, fa = mh.linear_attn_scan(*(inp[k][:, :, :S - n] for k in ("q1", "q2", "k", "v")), g=inp["g"][:, :, :S - n],
                                 lam=inp["lam"], return_final_state=True)
    tail = {k: host(v[:, :4, -n:]) for k, v in inp.items() if torch.is_tensor(v)}
    o_ref, f_ref = ref.gated_chunked(tail["q1"], tail["q2"], tail["k"], tail["v"], tail["g"], inp["lam"],
                                     host(fa[:, :4]), chunk_size=64)
    check("kda5 o[-256:] vs oracle", o[:, :4, -n:], o_ref, 1e-2)
    check("kda5 final vs oracle", fin[:, :4], f_ref, 1e-2)
    check("kda5 prefix consistency", oa, host(o[:, :, :S - n]), 1e-2)
