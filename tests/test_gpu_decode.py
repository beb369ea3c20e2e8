"""GPU parity of the decode state update (selective_state_update / recurrent_step)."""

from pathlib import Path

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from mamformer_amd import workloads as W
from oracle import ssd as ref
from tests.gpu_helpers import check, dev, host, say

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def test_decode_golden_three_steps():
    z = np.load(GOLD / "decode_small.npz")
    state = dev(z["state0"]).contiguous()
    for i in range(z["x"].shape[0]):
        say(f"decode golden step {i}")
        y = mh.selective_state_update(state, dev(z["x"][i], torch.bfloat16), dev(z["dt"][i]), dev(z["A"]),
                                      dev(z["B"][i], torch.bfloat16), dev(z["C"][i], torch.bfloat16), dev(z["D"]),
                                      dt_bias=dev(z["dt_bias"]), dt_softplus=True)
        check(f"y[{i}]", y, z["y"][i], 1e-2)
    check("state", state, z["state"], 1e-4)


@pytest.mark.parametrize("N", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_all_dstates(N, dtype):
    g = torch.Generator().manual_seed(N)
    b, H, P, G = 5, 6, 64, 3
    s0 = torch.randn(b, H, P, N, generator=g) * 0.1
    x = torch.randn(b, H, P, generator=g).to(dtype)
    B = torch.randn(b, G, N, generator=g).to(dtype)
    C = torch.randn(b, G, N, generator=g).to(dtype)
    dt = torch.randn(b, H, generator=g)
    A = -torch.exp(torch.rand(H, generator=g) * 2.7)
    D = torch.randn(H, P, generator=g)
    say(f"decode N={N} {dtype}")
    out = torch.empty(b, H, P, N, device="cuda")
    y = mh.selective_state_update(dev(s0), dev(x, dtype), dev(dt), dev(A), dev(B, dtype), dev(C, dtype), dev(D),
                                  dt_softplus=True, dt_limit=(0.001, 2.0), out_state=out)
    y_ref, s_ref = ref.state_update_direct(s0.double().numpy(), x.double().numpy(), dt.numpy(), A.numpy(),
                                           B.double().numpy(), C.double().numpy(), D.numpy(), dt_softplus=True,
                                           dt_limit=(0.001, 2.0))
    check("y", y, y_ref, 1e-2 if dtype == torch.bfloat16 else 1e-4)
    check("state", out, s_ref, 1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_output_gate(dtype):
    """Fused z-gate on the one-token path: y * silu(z) (mamba2.py:337-338); the state is not gated."""
    g = torch.Generator().manual_seed(5)
    b, H, P, N = 3, 8, 64, 128
    s0 = torch.randn(b, H, P, N, generator=g) * 0.1
    x = torch.randn(b, H, P, generator=g).to(dtype)
    z = (torch.randn(b, H, P, generator=g) * 3).to(dtype)
    B = torch.randn(b, 1, N, generator=g).to(dtype)
    C = torch.randn(b, 1, N, generator=g).to(dtype)
    dt = torch.randn(b, H, generator=g)
    A = -torch.exp(torch.rand(H, generator=g) * 2.7)
    D = torch.randn(H, generator=g)
    say(f"decode gate {dtype}")
    out = torch.empty(b, H, P, N, device="cuda")
    y = mh.selective_state_update(dev(s0), dev(x, dtype), dev(dt), dev(A), dev(B, dtype), dev(C, dtype), dev(D),
                                  dt_softplus=True, out_state=out, z=dev(z, dtype))
    y_ref, s_ref = ref.state_update_direct(s0.double().numpy(), x.double().numpy(), dt.numpy(), A.numpy(),
                                           B.double().numpy(), C.double().numpy(), D.numpy(), dt_softplus=True)
    zr = z.double().numpy()
    check("gated y", y, y_ref * (zr / (1.0 + np.exp(-zr))), 1e-2 if dtype == torch.bfloat16 else 1e-4)
    check("state", out, s_ref, 1e-4)


@pytest.mark.parametrize("batch", [64, 256])
def test_decode_benchmark_shape(batch):
    inp = W.decode_inputs(W.DEC3.scaled(batch=batch))
    say(f"dec3 batch={batch}")
    st = dev(inp["state"]).contiguous()
    y = mh.selective_state_update(st, dev(inp["x"], torch.bfloat16), dev(inp["dt"]), dev(inp["A"]),
                                  dev(inp["B"], torch.bfloat16), dev(inp["C"], torch.bfloat16), dev(inp["D"]),
                                  dt_bias=dev(inp["dt_bias"]), dt_softplus=True)
    y_ref, s_ref = ref.state_update_via_reference(inp["state"].double().numpy(), inp["x"].double().numpy(),
                                                  inp["dt"].numpy(), inp["A"].numpy(),
                                                  inp["B"].double().numpy(), inp["C"].double().numpy(),
                                                  inp["D"].numpy(), dt_bias=inp["dt_bias"].numpy(),
                                                  dt_softplus=True)
    check("y", y, y_ref, 1e-2)
    check("state", st, s_ref, 1e-4)


def test_prefill_then_decode_matches_longer_prefill():
    """State carry across ops: GPU prefill of L-3 tokens, 3 GPU decode steps == GPU prefill of L tokens."""
    cfg = W.SSDConfig("carry", 2, 300, 8, 64, 128, 2, 256, torch.bfloat16, 41, init_state=True)
    inp = W.ssd_inputs(cfg)
    d = {k: dev(v, torch.bfloat16 if k in ("x", "B", "C") else torch.float32) for k, v in inp.items()}
    say("prefill+decode carry")
    y_full, f_full = mh.selective_scan(d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], return_final_state=True,
                                       initial_state=d["initial_state"])
    m = 3
    y_pre, st = mh.selective_scan(d["x"][:, :-m], d["dt"][:, :-m], d["A"], d["B"][:, :-m], d["C"][:, :-m], d["D"],
                                  return_final_state=True, initial_state=d["initial_state"])
    ys = []
    for t in range(cfg.seqlen - m, cfg.seqlen):
        ys.append(mh.selective_state_update(st, d["x"][:, t], d["dt"][:, t], d["A"], d["B"][:, t], d["C"][:, t],
                                            d["D"], dt_softplus=False))
    check("decoded y", torch.stack(ys, 1), host(y_full[:, -m:]), 1e-2)
    check("state", st, host(f_full), 1e-2)


def test_recurrent_step_wrapper_returns_new_state():
    g = torch.Generator().manual_seed(5)
    b, H, P, N = 2, 4, 64, 64
    x = torch.randn(b, 3, H * P, generator=g)
    dt = torch.rand(b, 3, H, generator=g) * 0.1
    B = torch.randn(b, 3, N, generator=g)
    C = torch.randn(b, 3, N, generator=g)
    h = torch.randn(b, H * P, N, generator=g)
    A = -torch.exp(torch.rand(H, generator=g))
    D = torch.ones(H)
    hd = dev(h)
    y, hn = mh.recurrent_step(dev(x), dev(dt), dev(B), dev(C), hd, dev(A), dev(D))
    assert y.shape == (b, 1, H * P) and hn.shape == (b, H * P, N)
    assert torch.equal(hd, dev(h)), "h_prev must not be modified"
    y_ref, h_ref = ref.state_update_direct(h.double().numpy().reshape(b, H, P, N), x[:, -1].double().numpy()
                                           .reshape(b, H, P), dt[:, -1].numpy(), A.numpy(), B[:, -1].numpy(),
                                           C[:, -1].numpy(), D.numpy(), dt_softplus=False)
    check("y", y.view(b, H, P), y_ref, 1e-4)
    check("h", hn.view(b, H, P, N), h_ref, 1e-4)


@pytest.mark.parametrize("b,d_inner,N,dtype,h0", [
    (2, 64, 16, torch.float32, False),      # the reference fixture's sizes (tests/test_mamba2.py:22-30)
    (2, 32, 8, torch.float32, True),        # its per-seqlen case (tests/test_mamba2.py:74-80)
    (3, 256, 32, torch.bfloat16, True),     # the debug preset's d_state
    (2, 4096, 128, torch.bfloat16, True),
])
def test_reference_form_step_vs_oracle(b, d_inner, N, dtype, h0):
    """recurrent_step_reference: the reference's own decode parameterisation (A_log per state, dt per channel,
    mamba2.py:431-458) against the oracle's restatement, five steps chained through the returned state."""
    g = torch.Generator().manual_seed(d_inner + N)
    A_log = torch.log(torch.linspace(0.5, 8.0, N))
    D = torch.ones(d_inner) + 0.1 * torch.randn(d_inner, generator=g)
    h = torch.randn(b, d_inner, N, generator=g) * 0.1 if h0 else None
    hr = None if h is None else h.double().numpy()
    hd = dev(h)
    say(f"reference-form step b={b} d_inner={d_inner} N={N} {dtype} h0={h0}")
    for step in range(5):
        x = torch.randn(b, 2, d_inner, generator=g).to(dtype)
        dt = torch.nn.functional.softplus(torch.randn(b, 2, d_inner, generator=g))
        B = torch.randn(b, 2, N, generator=g).to(dtype)
        C = torch.randn(b, 2, N, generator=g).to(dtype)
        y, hd_new = mh.recurrent_step_reference(dev(x, dtype), dev(dt), dev(B, dtype), dev(C, dtype), hd,
                                                dev(A_log), dev(D))
        torch.cuda.synchronize()
        y_ref, hr = ref.ref_recurrent_step(x.double().numpy(), dt.double().numpy(), B.double().numpy(),
                                           C.double().numpy(), hr, A_log.double().numpy(), D.double().numpy())
        assert y.shape == (b, 1, d_inner) and y.dtype == dtype and hd_new.shape == (b, d_inner, N)
        check(f"y[{step}]", y, y_ref, 1e-2 if dtype == torch.bfloat16 else 1e-4)
        check(f"h[{step}]", hd_new, hr, 1e-4)
        hd = hd_new
