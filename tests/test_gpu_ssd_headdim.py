"""GPU parity of the SSD prefill at head sizes other than 64 against the float64 oracle.

The kernels run heads of 64 channels; ``selective_scan`` and ``selective_scan_bwd`` run a head of 64 k channels
as k heads of 64 that share its dt, A, dt_bias and B / C group, and zero-pad other sizes to the next multiple
of 64 first (``ops._Heads64``).  The oracle (oracle/ssd.py, oracle/ssd_bwd.py) takes any head size directly,
so these tests check the split, the padding and the maps back (outputs, final state, h_states rescaled over the
real channels, gradients of the shared per-head values summed) at P = 32, 96, 128, 192.

Tolerance as for every SSD test: relative L2 <= 1e-2 for bf16 I/O, <= 1e-4 for fp32 I/O.
"""

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from oracle import ssd as ossd
from tests.gpu_helpers import TOL, check, dev, host, say
from tests.test_gpu_ssd_bwd import compare, make, oracle, run_bwd

pytestmark = pytest.mark.gpu

BF, F32 = torch.bfloat16, torch.float32

FWD = [
    # (b, L, H, P, N, G, dtype, h0, D mode, 3-D layout, seed)
    (1, 150, 4, 128, 128, 2, BF, True, "channel", True, 11),
    (2, 100, 4, 32, 64, 1, F32, True, "head", False, 12),
    (1, 130, 2, 96, 128, 1, BF, False, "channel", False, 13),
    (1, 70, 3, 192, 64, 1, F32, True, None, True, 14),
]


@pytest.mark.parametrize("b,L,H,P,N,G,dtype,h0,dmode,three_d,seed", FWD)
def test_forward_head_sizes(b, L, H, P, N, G, dtype, h0, dmode, three_d, seed):
    rng = np.random.default_rng(seed)
    d = make(rng, b, L, H, N, G, dtype, h0, False, dmode, P=P)
    say(f"ssd head size P={P}: b={b} L={L} H={H} N={N} G={G} {dtype} h0={h0} D={dmode} 3-D={three_d}")
    x = dev(d["x"], dtype)
    s0 = dev(d["h0"])
    if three_d:
        x = x.reshape(b, L, H * P)
        s0 = None if s0 is None else s0.reshape(b, H * P, N)
    y, fin = mh.selective_scan(x, dev(d["dt"]), dev(d["A"]), dev(d["B"], dtype), dev(d["C"], dtype), dev(d["D"]),
                               return_final_state=True, initial_state=s0, dt_bias=dev(d["bias"]), dt_softplus=True)
    torch.cuda.synchronize()
    assert y.shape == x.shape and fin.shape == ((b, H * P, N) if three_d else (b, H, P, N))
    dtp = ossd.process_dt(d["dt"], dt_bias=d["bias"], dt_softplus=True)
    D = None if d["D"] is None else (d["D"] if dmode == "head" else d["D"].reshape(H, P))
    yr, fr = ossd.ssd_via_reference(d["x"], dtp, d["A"], d["B"], d["C"], D, initial_state=d["h0"])
    check(f"y P={P}", host(y).reshape(b, L, H, P), yr, TOL[dtype])
    check(f"final state P={P}", host(fin).reshape(b, H, P, N), fr, TOL[dtype])


@pytest.mark.parametrize("P,dtype,h0", [(128, BF, False), (32, F32, True), (96, F32, False)])
def test_h_states_head_sizes(P, dtype, h0):
    """h_states is the mean over every real channel: the padded channels hold zero state and the mean is
    rescaled from the padded count to the real one."""
    b, L, H, N, G = 1, 140, 4, 128, 1
    rng = np.random.default_rng(20 + P)
    d = make(rng, b, L, H, N, G, dtype, h0, False, None, P=P)
    say(f"h_states head size P={P} {dtype} h0={h0}")
    y, hs = mh.selective_scan(dev(d["x"], dtype), dev(d["dt"]), dev(d["A"]), dev(d["B"], dtype),
                              dev(d["C"], dtype), None, return_h_states=True, initial_state=dev(d["h0"]),
                              dt_bias=dev(d["bias"]), dt_softplus=True)
    torch.cuda.synchronize()
    dtp = ossd.process_dt(d["dt"], dt_bias=d["bias"], dt_softplus=True)
    r = ossd.ssd_h_states(d["x"], dtp, d["A"], d["B"], initial_state=d["h0"])
    check(f"h_states P={P}", hs, r, TOL[dtype])


BWD = [
    # (b, L, H, P, N, G, dtype, h0, dfin, softplus, D mode, seed)
    (1, 130, 4, 128, 128, 2, BF, True, True, True, "head", 31),
    (2, 70, 2, 32, 64, 1, F32, True, True, True, "channel", 32),
    (1, 100, 3, 96, 128, 1, F32, False, True, False, "head", 33),
]


@pytest.mark.parametrize("b,L,H,P,N,G,dtype,h0,dfin,softplus,dmode,seed", BWD)
def test_backward_head_sizes(b, L, H, P, N, G, dtype, h0, dfin, softplus, dmode, seed):
    """selective_scan_bwd at other head sizes: dx and d_initial_state mapped back (padding dropped), ddt, dA,
    d_dt_bias and a per-head dD summed over each head's 64-channel pieces."""
    rng = np.random.default_rng(seed)
    d = make(rng, b, L, H, N, G, dtype, h0, dfin, dmode, P=P)
    if not softplus:
        d["dt"] = ossd.softplus(d["dt"])     # without the prologue, dt must already be a positive step
    say(f"ssd backward head size P={P}: b={b} L={L} H={H} N={N} G={G} {dtype} D={dmode} softplus={softplus}")
    g = run_bwd(d, dtype, softplus, None)
    compare(g, oracle(d, softplus, None), dtype, f"P={P}")


def test_autograd_head_size_matches_explicit_backward():
    """Autograd through selective_scan at P = 96 (split and padded) gives the explicit backward's gradients."""
    b, L, H, P, N, G = 1, 90, 2, 96, 64, 1
    rng = np.random.default_rng(41)
    d = make(rng, b, L, H, N, G, F32, True, True, "channel", P=P)
    say("ssd autograd head size P=96")
    leaves = {k: dev(d[k]).requires_grad_() for k in ("x", "dt", "A", "B", "C", "D", "h0", "bias")}
    y, fin = mh.selective_scan(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], leaves["D"],
                               return_final_state=True, initial_state=leaves["h0"], dt_bias=leaves["bias"],
                               dt_softplus=True)
    loss = (y * dev(d["dy"])).sum() + (fin * dev(d["dfin"])).sum()
    grads = torch.autograd.grad(loss, [leaves[k] for k in ("x", "dt", "A", "B", "C", "D", "h0", "bias")])
    torch.cuda.synchronize()
    g = run_bwd(d, F32, True, None)
    for name, got, key in zip(("dx", "ddt", "dA", "dB", "dC", "dD", "dh0", "d_dt_bias"), grads,
                              ("dx", "ddt", "dA", "dB", "dC", "dD", "d_initial_state", "d_dt_bias")):
        check(f"autograd {name}", got, host(g[key]), 1e-5)


@pytest.mark.parametrize("P,dtype", [(96, BF), (128, F32)])
def test_gate_head_sizes(P, dtype):
    """The z-gate y * silu(z) at other head sizes (z split and padded like x; a padded channel's gate is silu(0) = 0
    on a zero output)."""
    b, L, H, N, G = 1, 120, 2, 64, 1
    rng = np.random.default_rng(50 + P)
    d = make(rng, b, L, H, N, G, dtype, False, False, "head", P=P)
    z = rng.standard_normal((b, L, H * P))
    if dtype == BF:
        z = torch.tensor(z, dtype=torch.float32).to(torch.bfloat16).to(torch.float64).numpy()
    say(f"ssd gate head size P={P} {dtype}")
    y = mh.selective_scan(dev(d["x"], dtype).reshape(b, L, H * P), dev(d["dt"]), dev(d["A"]), dev(d["B"], dtype),
                          dev(d["C"], dtype), dev(d["D"]), dt_bias=dev(d["bias"]), dt_softplus=True, z=dev(z, dtype))
    torch.cuda.synchronize()
    dtp = ossd.process_dt(d["dt"], dt_bias=d["bias"], dt_softplus=True)
    yr, _ = ossd.ssd_via_reference(d["x"], dtp, d["A"], d["B"], d["C"], d["D"])
    zr = z.reshape(b, L, H, P)
    check(f"gated y P={P}", host(y).reshape(b, L, H, P), yr * zr / (1 + np.exp(-zr)), TOL[dtype])


def test_empty_sequence_head_size():
    """L = 0 at P = 96: an empty output and the initial state back as the final state."""
    b, H, P, N = 2, 3, 96, 64
    x = torch.zeros(b, 0, H * P, device="cuda")
    dt = torch.zeros(b, 0, H, device="cuda")
    B = torch.zeros(b, 0, N, device="cuda")
    h0 = torch.randn(b, H * P, N, device="cuda")
    say("ssd empty sequence head size P=96")
    y, fin = mh.selective_scan(x, dt, -torch.ones(H, device="cuda"), B, B, None, return_final_state=True,
                               initial_state=h0)
    torch.cuda.synchronize()
    assert y.shape == (b, 0, H * P) and fin.shape == (b, H * P, N)
    assert torch.equal(fin, h0)

