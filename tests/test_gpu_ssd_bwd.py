"""GPU parity of the SSD prefill backward (mh_ssd_chunk_scan_bwd) against the float64 oracle
(oracle/ssd_bwd.py, the adjoint recurrence pinned against autograd of the reference scan).

Tolerance: global relative L2 <= 1e-2 for bf16 I/O and <= 1e-4 for fp32 I/O on every gradient (dx, ddt,
dA, dB, dC, dD, d_dt_bias, d_initial_state).  Every sum over workgroups (dB, dC per head block; dA, dD,
d_dt_bias per segment) is taken in a fixed order, so two calls agree bit for bit.  Small shapes and edge
lengths (1, 7, 64, 65, partial last segments) are compared with the oracle directly; the full benchmark
shape is checked through linearity in (dy, d_final) and a leading-slice oracle check (dy = 0 after T0, no final-state gradient:
every gradient past T0 is zero and the rest equals the truncated problem's).
"""

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from oracle import ssd as ossd
from oracle import ssd_bwd as obwd
from tests.gpu_helpers import TOL, check, dev, host, say

pytestmark = pytest.mark.gpu


def make(rng, b, L, H, N, G, dtype, h0, dfin, dmode, P=64):
    def rnd(*shape, scale=1.0):
        a = scale * rng.standard_normal(shape)
        if dtype == torch.bfloat16:     # exact bf16 values, so the oracle sees what the kernel sees
            a = torch.tensor(a, dtype=torch.float32).to(torch.bfloat16).to(torch.float64).numpy()
        return a
    d = dict(x=rnd(b, L, H, P), B=rnd(b, L, G, N), C=rnd(b, L, G, N), dy=rnd(b, L, H, P),
             dt=rng.standard_normal((b, L, H)) - 1.0, A=-np.exp(rng.uniform(0, np.log(16), H)),
             bias=0.3 * rng.standard_normal(H))
    d["D"] = None if dmode is None else (1 + 0.1 * rng.standard_normal(H) if dmode == "head"
                                         else 1 + 0.1 * rng.standard_normal(H * P))
    d["h0"] = 0.1 * rng.standard_normal((b, H, P, N)) if h0 else None
    d["dfin"] = 0.1 * rng.standard_normal((b, H, P, N)) if dfin else None
    return d


def run_bwd(d, dtype, softplus, limit):
    g = mh.selective_scan_bwd(
        dev(d["dy"], dtype), dev(d["x"], dtype), dev(d["dt"]), dev(d["A"]), dev(d["B"], dtype), dev(d["C"], dtype),
        dev(d["D"]), d_final_state=dev(d["dfin"]), initial_state=dev(d["h0"]),
        dt_bias=dev(d["bias"]) if softplus else None, dt_softplus=softplus, dt_limit=limit)
    torch.cuda.synchronize()
    return g


def oracle(d, softplus, limit):
    return obwd.ssd_backward(d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["dy"], d_final=d["dfin"],
                             initial_state=d["h0"], dt_bias=d["bias"] if softplus else None,
                             dt_softplus=softplus, dt_limit=limit)


def compare(g, r, dtype, tag):
    """Every gradient is reported before the first failure is raised."""
    tol = TOL[dtype]
    pairs = [("dx", "dx"), ("ddt", "ddt"), ("dA", "dA"), ("dB", "dB"), ("dC", "dC"), ("d_initial_state", "dh0")]
    if "dD" in r:
        pairs.append(("dD", "dD"))
    if "d_dt_bias" in g:
        pairs.append(("d_dt_bias", "ddt_bias"))
    errs = []
    for k, rk in pairs:
        try:
            check(f"{tag} {k}", g[k], r[rk], tol)
        except AssertionError as e:
            errs.append(str(e))
    assert not errs, "; ".join(errs)


CASES = [
    # (b, L, H, N, G, dtype, h0, dfin, softplus, limit, D, seed)
    (1, 200, 8, 128, 1, torch.bfloat16, True, True, True, None, "head", 1),
    (2, 130, 4, 64, 2, torch.bfloat16, False, True, False, None, "channel", 2),
    (1, 150, 4, 128, 2, torch.float32, True, True, True, (0.05, 0.4), "head", 3),
    (2, 64, 2, 64, 1, torch.float32, False, False, True, None, None, 4),
    (1, 1, 2, 128, 1, torch.bfloat16, True, True, True, None, "head", 5),
    (1, 7, 2, 64, 1, torch.float32, True, True, False, None, "channel", 6),
    (1, 65, 16, 128, 2, torch.bfloat16, False, True, True, None, "head", 7),
    (1, 320, 16, 64, 4, torch.float32, True, False, True, None, "head", 8),
    # dstate outside the 64 / 128 tiles (composed by the C ABI: zero-padded, or two 128-column halves)
    (2, 32, 4, 16, 1, torch.float32, True, True, True, None, "head", 9),       # the reference fixture's sizes
    (1, 150, 4, 32, 2, torch.bfloat16, True, True, True, None, "channel", 10),
    (1, 99, 2, 8, 1, torch.float32, False, True, False, None, "head", 11),
    (1, 140, 4, 256, 1, torch.bfloat16, True, True, True, None, "head", 12),  # halves read in place
    (1, 70, 4, 256, 2, torch.float32, True, True, True, (0.05, 0.4), "channel", 13),
    (1, 66, 2, 200, 1, torch.float32, True, False, True, None, None, 14),     # second half padded
    (1, 130, 2, 96, 2, torch.float32, False, True, True, None, "head", 15),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"b{c[0]}L{c[1]}H{c[2]}N{c[3]}G{c[4]}-{str(c[5])[6:]}")
def test_bwd_vs_oracle(case):
    b, L, H, N, G, dtype, h0, dfin, sp, lim, dmode, seed = case
    say(f"bwd b{b} L{L} H{H} N{N} G{G} {dtype} h0={h0} dfin={dfin} softplus={sp} limit={lim} D={dmode}")
    d = make(np.random.default_rng(seed), b, L, H, N, G, dtype, h0, dfin, dmode)
    if not sp:
        d["dt"] = ossd.softplus(d["dt"])     # without the prologue, dt must already be a positive step
    compare(run_bwd(d, dtype, sp, lim), oracle(d, sp, lim), dtype, f"L{L}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_autograd_through_selective_scan(dtype):
    """loss.backward() through selective_scan (3-D reference layout, z-gate in torch) equals the explicit op,
    and dz matches the oracle's y: dz = dy * y_ungated * silu'(z)."""
    rng = np.random.default_rng(11)
    b, L, H, N, G = 1, 150, 4, 128, 1
    d = make(rng, b, L, H, N, G, dtype, True, True, "head")
    z = rng.standard_normal((b, L, H, 64))
    if dtype == torch.bfloat16:
        z = torch.tensor(z, dtype=torch.float32).to(torch.bfloat16).to(torch.float64).numpy()
    say(f"autograd {dtype}")
    leaf = lambda a, t=torch.float32: dev(a, t).requires_grad_(True)
    x, dt, A = leaf(d["x"].reshape(b, L, H * 64), dtype), leaf(d["dt"]), leaf(d["A"])
    B, C, D = leaf(d["B"][:, :, 0], dtype), leaf(d["C"][:, :, 0], dtype), leaf(d["D"])
    h0, bias = leaf(d["h0"].reshape(b, H * 64, N)), leaf(d["bias"])
    zz = leaf(z.reshape(b, L, H * 64), dtype)
    y, fin = mh.selective_scan(x, dt, A, B, C, D, return_final_state=True, initial_state=h0, dt_bias=bias,
                               dt_softplus=True, z=zz)
    dy = dev(d["dy"].reshape(b, L, H * 64), dtype)
    loss = (y.float() * dy.float()).sum() + (fin * dev(d["dfin"].reshape(b, H * 64, N))).sum()
    loss.backward()
    torch.cuda.synchronize()
    # the ungated output and the gradient reaching it
    y0, _ = ossd.ssd_direct(d["x"], ossd.process_dt(d["dt"], d["bias"], True), d["A"], d["B"], d["C"], d["D"],
                            initial_state=d["h0"])
    sz = 1 / (1 + np.exp(-z))
    dz_ref = d["dy"] * y0 * (sz * (1 + z * (1 - sz)))
    dy_in = d["dy"] * z * sz
    if dtype == torch.bfloat16:
        dy_in = host(dev(dy_in, torch.bfloat16))       # the kernel receives the bf16-rounded gated gradient
    r = obwd.ssd_backward(d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], dy_in, d_final=d["dfin"],
                          initial_state=d["h0"], dt_bias=d["bias"], dt_softplus=True)
    tol = TOL[dtype]
    check("autograd dx", x.grad.reshape(b, L, H, 64), r["dx"], tol)
    check("autograd ddt", dt.grad, r["ddt"], tol)
    check("autograd dA", A.grad, r["dA"], tol)
    check("autograd dB", B.grad, r["dB"][:, :, 0], tol)
    check("autograd dC", C.grad, r["dC"][:, :, 0], tol)
    check("autograd dD", D.grad, r["dD"], tol)
    check("autograd dh0", h0.grad.reshape(b, H, 64, N), r["dh0"], tol)
    check("autograd dbias", bias.grad, r["ddt_bias"], tol)
    check("autograd dz", zz.grad.reshape(b, L, H, 64), dz_ref, tol)


def test_bwd_empty_sequence():
    say("bwd L=0")
    b, H, N = 2, 4, 64
    rng = np.random.default_rng(3)
    dfin = rng.standard_normal((b, H, 64, N))
    x = torch.zeros((b, 0, H, 64), device="cuda", dtype=torch.bfloat16)
    B = torch.zeros((b, 0, 1, N), device="cuda", dtype=torch.bfloat16)
    g = mh.selective_scan_bwd(x, x, torch.zeros((b, 0, H), device="cuda"), dev(-np.ones(H)), B, B,
                              dev(np.ones(H)), d_final_state=dev(dfin), dt_bias=dev(np.zeros(H)), dt_softplus=True)
    torch.cuda.synchronize()
    assert g["dx"].shape == x.shape and g["dB"].shape == B.shape
    assert float(g["dA"].abs().max()) == 0.0 and float(g["dD"].abs().max()) == 0.0
    assert float(g["d_dt_bias"].abs().max()) == 0.0
    assert np.array_equal(host(g["d_initial_state"]), dfin.astype(np.float32).astype(np.float64))


@pytest.mark.parametrize("dmode,dtype", [("head", torch.bfloat16), ("channel", torch.bfloat16),
                                         ("channel", torch.float32)])
def test_bwd_is_deterministic(dmode, dtype):
    """Two calls on the same inputs agree bit for bit on every gradient: dA, dD (per head or per channel) and
    d_dt_bias are per-segment partials summed in a fixed order, dB / dC per-head-block partials likewise."""
    d = make(np.random.default_rng(17), 2, 700, 16, 128, 2, dtype, True, True, dmode)
    say(f"bwd determinism D={dmode} {dtype}")
    g1 = run_bwd(d, dtype, True, None)
    g2 = run_bwd(d, dtype, True, None)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), f"{k} differs between two identical calls"


@pytest.mark.parametrize("N", [32, 256])
def test_bwd_empty_sequence_composed(N):
    """L = 0 through the composed paths: d_initial_state = d_final_state column for column, zero dA / dD."""
    say(f"bwd L=0 N={N}")
    b, H = 1, 2
    dfin = np.random.default_rng(N).standard_normal((b, H, 64, N))
    x = torch.zeros((b, 0, H, 64), device="cuda", dtype=torch.float32)
    B = torch.zeros((b, 0, 1, N), device="cuda", dtype=torch.float32)
    g = mh.selective_scan_bwd(x, x, torch.zeros((b, 0, H), device="cuda"), dev(-np.ones(H)), B, B,
                              dev(np.ones(H)), d_final_state=dev(dfin), dt_bias=dev(np.zeros(H)), dt_softplus=True)
    torch.cuda.synchronize()
    assert float(g["dA"].abs().max()) == 0.0 and float(g["dD"].abs().max()) == 0.0
    assert float(g["d_dt_bias"].abs().max()) == 0.0
    assert np.array_equal(host(g["d_initial_state"]), dfin.astype(np.float32).astype(np.float64))


def test_bwd_full_shape_linearity_and_leading_slice():
    """ssd2 shape (b2 L4096 H64 P64 N128 G1, bf16): doubling dy and d_final doubles every gradient bit for bit
    (every sum is taken in a fixed order);
    with dy = 0 from token T0 on and no final-state gradient, gradients past T0 vanish and the first T0 tokens
    match the oracle of the truncated problem."""
    rng = np.random.default_rng(21)
    b, L, H, N, G, T0 = 2, 4096, 64, 128, 1, 192
    dtype = torch.bfloat16
    say(f"bwd full shape b{b} L{L} H{H} N{N}")
    x = dev(rng.standard_normal((b, L, H, 64)), dtype)
    B = dev(rng.standard_normal((b, L, G, N)), dtype)
    C = dev(rng.standard_normal((b, L, G, N)), dtype)
    dt = dev(rng.standard_normal((b, L, H)) - 1.0)
    A = dev(-np.exp(rng.uniform(0, np.log(16), H)))
    D = dev(1 + 0.1 * rng.standard_normal(H))
    bias = dev(0.3 * rng.standard_normal(H))
    dy = dev(rng.standard_normal((b, L, H, 64)), dtype)
    dfin = dev(0.1 * rng.standard_normal((b, H, 64, N)))
    kw = dict(dt_bias=bias, dt_softplus=True)
    g1 = mh.selective_scan_bwd(dy, x, dt, A, B, C, D, d_final_state=dfin, **kw)
    g2 = mh.selective_scan_bwd(dy * 2, x, dt, A, B, C, D, d_final_state=dfin * 2, **kw)
    torch.cuda.synchronize()
    for k in ("dx", "ddt", "d_initial_state", "dA", "dD", "d_dt_bias", "dB", "dC"):
        assert torch.equal(g1[k] * 2, g2[k]), f"linearity {k}"
    say("linearity ok")
    dyz = dy.clone()
    dyz[:, T0:] = 0
    g = mh.selective_scan_bwd(dyz, x, dt, A, B, C, D, **kw)
    torch.cuda.synchronize()
    for k in ("dx", "ddt", "dB", "dC"):
        assert float(g[k][:, T0:].abs().max()) == 0.0, f"{k} past T0"
    r = obwd.ssd_backward(host(x[:, :T0]), host(dt[:, :T0]), host(A), host(B[:, :T0]), host(C[:, :T0]), host(D),
                          host(dy[:, :T0]), dt_bias=host(bias), dt_softplus=True)
    tol = TOL[dtype]
    check("slice dx", g["dx"][:, :T0], r["dx"], tol)
    check("slice ddt", g["ddt"][:, :T0], r["ddt"], tol)
    check("slice dB", g["dB"][:, :T0], r["dB"], tol)
    check("slice dC", g["dC"][:, :T0], r["dC"], tol)
    check("slice dA", g["dA"], r["dA"], tol)
    check("slice dD", g["dD"], r["dD"], tol)
    check("slice dh0", g["d_initial_state"], r["dh0"], tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_output_gate_kernels_vs_float64(dtype):
    """The training path's fused gate (mh_silu_gate_fwd / mh_silu_gate_bwd) against float64 torch: out = y silu(z),
    dy = g silu(z), dz = g y silu'(z); z a strided view (a slice of a wider projection), and a broadcast gradient
    (the gradient of a sum) with zero strides."""
    from mamformer_amd.ops import _GateFn
    g0 = torch.Generator().manual_seed(12)
    b, L, H, P = 2, 37, 3, 64
    y = torch.randn(b, L, H, P, generator=g0).to(dtype)
    zw = (torch.randn(b, L, H, 2 * P, generator=g0) * 3).to(dtype)
    gr = torch.randn(b, L, H, P, generator=g0).to(dtype)
    say(f"output gate kernels {dtype}")
    yd = y.cuda().requires_grad_()
    zd = zw.cuda()[..., :P].detach().requires_grad_()
    out = _GateFn.apply(yd, zd)
    out.backward(gr.cuda())
    torch.cuda.synchronize()
    y64, z64, g64 = y.double(), zw[..., :P].double(), gr.double()
    s = torch.sigmoid(z64)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    check("out", out, (y64 * z64 * s).numpy(), tol)
    check("dy", yd.grad, (g64 * z64 * s).numpy(), tol)
    check("dz", zd.grad, (g64 * y64 * s * (1 + z64 * (1 - s))).numpy(), tol)
    yd.grad = None
    zd.grad = None
    _GateFn.apply(yd, zd).float().sum().backward()
    torch.cuda.synchronize()
    check("dz (broadcast gradient)", zd.grad, (y64 * s * (1 + z64 * (1 - s))).numpy(), tol)
