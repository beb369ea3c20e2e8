"""GPU parity of the layer-level pieces around the scans against the float64 oracle.

* ``causal_conv1d`` (HIP) vs ``oracle.ssd.ref_causal_conv1d`` (mamba2.py:370-405), with and without the
  cached raw rows, bias and fused SiLU;
* ``selective_scan(return_h_states=True)`` vs ``oracle.ssd.ssd_h_states`` (mamba2.py:114-116), and its
  gradients under autograd vs autograd of the float64 recurrence;
* ``Mamba2Layer`` (A3 dispatch and cache, mamba2.py:249-364) vs the same layer composed in float64 from the
  oracle pieces, and prefill + one incremental step vs one longer prefill;
* ``kda_linear_attention`` (A13 state semantics, kda_diff.py:286-338) vs the reference-mode KDA oracle.
Tolerances: relative L2 <= 1e-4 for fp32 I/O, <= 1e-2 for bf16 I/O.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import mamformer_amd as mh
from mamformer_amd import ops
from mamformer_amd.layers import Mamba2Layer, kda_linear_attention
from oracle import kda as okda
from oracle import ssd as ref
from tests.gpu_helpers import TOL, check, dev, host, say

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------- conv1d

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L,D,K,cs_len", [(1, 8, 4, 0), (5, 64, 4, 3), (70, 256, 4, 2), (1000, 512, 3, 0),
                                          (33, 4096, 2, 1)])
def test_conv1d_vs_oracle(dtype, L, D, K, cs_len):
    g = torch.Generator().manual_seed(L * 7 + D)
    b = 2
    x = torch.randn(b, L, D, generator=g)
    w = torch.randn(D, 1, K, generator=g) * 0.5
    bias = torch.randn(D, generator=g)
    cs = torch.randn(b, cs_len, D, generator=g) if cs_len else None
    xd, csd = dev(x, dtype), (dev(cs, dtype) if cs is not None else None)
    for silu in (False, True):
        say(f"conv1d L={L} D={D} K={K} cs={cs_len} silu={silu} {dtype}")
        y = mh.causal_conv1d(xd, dev(w), dev(bias), csd, silu=silu)
        torch.cuda.synchronize()
        r = ref.ref_causal_conv1d(host(xd), w.numpy(), bias.numpy(), host(csd) if csd is not None else None)
        if silu:
            r = r / (1.0 + np.exp(-r))
        check("conv1d y", y, r, TOL[dtype])


# ----------------------------------------------------------------- h_states

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("G,N,h0", [(1, 64, False), (2, 128, True)])
def test_h_states_vs_oracle(dtype, G, N, h0):
    g = torch.Generator().manual_seed(5 + N)
    b, L, H, P = 2, 150, 4, 64
    x = torch.randn(b, L, H, P, generator=g)
    B = torch.randn(b, L, G, N, generator=g)
    C = torch.randn(b, L, G, N, generator=g)
    dt = F.softplus(torch.randn(b, L, H, generator=g) - 2.0)
    A = -torch.exp(torch.rand(H, generator=g) * 2.5)
    s0 = 0.1 * torch.randn(b, H, P, N, generator=g) if h0 else None
    say(f"h_states G={G} N={N} h0={h0} {dtype}")
    xd, Bd, Cd = dev(x, dtype), dev(B, dtype), dev(C, dtype)
    y, hs, fin = mh.selective_scan(xd, dev(dt), dev(A), Bd, Cd, None, return_h_states=True, return_final_state=True,
                                   initial_state=dev(s0) if h0 else None)
    torch.cuda.synchronize()
    assert hs.shape == (b, L, N) and hs.dtype == dtype
    r = ref.ssd_h_states(host(xd), dt.double().numpy(), A.double().numpy(), host(Bd),
                         initial_state=s0.double().numpy() if h0 else None)
    check("h_states", hs, r, TOL[dtype])
    check("h_states last row = mean of final state", hs[:, -1], host(fin).mean(axis=(1, 2)), TOL[dtype])


def _scan_recurrence_f64(x, dt_raw, A, B, C, D, bias, h0):
    """The scan written as its plain recurrence in float64 torch (autograd gives the reference gradients):
    dt = softplus(dt_raw + bias); h_t = e^{A dt_t} h_{t-1} + dt_t x_t B_t^T; y_t = C_t h_t + D x_t;
    h_states_t = mean over (h, p) of h_t (mamba2.py:98-116)."""
    b, L, H, P = x.shape
    G = B.shape[2]
    gidx = torch.arange(H) // (H // G)
    dt = F.softplus(dt_raw + bias)
    h = h0 if h0 is not None else torch.zeros(b, H, P, B.shape[3], dtype=torch.float64)
    ys, hs = [], []
    for t in range(L):
        h = torch.exp(A * dt[:, t])[..., None, None] * h + \
            (dt[:, t, :, None, None] * x[:, t, :, :, None]) * B[:, t][:, gidx][:, :, None, :]
        ys.append(torch.einsum("bhpn,bhn->bhp", h, C[:, t][:, gidx]) + D[:, None] * x[:, t])
        hs.append(h.mean(dim=(1, 2)))
    return torch.stack(ys, 1), torch.stack(hs, 1), h


@pytest.mark.parametrize("dtype,A_scale", [(torch.float32, 40.0), (torch.bfloat16, 200.0)])
def test_h_states_extreme_decay_vs_oracle(dtype, A_scale):
    """Decay ranges far beyond what one factorised product holds within a 32-token segment (heads with
    A dt up to -A_scale per token next to slow ones): those heads take the direct exponential path."""
    g = torch.Generator().manual_seed(int(A_scale))
    b, L, H, P, N, G = 2, 150, 8, 64, 64, 2
    x = torch.randn(b, L, H, P, generator=g)
    B = torch.randn(b, L, G, N, generator=g)
    C = torch.randn(b, L, G, N, generator=g)
    dt = torch.rand(b, L, H, generator=g) + 0.05
    A = -torch.tensor([A_scale, 0.5, 3.0, A_scale / 4, 0.01, 10.0, A_scale, 1.0])
    s0 = torch.randn(b, H, P, N, generator=g) * 0.1
    say(f"h_states extreme decay {dtype} A_scale={A_scale}")
    _, hs = mh.selective_scan(dev(x, dtype), dev(dt), dev(A), dev(B, dtype), dev(C, dtype), None,
                              return_h_states=True, initial_state=dev(s0))
    torch.cuda.synchronize()
    r = ref.ssd_h_states(host(dev(x, dtype)), dt.double().numpy(), A.double().numpy(), host(dev(B, dtype)),
                         initial_state=s0.double().numpy())
    check("h_states", hs, r, TOL[dtype])


@pytest.mark.parametrize("dtype,G,N,h0", [(torch.float32, 1, 64, False), (torch.float32, 2, 128, True),
                                          (torch.bfloat16, 1, 128, True), (torch.float32, 1, 32, True),
                                          (torch.float32, 2, 256, False)])
def test_h_states_autograd_vs_recurrence(dtype, G, N, h0):
    """selective_scan(return_h_states=True) under autograd (the path Mamba2Layer trains through with
    return_h_states, hybrid.py:383-395): every input gradient of <wy, y> + <wh, h_states> + <wf, final_state>
    against autograd of the float64 recurrence."""
    g = torch.Generator().manual_seed(31 + N + G)
    b, L, H, P = 1, 70, 4, 64
    q = lambda t: t.to(dtype).to(torch.float64)       # inputs exactly representable in the I/O dtype
    x, B, C = q(torch.randn(b, L, H, P, generator=g)), q(torch.randn(b, L, G, N, generator=g)), \
        q(torch.randn(b, L, G, N, generator=g))
    dt_raw = torch.randn(b, L, H, generator=g, dtype=torch.float64) - 1.0
    bias = 0.3 * torch.randn(H, generator=g, dtype=torch.float64)
    A = -torch.exp(torch.rand(H, generator=g, dtype=torch.float64) * 2.5)
    D = 1 + 0.1 * torch.randn(H, generator=g, dtype=torch.float64)
    s0 = 0.1 * torch.randn(b, H, P, N, generator=g, dtype=torch.float64) if h0 else None
    wy = torch.randn(b, L, H, P, generator=g, dtype=torch.float64)
    wh = torch.randn(b, L, N, generator=g, dtype=torch.float64) * 10.0
    wf = torch.randn(b, H, P, N, generator=g, dtype=torch.float64) * 0.1
    say(f"h_states autograd G={G} N={N} h0={h0} {dtype}")
    leaves = dict(x=dev(x, dtype), dt=dev(dt_raw), A=dev(A), B=dev(B, dtype), C=dev(C, dtype), D=dev(D),
                  bias=dev(bias), h0=dev(s0) if h0 else None)
    for t in leaves.values():
        if t is not None:
            t.requires_grad_()
    y, hs, fin = mh.selective_scan(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], leaves["D"],
                                   return_h_states=True, return_final_state=True, initial_state=leaves["h0"],
                                   dt_bias=leaves["bias"], dt_softplus=True)
    loss = (y.float() * dev(wy)).sum() + (hs.float() * dev(wh)).sum() + (fin * dev(wf)).sum()
    loss.backward()
    torch.cuda.synchronize()
    r = dict(x=x, dt=dt_raw, A=A, B=B, C=C, D=D, bias=bias, h0=s0)
    for t in r.values():
        if t is not None:
            t.requires_grad_()
    ry, rhs, rfin = _scan_recurrence_f64(r["x"], r["dt"], r["A"], r["B"], r["C"], r["D"], r["bias"], r["h0"])
    check("h_states", hs, rhs.detach().numpy(), TOL[dtype])
    ((ry * wy).sum() + (rhs * wh).sum() + (rfin * wf).sum()).backward()
    for name in ("x", "dt", "A", "B", "C", "D", "bias") + (("h0",) if h0 else ()):
        check(f"d{name}", leaves[name].grad, r[name].grad.numpy(), TOL[dtype])


def _h_states_f64(x, dt_raw, A, B, bias, h0, limit):
    """h_states alone as the plain float64 recurrence of the full state (autograd gives the reference gradients):
    dt = clamp(softplus(dt_raw + bias), *limit); h_t = e^{A dt_t} h_{t-1} + dt_t x_t B_t^T; h_states_t = mean over
    (h, p) of h_t (mamba2.py:98-116)."""
    b, L, H, P = x.shape
    G = B.shape[2]
    gidx = torch.arange(H) // (H // G)
    dt = F.softplus(dt_raw + bias)
    if limit is not None:
        dt = dt.clamp(*limit)
    h = h0 if h0 is not None else torch.zeros(b, H, P, B.shape[3], dtype=torch.float64)
    hs = []
    for t in range(L):
        h = torch.exp(A * dt[:, t])[..., None, None] * h + \
            (dt[:, t, :, None, None] * x[:, t, :, :, None]) * B[:, t][:, gidx][:, :, None, :]
        hs.append(h.mean(dim=(1, 2)))
    return torch.stack(hs, 1) if hs else torch.zeros(b, 0, B.shape[3], dtype=torch.float64)


@pytest.mark.parametrize("dtype,b,L,H,G,N,h0,limit,A_scale", [
    (torch.float32, 1, 70, 4, 1, 64, True, None, 2.5),
    (torch.float32, 2, 97, 6, 2, 128, False, (0.05, 0.9), 2.5),
    (torch.bfloat16, 1, 64, 8, 1, 128, True, None, 2.5),
    (torch.float32, 2, 1, 8, 4, 16, True, None, 2.5),
    (torch.float32, 1, 45, 6, 3, 24, True, None, 2.5),
    (torch.float32, 1, 40, 128, 2, 128, True, None, 2.5),
    (torch.float32, 1, 150, 8, 2, 64, True, None, 60.0),
    (torch.bfloat16, 2, 33, 5, 1, 8, False, (0.01, 2.0), 2.5),
    (torch.float32, 1, 40, 4, 1, 256, True, None, 2.5),        # dstate 256: two column pieces of 128
    (torch.float32, 1, 33, 192, 3, 64, True, None, 2.5),       # 192 heads: blocks of two groups and one group
    (torch.float32, 1, 20, 160, 1, 32, False, None, 2.5),      # one group of 160 heads, cut at 128
    (torch.bfloat16, 1, 30, 136, 2, 200, True, (0.02, 1.5), 2.5),   # both splits at once
])
def test_h_states_gradients_alone_vs_recurrence(dtype, b, L, H, G, N, h0, limit, A_scale):
    """The gradient of <wh, h_states> alone (mh_ssd_h_states_bwd; more than 128 heads or dstate above 128 as head
    blocks and state-column pieces of the same kernels) w.r.t. x, the raw dt, A, B, dt_bias and the initial state
    against autograd of the float64 full-state recurrence: ragged segment ends, several groups, odd heads per
    group, the clamp's zero gradient, 128 to 192 heads, dstate 200 and 256, one token, and decays far beyond e^-80
    per 32-token segment (A_scale)."""
    g = torch.Generator().manual_seed(L * 13 + H + N)
    P = 64
    q = lambda t: t.to(dtype).to(torch.float64)
    x, B = q(torch.randn(b, L, H, P, generator=g)), q(torch.randn(b, L, G, N, generator=g))
    dt_raw = torch.randn(b, L, H, generator=g, dtype=torch.float64) - 1.0
    bias = 0.3 * torch.randn(H, generator=g, dtype=torch.float64)
    A = -torch.exp(torch.rand(H, generator=g, dtype=torch.float64) * np.log(A_scale))
    s0 = 0.1 * torch.randn(b, H, P, N, generator=g, dtype=torch.float64) if h0 else None
    wh = torch.randn(b, L, N, generator=g, dtype=torch.float64) * 10.0
    say(f"h_states gradients alone {dtype} b={b} L={L} H={H} G={G} N={N} h0={h0} limit={limit} A_scale={A_scale}")
    leaves = dict(x=dev(x, dtype), dt=dev(dt_raw), A=dev(A), B=dev(B, dtype), bias=dev(bias),
                  h0=dev(s0) if h0 else None)
    for t in leaves.values():
        if t is not None:
            t.requires_grad_()
    C = dev(torch.zeros(b, L, G, N), dtype)
    _, hs = mh.selective_scan(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], C, None, return_h_states=True,
                              initial_state=leaves["h0"], dt_bias=leaves["bias"], dt_softplus=True, dt_limit=limit)
    (hs.float() * dev(wh)).sum().backward()
    torch.cuda.synchronize()
    r = dict(x=x, dt=dt_raw, A=A, B=B, bias=bias, h0=s0)
    for t in r.values():
        if t is not None:
            t.requires_grad_()
    rhs = _h_states_f64(r["x"], r["dt"], r["A"], r["B"], r["bias"], r["h0"], limit)
    check("h_states", hs, rhs.detach().numpy(), TOL[dtype])
    (rhs * wh).sum().backward()
    for name in ("x", "dt", "A", "B", "bias") + (("h0",) if h0 else ()):
        check(f"d{name}", leaves[name].grad, r[name].grad.numpy(), TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_h_states_bwd_matches_swapped_prefill_backward_at_size(dtype):
    """At a training size (b2 L2048 H64 N128) the dedicated h_states backward and autograd through the swapped
    prefill (the prefill backward kernels on the problem with x and B exchanged) give the same gradients."""
    g = torch.Generator(device="cuda").manual_seed(5)
    b, L, H, P, G, N = 2, 2048, 64, 64, 1, 128
    x = torch.randn(b, L, H, P, device="cuda", generator=g).to(dtype)
    B = torch.randn(b, L, G, N, device="cuda", generator=g).to(dtype)
    dt = torch.randn(b, L, H, device="cuda", generator=g) - 2.0
    A = -torch.exp(torch.rand(H, device="cuda", generator=g) * 2.0)
    bias = 0.2 * torch.randn(H, device="cuda", generator=g)
    h0 = 0.1 * torch.randn(b, H, P, N, device="cuda", generator=g)
    ghs = torch.randn(b, L, N, device="cuda", generator=g).to(dtype)
    say(f"h_states bwd vs swapped prefill at size {dtype}")
    got = ops._h_states_bwd_kernel(ghs, x, dt, A, B, h0, bias, True, None)
    leaves = [t.detach().clone().requires_grad_() for t in (x, dt, A, B, h0, bias)]
    hs = ops._h_states_swap(*leaves[:5], leaves[5], True, None, None, grad=True)
    want = torch.autograd.grad(hs, leaves, ghs)
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for name, a_, w_ in zip(("dx", "ddt", "dA", "dB", "dh0", "dbias"), got, want):
        check(name, a_, w_.double().cpu().numpy(), tol)


def test_h_states_bwd_empty_sequence():
    """L = 0: no token reaches h_states, so every gradient is zero (and the initial state's too)."""
    from mamformer_amd import ops
    b, H, P, G, N = 2, 4, 64, 1, 32
    x = torch.zeros(b, 0, H, P, device="cuda")
    B = torch.zeros(b, 0, G, N, device="cuda")
    dt = torch.zeros(b, 0, H, device="cuda")
    A = -torch.ones(H, device="cuda")
    h0 = torch.randn(b, H, P, N, device="cuda")
    bias = torch.ones(H, device="cuda")
    say("h_states bwd empty sequence")
    dx, ddt, dA, dB, dh0, dbias = ops._h_states_bwd_kernel(torch.zeros(b, 0, N, device="cuda"), x, dt, A, B, h0,
                                                           bias, True, None)
    torch.cuda.synchronize()
    assert dx.shape == (b, 0, H, P) and dB.shape == (b, 0, G, N)
    for t in (dA, dh0, dbias):
        assert torch.count_nonzero(t).item() == 0


# ----------------------------------------------------------------- Mamba2Layer

def _layer_ref(layer, u, cache=None):
    """Float64 composition of the layer from the oracle pieces.  Without a cache: the prefill, A_log clamped to
    [-5, 5] (mamba2.py:87); with one (conv_state, ssm_state): the decode step, A_log unclamped (:441-443)."""
    P64 = {k: v.detach().double().cpu().numpy() for k, v in layer.named_parameters()}
    un = u.detach().double().cpu().numpy()
    xz = un @ P64["in_proj.weight"].T
    x, z = np.split(xz, 2, axis=-1)
    conv_state = None if cache is None else host(cache["conv_state"])
    xc = ref.ref_causal_conv1d(x, P64["conv_weight"], conv_state=conv_state)
    xa = xc / (1.0 + np.exp(-xc))
    dt_raw = (xa @ P64["dt_proj.0.weight"].T) @ P64["dt_proj.1.weight"].T
    Bm = xa @ P64["B_proj.weight"].T
    Cm = xa @ P64["C_proj.weight"].T
    b, L, _ = un.shape
    H, Pd, G, N = layer.nheads, layer.headdim, layer.ngroups, layer.d_state
    dt = ref.softplus(dt_raw + P64["dt_bias"])
    A = -np.exp(P64["A_log"] if cache is not None else np.clip(P64["A_log"], -5.0, 5.0))
    h0 = None if cache is None else host(cache["ssm_state"]).reshape(b, H, Pd, N)
    y, fin = ref.ssd_direct(xa.reshape(b, L, H, Pd), dt, A, Bm.reshape(b, L, G, N), Cm.reshape(b, L, G, N),
                            P64["D"], initial_state=h0)
    hs = ref.ssd_h_states(xa.reshape(b, L, H, Pd), dt, A, Bm.reshape(b, L, G, N))
    y = y.reshape(b, L, H * Pd) * (z / (1.0 + np.exp(-z)))
    out = y @ P64["out_proj.weight"].T
    return out, fin.reshape(b, H * Pd, N), hs, x


@pytest.mark.parametrize("G,N,P", [(1, 64, 64), (2, 128, 64), (1, 16, 64), (2, 32, 64), (1, 256, 64), (2, 128, 128),
                                   (1, 64, 32)])
def test_mamba2_layer_forward_vs_oracle(G, N, P):
    """The layer's prefill (and its h_states and cache) against the float64 composition; head sizes 128 and 32 run
    through the ops' 64-channel heads."""
    torch.manual_seed(11)
    layer = Mamba2Layer(256, d_state=N, expand=1, headdim=P, ngroups=G, device="cuda", dtype=torch.float32)
    with torch.no_grad():   # larger dt projections than the default init so the scan dominates the output
        for lin in layer.dt_proj:
            lin.weight.normal_(std=0.05)
    u = torch.randn(2, 97, 256, device="cuda")
    say(f"Mamba2Layer forward G={G} N={N} headdim={P}")
    with torch.no_grad():
        out, cache = layer(u)
        out2, cache2, hs = layer(u, use_cache=True, return_h_states=True)
    torch.cuda.synchronize()
    assert cache is None
    r_out, r_fin, r_hs, r_x = _layer_ref(layer, u)
    check("layer out", out, r_out, 1e-4)
    check("layer out (cache path)", out2, r_out, 1e-4)
    check("layer h_states", hs, r_hs, 1e-4)
    check("layer ssm_state", cache2["ssm_state"], r_fin, 1e-4)
    assert cache2["ssm_state"].shape == (2, 256, N)
    assert torch.equal(cache2["conv_state"], layer.in_proj(u)[:, -3:, :256])


def test_mamba2_layer_A_log_clamped_in_prefill_only():
    """A_log beyond [-5, 5]: the prefill uses exp(clamp(A_log)) (mamba2.py:87), the decode step exp(A_log)
    (:441-443), as the reference does."""
    torch.manual_seed(13)
    layer = Mamba2Layer(256, d_state=64, expand=1, headdim=64, ngroups=1, device="cuda", dtype=torch.float32)
    with torch.no_grad():
        layer.A_log.copy_(torch.tensor([6.0, -6.0, 1.0, 5.5], device="cuda"))
        for lin in layer.dt_proj:
            lin.weight.normal_(std=0.05)
    u = torch.randn(2, 40, 256, device="cuda")
    say("Mamba2Layer A_log clamp: prefill vs decode")
    with torch.no_grad():
        pre, c = layer(u[:, :39], use_cache=True)
        step, c2 = layer(u[:, 39:], use_cache=True, cache=c)
    torch.cuda.synchronize()
    r_pre, r_fin, _, _ = _layer_ref(layer, u[:, :39])
    check("prefill (clamped A)", pre, r_pre, 1e-4)
    check("prefill state", c["ssm_state"], r_fin, 1e-4)
    r_step, r_sfin, _, _ = _layer_ref(layer, u[:, 39:], cache=c)
    check("step (unclamped A)", step, r_step, 1e-4)
    check("step state", c2["ssm_state"], r_sfin, 1e-4)


@pytest.mark.parametrize("P", [64, 128, 32])
def test_mamba2_layer_prefill_then_step_equals_longer_prefill(P):
    torch.manual_seed(12)
    layer = Mamba2Layer(256, d_state=128, expand=2, headdim=P, ngroups=1, device="cuda", dtype=torch.float32)
    u = torch.randn(2, 65, 256, device="cuda")
    say(f"Mamba2Layer prefill 64 + step vs prefill 65, headdim {P}")
    with torch.no_grad():
        full, cfull = layer(u, use_cache=True)
        pre, c = layer(u[:, :64], use_cache=True)
        step, c2 = layer(u[:, 64:], use_cache=True, cache=c)
        step2, c3 = layer(u[:, 64:], use_cache=True, cache=c2)   # a second step keeps going
    torch.cuda.synchronize()
    check("prefill prefix", pre, host(full[:, :64]), 1e-4)
    check("step output", step, host(full[:, 64:]), 1e-4)
    check("step ssm_state", c2["ssm_state"], host(cfull["ssm_state"]), 1e-4)
    # raw x rows come from in_proj GEMMs of different sizes: equal to fp32 rounding, not bit for bit
    check("step conv_state", c2["conv_state"], host(cfull["conv_state"]), 1e-5)
    assert step2.shape == (2, 1, 256) and torch.isfinite(step2).all()


def test_mamba2_layer_bf16_runs_the_hip_path():
    torch.manual_seed(13)
    layer = Mamba2Layer(512, d_state=128, expand=2, headdim=64, device="cuda", dtype=torch.bfloat16)
    u = torch.randn(1, 300, 512, device="cuda", dtype=torch.bfloat16)
    say("Mamba2Layer bf16")
    with torch.no_grad():
        out, cache = layer(u, use_cache=True)
        lay32 = Mamba2Layer(512, d_state=128, expand=2, headdim=64, device="cuda", dtype=torch.float32)
        lay32.load_state_dict({k: v.float() for k, v in layer.state_dict().items()})
        out32, _ = lay32(u.float(), use_cache=True)
    torch.cuda.synchronize()
    check("bf16 layer vs fp32 layer", out, host(out32), 2e-2)
    assert cache["ssm_state"].dtype == torch.float32


# ----------------------------------------------------------------- KDA state semantics

def _kda_inputs(seed, B=2, H=2, S=40, D=128):
    g = torch.Generator().manual_seed(seed)
    mk = lambda: (torch.randn(B, H, S, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    return mk(), mk(), mk(), mk(), torch.randn(H, generator=g)


@pytest.mark.parametrize("K", [128, 64])
def test_kda_linear_attention_cache_semantics(K):
    q1, q2, k, v, lr = _kda_inputs(3 + K)
    B, H, S, D = q1.shape
    a = {n: t.double().numpy() for n, t in dict(q1=q1, q2=q2, k=k, v=v).items()}
    say(f"kda_linear_attention K={K}")
    # no cache: the normalised scan from zero
    out, c = kda_linear_attention(dev(q1, torch.bfloat16), dev(q2, torch.bfloat16), dev(k, torch.bfloat16),
                                  dev(v, torch.bfloat16), dev(lr), K)
    torch.cuda.synchronize()
    r = okda.ref_attention_scan(a["q1"], a["q2"], a["k"], a["v"], K, lr.double().numpy())
    check("no-cache output", out, r, 1e-2)
    assert c is None
    # multi-token with a cache: outputs ignore S_prev, the cache accumulates it (kda_diff.py:287-338)
    gs = torch.Generator().manual_seed(99)
    S_prev = torch.rand(B, H, K, D, generator=gs)
    z_prev = torch.rand(B, H, K, 1, generator=gs) + 1.0
    cache = {"S": dev(S_prev), "z": dev(z_prev), "attn_type": "linear"}
    out2, c2 = kda_linear_attention(dev(q1, torch.bfloat16), dev(q2, torch.bfloat16), dev(k, torch.bfloat16),
                                    dev(v, torch.bfloat16), dev(lr), K, use_cache=True, cache=cache)
    torch.cuda.synchronize()
    check("cached multi-token output", out2, r, 1e-2)
    _, _, S_sum, z_sum = okda.ref_scan_pair(a["q1"], a["q2"], a["k"], a["v"], K)
    # bf16 I/O: the scan's MFMAs take phi(k) and v as bf16 operands, so the state is within the bf16 bound
    check("cache S", c2["S"], S_prev.double().numpy() + S_sum, 1e-2)
    check("cache z", c2["z"], z_prev.double().numpy() + z_sum[..., None], 1e-2)
    # one-token step from that cache
    t1 = lambda x: x[:, :, :1]
    out3, c3 = kda_linear_attention(dev(t1(q1), torch.bfloat16), dev(t1(q2), torch.bfloat16),
                                    dev(t1(k), torch.bfloat16), dev(t1(v), torch.bfloat16), dev(lr), K,
                                    use_cache=True, cache=c2)
    torch.cuda.synchronize()
    fm = lambda x: okda.feature_map(x[:, :, :1], K)
    r3, S3, z3 = okda.ref_attention_recurrent(fm(a["q1"]), fm(a["q2"]), fm(a["k"]), a["v"][:, :, :1],
                                              host(c2["S"]), host(c2["z"]), lr.double().numpy())
    check("one-token output", out3, r3, 1e-2)
    check("one-token cache S", c3["S"], S3, 1e-4)
    check("one-token cache z", c3["z"], z3, 1e-4)
    assert c3["attn_type"] == "linear" and c3["S"].shape == (B, H, K, D) and c3["z"].shape == (B, H, K, 1)


def test_h_states_bwd_rows_match_dx_and_scan_bwd_adds_rows():
    """mh_ssd_h_states_bwd with dx_rows writes the one value per (token, head) that it otherwise broadcasts over
    the row of dx (equal after the bf16 rounding), leaving its other outputs bit-identical; mh_ssd_chunk_scan_bwd
    with dx_rows adds them to every channel of its dx and leaves its other outputs bit-identical."""
    g = torch.Generator().manual_seed(5)
    b, L, H, P, N, G = 2, 200, 8, 64, 64, 2
    bf = torch.bfloat16
    x = torch.randn(b, L, H, P, generator=g).to(bf).cuda()
    dt = F.softplus(torch.randn(b, L, H, generator=g) - 1.0).cuda()
    A = -torch.exp(torch.rand(H, generator=g) * 2.0).cuda()
    B = torch.randn(b, L, G, N, generator=g).to(bf).cuda()
    C = torch.randn(b, L, G, N, generator=g).to(bf).cuda()
    D = (1 + 0.1 * torch.randn(H, generator=g)).cuda()
    ghs = torch.randn(b, L, N, generator=g).to(bf).cuda()
    dy = torch.randn(b, L, H, P, generator=g).to(bf).cuda()
    say("h_states bwd rows / scan bwd dx_rows")
    r_dx = ops._h_states_bwd_kernel(ghs, x, dt, A, B, None, None, False, None)
    r_rows = ops._h_states_bwd_kernel(ghs, x, dt, A, B, None, None, False, None, rows=True)
    cfg = (False, None, None, None)
    base = ops._scan_bwd(x, dt, A, B, C, D, None, None, cfg, dy, None, False)
    withr = ops._scan_bwd(x, dt, A, B, C, D, None, None, cfg, dy, None, False, dx_rows=r_rows[0])
    torch.cuda.synchronize()
    assert r_rows[0].shape == (b, L, H) and r_rows[0].dtype == torch.float32
    assert torch.equal(r_dx[0], r_rows[0].to(bf)[..., None].expand(b, L, H, P))
    for k in (1, 2, 3):
        assert torch.equal(r_dx[k], r_rows[k])
    ref = base[0].double().cpu() + r_rows[0].double().cpu()[..., None]
    check("dx + rows", withr[0], ref.numpy(), 5e-3)
    for k in range(1, 6):
        assert torch.equal(base[k], withr[k])
