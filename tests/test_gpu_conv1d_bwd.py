"""GPU parity of the causal conv1d backward (mh_causal_conv1d_bwd) and of training through Mamba2Layer.

* ``causal_conv1d`` gradients (dx, dweight, dbias, d_conv_state) through autograd vs the float64 oracle
  ``oracle.ssd_bwd.causal_conv1d_backward`` (pinned against torch autograd of F.conv1d + SiLU): global
  relative L2 <= 1e-2 for bf16 I/O, <= 1e-4 for fp32 I/O.  Widths 1..8, cached rows 0..K-1, no bias,
  empty sequences, runs shorter than the K-1 token halo and lengths that are not multiples of the 32-token
  run.  dweight / dbias are reduced in a fixed order: two calls agree bit for bit.
* ``Mamba2Layer`` (fp32) parameter and input gradients vs torch autograd of a float64 CPU restatement of the
  same layer (F.conv1d, the SSD recurrence token by token): every gradient within relative L2 1e-3 (a
  chain of fp32 GEMMs and kernels, looser than one kernel's 1e-4).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import mamformer_amd as mh
from mamformer_amd.layers import Mamba2Layer
from oracle import ssd_bwd as obwd
from tests.gpu_helpers import TOL, check, dev, host, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("L,D,K,cs_len,has_bias", [
    (1, 8, 4, 0, True), (5, 64, 4, 3, True), (70, 256, 4, 2, False), (1000, 512, 3, 0, True),
    (33, 4096, 2, 1, True), (31, 64, 8, 7, True), (2, 128, 1, 0, False), (3, 64, 6, 5, True),
    (64, 96, 5, 0, True), (0, 64, 4, 3, True),
])
def test_conv1d_bwd_vs_oracle(dtype, L, D, K, cs_len, has_bias):
    g = torch.Generator().manual_seed(L * 13 + D + K)
    b = 2
    x = torch.randn(b, L, D, generator=g)
    w = torch.randn(D, 1, K, generator=g) * 0.5
    bias = torch.randn(D, generator=g) if has_bias else None
    cs = torch.randn(b, cs_len, D, generator=g) if cs_len else None
    dy = torch.randn(b, L, D, generator=g)
    for silu in (False, True):
        say(f"conv1d_bwd L={L} D={D} K={K} cs={cs_len} bias={has_bias} silu={silu} {dtype}")
        xd = dev(x, dtype).requires_grad_()
        wd = dev(w).requires_grad_()
        bd = dev(bias).requires_grad_() if has_bias else None
        csd = dev(cs, dtype).requires_grad_() if cs_len else None
        dyd = dev(dy, dtype)
        y = mh.causal_conv1d(xd, wd, bd, csd, silu=silu)
        ins = [t for t in (xd, wd, bd, csd) if t is not None]
        grads = torch.autograd.grad(y, ins, dyd)
        torch.cuda.synchronize()
        gx, gw = grads[0], grads[1]
        rx, rw, rb, rcs = obwd.causal_conv1d_backward(host(xd), w.numpy(), bias.numpy() if has_bias else None,
                                                      host(dyd), host(csd) if cs_len else None, silu=silu,
                                                      with_state_grad=True)
        assert gx.dtype == dtype and gx.shape == x.shape and gw.shape == w.shape
        tol = TOL[dtype]
        if L:
            check("dx", gx, rx, tol)
        check("dweight", gw.reshape(D, K), rw, tol)
        if has_bias:
            check("dbias", grads[2], rb, tol)
        if cs_len:
            gcs = grads[-1]
            assert gcs.dtype == dtype and gcs.shape == cs.shape
            if L:
                check("d_conv_state", gcs, rcs, tol)
            else:
                np.testing.assert_array_equal(host(gcs), 0.0)


def test_conv1d_bwd_weight_grad_is_deterministic():
    g = torch.Generator().manual_seed(5)
    x = dev(torch.randn(4, 777, 1024, generator=g), torch.bfloat16).requires_grad_()
    w = dev(torch.randn(1024, 1, 4, generator=g)).requires_grad_()
    bias = dev(torch.randn(1024, generator=g)).requires_grad_()
    dy = dev(torch.randn(4, 777, 1024, generator=g), torch.bfloat16)
    say("conv1d_bwd determinism")
    outs = []
    for _ in range(2):
        y = mh.causal_conv1d(x, w, bias, silu=True)
        outs.append(torch.autograd.grad(y, [x, w, bias], dy))
    torch.cuda.synchronize()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


def _layer_ref64(layer, u, with_h_states=False):
    """float64 CPU restatement of Mamba2Layer.forward (full scan, no cache) with autograd leaves; with
    ``with_h_states`` also the per-token mean of the state over the channels."""
    P = {k: v.detach().to("cpu", torch.float64).requires_grad_() for k, v in layer.named_parameters()}
    u64 = u.detach().to("cpu", torch.float64).requires_grad_()
    b, L, _ = u.shape
    H, Pd, N, G, K = layer.nheads, layer.headdim, layer.d_state, layer.ngroups, layer.d_conv
    x, z = F.linear(u64, P["in_proj.weight"], P.get("in_proj.bias")).chunk(2, dim=-1)
    xc = F.conv1d(F.pad(x.transpose(1, 2), (K - 1, 0)), P["conv_weight"], P.get("conv_bias"),
                  groups=layer.d_inner).transpose(1, 2)
    xa = F.silu(xc)
    dt = F.linear(F.linear(xa, P["dt_proj.0.weight"], P.get("dt_proj.0.bias")), P["dt_proj.1.weight"],
                  P.get("dt_proj.1.bias"))
    dt = F.softplus(dt + P["dt_bias"])
    Bm = F.linear(xa, P["B_proj.weight"], P.get("B_proj.bias")).view(b, L, G, N)
    Cm = F.linear(xa, P["C_proj.weight"], P.get("C_proj.bias")).view(b, L, G, N)
    A = -torch.exp(P["A_log"])
    gidx = torch.arange(H) // (H // G)
    x4 = xa.view(b, L, H, Pd)
    h = torch.zeros(b, H, Pd, N, dtype=torch.float64)
    ys, hs = [], []
    for t in range(L):
        a = torch.exp(A[None, :] * dt[:, t])
        h = a[:, :, None, None] * h + (dt[:, t, :, None, None] * x4[:, t, :, :, None]) * Bm[:, t][:, gidx][:, :, None]
        ys.append(torch.einsum("bhpn,bhn->bhp", h, Cm[:, t][:, gidx]) + P["D"][None, :, None] * x4[:, t])
        hs.append(h.mean(dim=(1, 2)))                       # h_states: mean over the channels (mamba2.py:114-116)
    y = torch.stack(ys, 1).reshape(b, L, layer.d_inner) * F.silu(z)
    out = F.linear(y, P["out_proj.weight"], P.get("out_proj.bias"))
    if with_h_states:
        return out, torch.stack(hs, 1), P, u64
    return out, P, u64


@pytest.mark.parametrize("G,bias", [(1, False), (2, True)])
def test_mamba2_layer_gradients_vs_float64_reference(G, bias):
    torch.manual_seed(21 + G)
    layer = Mamba2Layer(128, d_state=64, expand=2, headdim=64, ngroups=G, bias=bias, device="cuda",
                        dtype=torch.float32)
    with torch.no_grad():       # larger weights than the init so that every path carries a visible gradient
        for name, p in layer.named_parameters():
            if name.endswith("weight"):
                p.normal_(0.0, 0.2 if "dt_proj" not in name else 0.05)
            elif name.endswith("bias") and name != "dt_bias":
                p.normal_(0.0, 0.1)
    u = torch.randn(2, 40, 128, device="cuda", requires_grad=True)
    gout = torch.randn(2, 40, 128, device="cuda")
    say(f"Mamba2Layer gradients G={G} bias={bias}")
    out, _ = layer(u)
    (out * gout).sum().backward()
    torch.cuda.synchronize()
    ref, P, u64 = _layer_ref64(layer, u)
    (ref * gout.cpu().double()).sum().backward()
    check("layer out", out, ref.detach().numpy(), 1e-4)
    check("du", u.grad, u64.grad.numpy(), 1e-3)
    for name, p in layer.named_parameters():
        assert p.grad is not None, f"{name}: no gradient reached the parameter"
        check(f"d{name}", p.grad, P[name].grad.numpy(), 1e-3)


@pytest.mark.parametrize("G,N", [(1, 64), (2, 32)])
def test_mamba2_layer_h_states_gradients_vs_float64_reference(G, N):
    """Mamba2Layer(..., return_h_states=True) trained through both outputs (the fusion layers' use,
    hybrid.py:383-395): the gradient of <gout, out> + <ghs, h_states> w.r.t. the input and every parameter against
    autograd of the float64 restatement."""
    torch.manual_seed(41 + G)
    layer = Mamba2Layer(128, d_state=N, expand=2, headdim=64, ngroups=G, device="cuda", dtype=torch.float32)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith("weight"):
                p.normal_(0.0, 0.2 if "dt_proj" not in name else 0.05)
    u = torch.randn(2, 45, 128, device="cuda", requires_grad=True)
    gout = torch.randn(2, 45, 128, device="cuda")
    ghs = torch.randn(2, 45, N, device="cuda") * 20.0      # h_states is small (a mean over d_inner channels)
    say(f"Mamba2Layer h_states gradients G={G} N={N}")
    out, _, hs = layer(u, return_h_states=True)
    ((out * gout).sum() + (hs * ghs).sum()).backward()
    torch.cuda.synchronize()
    ref, rhs, P, u64 = _layer_ref64(layer, u, with_h_states=True)
    ((ref * gout.cpu().double()).sum() + (rhs * ghs.cpu().double()).sum()).backward()
    check("layer out", out, ref.detach().numpy(), 1e-4)
    check("h_states", hs, rhs.detach().numpy(), 1e-4)
    check("du", u.grad, u64.grad.numpy(), 1e-3)
    for name, p in layer.named_parameters():
        assert p.grad is not None, f"{name}: no gradient reached the parameter"
        check(f"d{name}", p.grad, P[name].grad.numpy(), 1e-3)


def test_mamba2_layer_bf16_gradients_track_fp32():
    """bf16 training through the HIP conv and scan backward (bf16 operands, fp32 accumulation) against the same
    layer in fp32: a consistency bound (rel-L2 5e-2 per parameter gradient, bf16 GEMMs and activations on the way),
    not an oracle comparison -- the fp32 layer is the one checked against the float64 restatement above."""
    torch.manual_seed(31)
    lay16 = Mamba2Layer(256, d_state=128, expand=2, headdim=64, ngroups=1, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        for name, p in lay16.named_parameters():
            if name.endswith("weight"):
                p.normal_(0.0, 0.1 if "dt_proj" not in name else 0.05)
    lay32 = Mamba2Layer(256, d_state=128, expand=2, headdim=64, ngroups=1, device="cuda", dtype=torch.float32)
    lay32.load_state_dict({k: v.float() for k, v in lay16.state_dict().items()})
    u = torch.randn(2, 200, 256, device="cuda")
    gout = torch.randn(2, 200, 256, device="cuda")
    say("Mamba2Layer bf16 vs fp32 gradients")
    out16, _ = lay16(u.to(torch.bfloat16))
    (out16.float() * gout).sum().backward()
    out32, _ = lay32(u)
    (out32 * gout).sum().backward()
    torch.cuda.synchronize()
    p32 = dict(lay32.named_parameters())
    for name, p in lay16.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name
        check(f"bf16 d{name}", p.grad, host(p32[name].grad), 5e-2)
