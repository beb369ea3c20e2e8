"""Host logic of ops._Heads64, the map of SSD heads of any size onto the kernels' 64-channel heads (CPU only):
round trips of every map, and the gradient maps as the adjoints of the forward maps (<f(a), b> = <a, f*(b)>
for the per-head values and D), checked with torch autograd on the CPU."""

import pytest
import torch

from mamformer_amd.ops import _Heads64


@pytest.mark.parametrize("P", [32, 64, 96, 128, 192, 1])
def test_round_trips(P):
    torch.manual_seed(P)
    b, L, H, N = 2, 5, 3, 8
    hm = _Heads64(H, P)
    assert hm.Pp % 64 == 0 and hm.Pp >= P and hm.k == hm.Pp // 64
    x = torch.randn(b, L, H, P, dtype=torch.float64)
    xc = hm.chan(x)
    assert xc.shape == (b, L, H * hm.k, 64)
    assert torch.equal(hm.unchan(xc), x)
    # channel p of head h lands in sub-head h k + p // 64, column p % 64; padding is zero
    full = xc.reshape(b, L, H, hm.Pp)
    assert torch.equal(full[..., :P], x) and not full[..., P:].any()
    s = torch.randn(b, H, P, N, dtype=torch.float64)
    sc = hm.state(s)
    assert sc.shape == (b, H * hm.k, 64, N)
    assert torch.equal(hm.unstate(sc), s)
    assert not sc.reshape(b, H, hm.Pp, N)[:, :, P:].any()


@pytest.mark.parametrize("P", [32, 128, 96])
def test_per_head_values_and_adjoints(P):
    torch.manual_seed(100 + P)
    b, L, H = 2, 4, 3
    hm = _Heads64(H, P)
    dt = torch.randn(b, L, H, dtype=torch.float64)
    dts = hm.head(dt, 2)
    assert dts.shape == (b, L, H * hm.k)
    for j in range(hm.k):
        assert torch.equal(dts[:, :, j::hm.k], dt)
    # unhead is the adjoint of head: <head(a), g> = <a, unhead(g)>
    a = torch.randn(H, dtype=torch.float64)
    g = torch.randn(H * hm.k, dtype=torch.float64)
    assert torch.allclose((hm.head(a) * g).sum(), (a * hm.unhead(g)).sum())
    # D per head and per channel: d_grad is the adjoint of d_vec
    for D in (torch.randn(H, dtype=torch.float64), torch.randn(H * P, dtype=torch.float64)):
        Dl = D.clone().requires_grad_()
        v = hm.d_vec(Dl)
        gv = torch.randn_like(v)
        (ga,) = torch.autograd.grad((v * gv).sum(), Dl)
        assert torch.allclose(hm.d_grad(gv, D), ga)
    assert hm.d_vec(None) is None and hm.head(None) is None and hm.unhead(None) is None
