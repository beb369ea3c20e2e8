"""GPU parity of the reference-form scan's backward (``ops.selective_scan_reference`` under autograd ->
mh_ssd_ref_scan_bwd, csrc/ssd_refform.hip) against autograd of the reference's recurrence written out in float64
torch (mamba2.py:84-126: A = -exp(clamp(A_log, -5, 5)), dA = exp(A dt), h = dA h + dt x B, y = C.h + D x,
h_states = mean over channels, final = h).  That restatement is first checked against the pinned float64 oracle
(``oracle.ssd.ref_selective_scan``, tests/test_oracle.py) on the same inputs, so the gradients are those of the
oracle's function.

Tolerance: relative L2 <= 1e-4 (fp32 I/O) and <= 1e-2 (bf16 I/O) on every gradient (x, dt, A_log, B, C, D, dt_bias,
the initial state).  Cases: N in {16, 32, 64, 128, 256}; a loss on y, h_states and the final state together, on
h_states alone and on y alone; A_log beyond the clamp (zero gradient there, as torch.clamp passes none); dt's
bias / softplus / clamp prologue; the z-gate; run-to-run identical gradients; and the 1b-preset shape (b 2, L 4096,
d_inner 2048, N 128) through two size-independent properties: the gradients are linear in the output gradient
(doubling dy doubles every gradient bit for bit), and with dy zero past token T0 they equal the T0-token problem's.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import mamformer_amd as mh
from oracle import ssd as ossd
from tests.gpu_helpers import check, say

pytestmark = pytest.mark.gpu
F32, BF = torch.float32, torch.bfloat16
TOLS = {F32: 1e-4, BF: 1e-2}


def ref_scan(x, dt_raw, A_log, B, C, D, h0, bias, softplus, limit):
    """The reference's recurrence in float64 torch (autograd gives the reference gradients)."""
    dt = dt_raw if bias is None else dt_raw + bias
    if softplus:
        dt = F.softplus(dt)
    if limit is not None:
        dt = torch.clamp(dt, limit[0], limit[1])
    A = -torch.exp(torch.clamp(A_log, -5.0, 5.0))
    b, L, di = x.shape
    h = h0 if h0 is not None else torch.zeros(b, di, A.shape[0], dtype=x.dtype)
    ys, hss = [], []
    for t in range(L):
        a = torch.exp(A[None, None, :] * dt[:, t, :, None])
        h = a * h + (dt[:, t, :, None] * x[:, t, :, None]) * B[:, t, None, :]
        y = (h * C[:, t, None, :]).sum(-1)
        if D is not None:
            y = y + D * x[:, t]
        ys.append(y)
        hss.append(h.mean(1))
    return torch.stack(ys, 1), torch.stack(hss, 1), h


def make(seed, b, L, di, N, dtype, h0=True, bias=True, D=True):
    g = torch.Generator().manual_seed(seed)
    q = lambda t: t.to(dtype).to(torch.float64)          # inputs exactly representable in the I/O dtype
    x = q(torch.randn(b, L, di, generator=g))
    B = q(torch.randn(b, L, N, generator=g))
    C = q(torch.randn(b, L, N, generator=g))
    dt_raw = torch.randn(b, L, di, generator=g, dtype=torch.float64) - 1.0
    A_log = torch.log(torch.linspace(0.5, 8.0, N, dtype=torch.float64))
    Dv = 1 + 0.1 * torch.randn(di, generator=g, dtype=torch.float64) if D else None
    s0 = 0.1 * torch.randn(b, di, N, generator=g, dtype=torch.float64) if h0 else None
    bv = 0.3 * torch.randn(di, generator=g, dtype=torch.float64) if bias else None
    wy = torch.randn(b, L, di, generator=g, dtype=torch.float64)
    wh = torch.randn(b, L, N, generator=g, dtype=torch.float64) * 10.0
    wf = torch.randn(b, di, N, generator=g, dtype=torch.float64) * 0.1
    return dict(x=x, dt=dt_raw, A_log=A_log, B=B, C=C, D=Dv, h0=s0, bias=bv), (wy, wh, wf)


def run_both(inp, ws, dtype, use=(True, True, True), softplus=True, limit=None, z=None):
    """Gradients of <wy, y> + <wh, h_states> + <wf, final> (the terms in `use`) from the HIP path and from the float64
    reference; returns (hip grads, reference grads) as dicts of float64 CPU tensors."""
    wy, wh, wf = ws
    io = {"x": dtype, "B": dtype, "C": dtype}
    leaves = {k: (None if v is None else v.to(io.get(k, torch.float32)).cuda().requires_grad_())
              for k, v in inp.items()}
    zc = None if z is None else z.to(dtype).cuda()
    y, hs, fin = mh.selective_scan_reference(leaves["x"], leaves["dt"], leaves["A_log"], leaves["B"], leaves["C"],
                                             leaves["D"], True, True, initial_state=leaves["h0"],
                                             dt_bias=leaves["bias"], dt_softplus=softplus, dt_limit=limit, z=zc)
    loss = 0.0
    if use[0]:
        loss = loss + (y.float() * wy.float().cuda()).sum()
    if use[1]:
        loss = loss + (hs.float() * wh.float().cuda()).sum()
    if use[2]:
        loss = loss + (fin * wf.float().cuda()).sum()
    loss.backward()
    torch.cuda.synchronize()
    got = {k: v.grad.double().cpu() for k, v in leaves.items() if v is not None}
    r = {k: (None if v is None else v.clone().requires_grad_()) for k, v in inp.items()}
    ry, rhs, rfin = ref_scan(r["x"], r["dt"], r["A_log"], r["B"], r["C"], r["D"], r["h0"], r["bias"], softplus,
                             limit)
    if z is not None:
        ry = ry * F.silu(z.to(dtype).double())
    rl = 0.0
    if use[0]:
        rl = rl + (ry * wy).sum()
    if use[1]:
        rl = rl + (rhs * wh).sum()
    if use[2]:
        rl = rl + (rfin * wf).sum()
    rl.backward()
    want = {k: (v.grad if v.grad is not None else torch.zeros_like(v)) for k, v in r.items() if v is not None}
    return got, want, (ry.detach(), rhs.detach(), rfin.detach())


def test_reference_recurrence_matches_the_oracle():
    """The float64 restatement the gradients come from equals the pinned oracle's forward."""
    inp, _ = make(1, 2, 37, 32, 16, F32, h0=False)
    with torch.no_grad():
        ry, rhs, rfin = ref_scan(inp["x"], inp["dt"], inp["A_log"], inp["B"], inp["C"], inp["D"], inp["h0"],
                                 inp["bias"], True, None)
    dt = F.softplus(inp["dt"] + inp["bias"]).numpy()
    oy, ohs, ofin = ossd.ref_selective_scan(inp["x"].numpy(), dt, inp["A_log"].numpy(), inp["B"].numpy(),
                                            inp["C"].numpy(), inp["D"].numpy(), True, True)
    np.testing.assert_allclose(ry.numpy(), oy, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(rhs.numpy(), ohs, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(rfin.numpy(), ofin, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype,b,L,di,N", [
    (F32, 2, 70, 64, 16), (F32, 1, 100, 48, 32), (F32, 2, 33, 32, 64), (F32, 1, 40, 32, 128), (F32, 1, 21, 16, 256),
    (BF, 2, 50, 64, 64), (BF, 1, 45, 32, 128), (BF, 1, 20, 16, 256),
], ids=lambda v: str(v).replace("torch.", ""))
def test_ref_scan_gradients_vs_recurrence(dtype, b, L, di, N):
    inp, ws = make(L + di + N, b, L, di, N, dtype)
    if N >= 32:
        inp["A_log"][0], inp["A_log"][-1] = -7.0, 6.5      # beyond the [-5, 5] clamp (mamba2.py:87)
    say(f"ref-form backward {dtype} b{b} L{L} d_inner{di} N{N}")
    got, want, _ = run_both(inp, ws, dtype)
    for k in want:
        check(f"d{k}", got[k], want[k].numpy(), TOLS[dtype])
    if N >= 32:
        assert got["A_log"][0] == 0 and got["A_log"][-1] == 0


@pytest.mark.parametrize("use", [(False, True, False), (True, False, False), (False, False, True)],
                         ids=["h_states-only", "y-only", "final-only"])
def test_ref_scan_gradients_single_terms(use):
    inp, ws = make(7, 2, 41, 32, 32, F32)
    say(f"ref-form backward terms {use}")
    got, want, _ = run_both(inp, ws, F32, use=use)
    for k in want:
        check(f"d{k}", got[k], want[k].numpy(), 1e-4)


def test_ref_scan_gradients_dt_limit_and_gate():
    b, L, di, N = 2, 39, 32, 32
    inp, ws = make(11, b, L, di, N, F32, h0=False)
    z = torch.randn(b, L, di, generator=torch.Generator().manual_seed(12), dtype=torch.float64)
    say("ref-form backward dt limit + gate")
    got, want, _ = run_both(inp, ws, F32, limit=(0.05, 0.4), z=z)
    for k in want:
        check(f"d{k}", got[k], want[k].numpy(), 1e-4)


def test_ref_scan_gradients_run_to_run_identical():
    inp, ws = make(13, 2, 64, 64, 64, BF)
    a, _, _ = run_both(inp, ws, BF)
    c, _, _ = run_both(inp, ws, BF)
    for k in a:
        assert torch.equal(a[k], c[k]), k


def test_ref_scan_bwd_1b_preset_full_shape_properties():
    """b 2, L 4096, d_inner 2048, N 128, bf16: doubling dy doubles every gradient bit for bit, and with dy zero
    past token T0 the gradients are those of the T0-token problem (zero past T0), checked against the float64
    recurrence on those T0 tokens."""
    b, L, di, N, T0 = 2, 4096, 2048, 128, 48
    g = torch.Generator().manual_seed(21)
    x = torch.randn(b, L, di, generator=g).to(BF)
    B = torch.randn(b, L, N, generator=g).to(BF)
    C = torch.randn(b, L, N, generator=g).to(BF)
    dt = F.softplus(torch.randn(b, L, di, generator=g) - 2.0)
    A_log = torch.log(torch.linspace(0.5, 8.0, N))
    D = 1 + 0.1 * torch.randn(di, generator=g)
    dy = torch.zeros(b, L, di)
    dy[:, :T0] = torch.randn(b, T0, di, generator=g)
    dy = dy.to(BF)
    say("ref-form backward 1b preset full shape")

    def grads(scale):
        lv = [t.cuda().requires_grad_() for t in (x, dt, A_log, B, C, D)]
        y = mh.selective_scan_reference(*lv)
        y.backward(dy.cuda() * scale)
        torch.cuda.synchronize()
        return [t.grad for t in lv]

    g1, g2 = grads(1.0), grads(2.0)
    for a, c in zip(g1, g2):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(c, a * 2)
    assert not g1[0][:, T0:].any() and not g1[1][:, T0:].any() and not g1[3][:, T0:].any()
    r = [t[:, :T0].double().clone().requires_grad_() if t.dim() == 3 else t.double().clone().requires_grad_()
         for t in (x, dt, A_log, B, C, D)]
    ry, _, _ = ref_scan(r[0], r[1], r[2], r[3], r[4], r[5], None, None, False, None)
    (ry * dy[:, :T0].double()).sum().backward()
    for name, k in (("dx", 0), ("ddt", 1), ("dB", 3), ("dC", 4)):
        check(name, g1[k][:, :T0], r[k].grad.numpy(), 1e-2)
    check("dA_log", g1[2], r[2].grad.numpy(), 1e-2)
    check("dD", g1[5], r[5].grad.numpy(), 1e-2)
