"""GPU parity of the reference-parameterised prefill (``ops.selective_scan_reference`` -> mh_ssd_ref_scan_fwd,
csrc/ssd_refform.hip) against the float64 restatement of the reference's scan (``oracle.ssd.ref_selective_scan``,
mamba2.py:70-130, pinned in tests/test_oracle.py).

The reference's own parameterisation: A_log (N,) clamped to [-5, 5], dt and D per channel, B and C shared by every
channel.  Tolerance: relative L2 <= 1e-4 (fp32 I/O) and <= 1e-2 (bf16 I/O) on y, h_states and the final state.
Cases: several (d_inner, N) including the 1b preset width (d_inner 2048, N 128), A_log beyond the clamp, per-channel
D, h_states and the final state, an initial state (through a split sequence: the second half started from the
first half's final state equals the whole), dt's bias / softplus / clamp prologue in the kernel, the z-gate,
an empty sequence, and the full 1b-preset shape (b 2, L 4096) through exact linearity in x and the split
sequence.  The backward is in tests/test_gpu_ssd_refform_bwd.py.
"""

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from mamformer_amd._lib import MHError
from oracle import ssd as ossd
from tests.gpu_helpers import TOL, check, dev, host, say

pytestmark = pytest.mark.gpu
F32, BF = torch.float32, torch.bfloat16


def case(seed, b, L, di, N, dtype, a_log=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, L, di, generator=g).to(dtype)
    dt = torch.nn.functional.softplus(torch.randn(b, L, di, generator=g) - 2.0)
    A_log = torch.log(torch.linspace(0.5, 8.0, N)) if a_log is None else a_log
    B = torch.randn(b, L, N, generator=g).to(dtype)
    C = torch.randn(b, L, N, generator=g).to(dtype)
    D = torch.randn(di, generator=g) * 0.1 + 1.0
    return x, dt, A_log, B, C, D


def oracle(x, dt, A_log, B, C, D, hs=True, fin=True):
    f = lambda t: t.double().numpy()
    return ossd.ref_selective_scan(f(x), f(dt), f(A_log), f(B), f(C), f(D), hs, fin)


@pytest.mark.parametrize("dtype,b,L,di,N", [
    (F32, 2, 100, 64, 16), (F32, 1, 257, 128, 64), (BF, 2, 70, 48, 32), (BF, 1, 65, 256, 256),
    (F32, 2, 96, 2048, 128), (BF, 2, 128, 2048, 128),
], ids=lambda v: str(v).replace("torch.", ""))
def test_ref_scan_vs_oracle(dtype, b, L, di, N):
    x, dt, A_log, B, C, D = case(L + di + N, b, L, di, N, dtype)
    if N >= 32:
        A_log = A_log.clone()
        A_log[0], A_log[-1] = -7.0, 6.5                    # beyond the [-5, 5] clamp (mamba2.py:87)
    say(f"ref-form scan {dtype} b{b} L{L} d_inner{di} N{N}")
    y, hs, fin = mh.selective_scan_reference(dev(x, dtype), dev(dt), dev(A_log), dev(B, dtype), dev(C, dtype), dev(D),
                                             return_h_states=True, return_final_state=True)
    torch.cuda.synchronize()
    ry, rhs, rfin = oracle(x, dt, A_log, B, C, D)
    tol = TOL[dtype]
    assert y.dtype == dtype and hs.dtype == dtype and fin.dtype == torch.float32
    check("y", y, ry, tol)
    check("h_states", hs, rhs, tol)
    check("final state", fin, rfin, tol)


def test_ref_scan_options_single_outputs():
    """Return forms of the reference: y alone, (y, final) and (y, h_states)."""
    x, dt, A_log, B, C, D = case(5, 1, 40, 32, 16, F32)
    args = (dev(x), dev(dt), dev(A_log), dev(B), dev(C), dev(D))
    y = mh.selective_scan_reference(*args)
    y2, fin = mh.selective_scan_reference(*args, return_final_state=True)
    y3, hs = mh.selective_scan_reference(*args, return_h_states=True)
    torch.cuda.synchronize()
    ry, rhs, rfin = oracle(x, dt, A_log, B, C, D)
    for t in (y, y2, y3):
        check("y", t, ry, 1e-4)
    check("final", fin, rfin, 1e-4)
    check("h_states", hs, rhs, 1e-4)


@pytest.mark.parametrize("dtype", [F32, BF], ids=["float32", "bfloat16"])
def test_ref_scan_initial_state_by_split(dtype):
    """The second part started from the first part's final state gives the whole sequence's outputs."""
    b, L, di, N, L1 = 2, 150, 64, 64, 61
    x, dt, A_log, B, C, D = case(9, b, L, di, N, dtype)
    d = lambda t, ty=torch.float32: dev(t, ty)
    say(f"ref-form split {dtype}")
    y, fin = mh.selective_scan_reference(d(x, dtype), d(dt), d(A_log), d(B, dtype), d(C, dtype), d(D),
                                         return_final_state=True)
    y1, f1 = mh.selective_scan_reference(d(x[:, :L1], dtype), d(dt[:, :L1]), d(A_log), d(B[:, :L1], dtype),
                                         d(C[:, :L1], dtype), d(D), return_final_state=True)
    y2, hs2, f2 = mh.selective_scan_reference(d(x[:, L1:], dtype), d(dt[:, L1:]), d(A_log), d(B[:, L1:], dtype),
                                              d(C[:, L1:], dtype), d(D), True, True, initial_state=f1)
    torch.cuda.synchronize()
    ry, rhs, rfin = oracle(x, dt, A_log, B, C, D)
    tol = TOL[dtype]
    check("y part 1", y1, ry[:, :L1], tol)
    check("y part 2 (initial state)", y2, ry[:, L1:], tol)
    check("h_states part 2", hs2, rhs[:, L1:], tol)
    check("final", f2, rfin, tol)
    check("whole vs split final", fin, host(f2), 1e-5)


def test_ref_scan_dt_prologue_and_gate():
    """dt_bias, softplus and the clamp applied in the kernel; the block's gate y * silu(z)."""
    b, L, di, N = 2, 77, 96, 32
    x, _, A_log, B, C, D = case(3, b, L, di, N, F32)
    g = torch.Generator().manual_seed(4)
    raw = torch.randn(b, L, di, generator=g)
    bias = torch.randn(di, generator=g) * 0.5 - 1.0
    z = torch.randn(b, L, di, generator=g)
    say("ref-form dt prologue + gate")
    y = mh.selective_scan_reference(dev(x), dev(raw), dev(A_log), dev(B), dev(C), dev(D), dt_bias=dev(bias),
                                    dt_softplus=True, dt_limit=(0.01, 0.5), z=dev(z))
    torch.cuda.synchronize()
    dt = torch.clamp(torch.nn.functional.softplus((raw + bias).double()), 0.01, 0.5)
    ry = oracle(x, dt, A_log, B, C, D, hs=False, fin=False)
    zz = z.double().numpy()
    check("gated y", y, ry * zz / (1.0 + np.exp(-zz)), 1e-4)


def test_ref_scan_empty_sequence_and_errors():
    b, di, N = 2, 32, 16
    s0 = torch.randn(b, di, N, device="cuda")
    e = torch.zeros(b, 0, di, device="cuda")
    eb = torch.zeros(b, 0, N, device="cuda")
    y, fin = mh.selective_scan_reference(e, e, torch.zeros(N, device="cuda"), eb, eb, None, return_final_state=True,
                                         initial_state=s0)
    torch.cuda.synchronize()
    assert y.shape == (b, 0, di) and torch.equal(fin, s0)
    x = torch.zeros(1, 4, 32, device="cuda")
    with pytest.raises(MHError):                       # dstate 8: outside what the kernel tiles
        mh.selective_scan_reference(x, x, torch.zeros(8, device="cuda"), torch.zeros(1, 4, 8, device="cuda"),
                                    torch.zeros(1, 4, 8, device="cuda"), None)
    with pytest.raises(ValueError):                    # D per channel only (the reference's (d_inner,))
        mh.selective_scan_reference(x, x, torch.zeros(16, device="cuda"), torch.zeros(1, 4, 16, device="cuda"),
                                    torch.zeros(1, 4, 16, device="cuda"), torch.ones(2, device="cuda"))


def test_ref_scan_1b_preset_full_shape_properties():
    """b 2, L 4096, d_inner 2048, N 128, bf16: doubling x doubles y, h_states and the final state bit for bit (the
    recurrence is linear in x); the sequence split at 2500 with the state carried equals the whole; a leading slice
    equals the oracle."""
    b, L, di, N = 2, 4096, 2048, 128
    x, dt, A_log, B, C, D = case(17, b, L, di, N, BF)
    X, DT, AL, BB, CC, DD = dev(x, BF), dev(dt), dev(A_log), dev(B, BF), dev(C, BF), dev(D)
    say("ref-form 1b preset full shape")
    y, hs, fin = mh.selective_scan_reference(X, DT, AL, BB, CC, DD, True, True)
    y2, hs2, fin2 = mh.selective_scan_reference(X * 2, DT, AL, BB, CC, DD, True, True)
    L1 = 2500
    ya, fa = mh.selective_scan_reference(X[:, :L1], DT[:, :L1], AL, BB[:, :L1], CC[:, :L1], DD,
                                         return_final_state=True)
    yb, fb = mh.selective_scan_reference(X[:, L1:], DT[:, L1:], AL, BB[:, L1:], CC[:, L1:], DD,
                                         return_final_state=True, initial_state=fa)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(fin).all()
    assert torch.equal(y2, y * 2) and torch.equal(hs2, hs * 2) and torch.equal(fin2, fin * 2)
    assert torch.equal(ya, y[:, :L1])
    check("split y", yb, host(y[:, L1:]), 1e-2)
    check("split final", fb, host(fin), 1e-5)
    T0 = 192
    ry, rhs, rfin = oracle(x[:, :T0], dt[:, :T0], A_log, B[:, :T0], C[:, :T0], D)
    check("leading slice y", y[:, :T0], ry, 1e-2)
    check("leading slice h_states", hs[:, :T0], rhs, 1e-2)
