"""GPU parity of the SSD chunked-scan prefill against the float64 oracle (oracle/ssd.py).

Tolerance: global relative L2 <= 1e-2 for bf16 I/O and <= 1e-4 for fp32 I/O,
on y and on the final state.  Small and medium shapes are compared with the
oracle directly (and with the committed golden fixtures); the full benchmark
shapes are checked through size-independent properties (exact linearity,
split-sequence state carry, chunk-length invariance) plus an oracle check on a
leading slice (y is causal) and on a trailing slice started from the GPU's own
carried state.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

import mamformer_amd as mh
from mamformer_amd import workloads as W
from oracle import ssd as ref
from tests.gpu_helpers import TOL, check, dev, host, say

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def run(inp, dtype, chunk=None, **kw):
    x = dev(inp["x"], dtype)
    B = dev(inp["B"], dtype)
    C = dev(inp["C"], dtype)
    dt, A = dev(inp["dt"]), dev(inp["A"])
    D = dev(inp["D"]) if inp.get("D") is not None else None
    h0 = dev(inp["initial_state"]) if inp.get("initial_state") is not None else None
    y, fin = mh.selective_scan(x, dt, A, B, C, D, return_final_state=True, chunk_size=chunk, initial_state=h0,
                               **kw)
    torch.cuda.synchronize()
    return y, fin


def test_ssd1_golden_fp32():
    say("ssd1 golden (b1 L512 H8 P64 N64 fp32)")
    z = np.load(GOLD / "ssd1.npz")
    y, fin = run({k: z[k] for k in ("x", "dt", "A", "B", "C", "D")}, torch.float32, chunk=64)
    check("ssd1 y", y, z["y"], 1e-4)
    check("ssd1 final", fin, z["final"], 1e-4)


def test_ssd_edge_golden():
    z = np.load(GOLD / "ssd_edge.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    for n in names:
        bf = bool(z[f"{n}/bf16"])
        dtype = torch.bfloat16 if bf else torch.float32
        inp = {k: z[f"{n}/{k}"] for k in ("x", "dt", "A", "B", "C", "D")}
        if f"{n}/initial_state" in z.files:
            inp["initial_state"] = z[f"{n}/initial_state"]
        for chunk in (64, 128, None):
            say(f"edge {n} dtype={dtype} chunk={chunk} shape={inp['x'].shape}")
            y, fin = run(inp, dtype, chunk=chunk)
            check(f"{n}/y", y, z[f"{n}/y"], TOL[dtype])
            check(f"{n}/final", fin, z[f"{n}/final"], TOL[dtype])


@pytest.mark.parametrize("case", [
    # (b, L, H, N, G, dtype, h0, seed)
    (2, 1024, 64, 128, 1, torch.bfloat16, False, 101),
    (1, 1500, 32, 128, 2, torch.bfloat16, True, 102),
    (1, 777, 8, 64, 1, torch.float32, True, 103),
    (2, 640, 8, 128, 2, torch.float32, False, 104),
])
def test_ssd_medium_vs_oracle(case):
    b, L, H, N, G, dtype, h0, seed = case
    cfg = W.SSDConfig("m", b, L, H, 64, N, G, 256, dtype, seed, init_state=h0)
    inp = W.ssd_inputs(cfg)
    say(f"medium b{b} L{L} H{H} N{N} G{G} {dtype} h0={h0}")
    y, fin = run(inp, dtype)
    arr = {k: (None if v is None else v.to(torch.float64).numpy()) for k, v in inp.items()}
    y_ref, f_ref = ref.ssd_chunked(arr["x"], arr["dt"], arr["A"], arr["B"], arr["C"], arr["D"],
                                   initial_state=arr["initial_state"], chunk_size=128)
    check("y", y, y_ref, TOL[dtype])
    check("final", fin, f_ref, TOL[dtype])


def test_ssd_dt_processing_and_per_channel_D_and_views():
    """dt_bias + softplus + dt_limit in the kernel, D per channel, x/B/C as strided views of one buffer."""
    g = torch.Generator().manual_seed(7)
    b, L, H, P, N = 2, 333, 8, 64, 64
    d_inner = H * P
    width = d_inner + 2 * N + 64                       # like a fused in_proj output: [x | B | C | pad]
    buf = torch.randn(b, L, width, generator=g).to(torch.bfloat16)
    x = buf[..., :d_inner]
    B = buf[..., d_inner:d_inner + N]
    C = buf[..., d_inner + N:d_inner + 2 * N]
    dt_raw = torch.randn(b, L, H, generator=g)
    bias = torch.randn(H, generator=g) - 3.0
    A = -torch.exp(torch.rand(H, generator=g) * 2.7)
    D = torch.randn(d_inner, generator=g)
    say("dt processing / views")
    y, fin = mh.selective_scan(dev(buf, torch.bfloat16)[..., :d_inner], dev(dt_raw), dev(A),
                               dev(buf, torch.bfloat16)[..., d_inner:d_inner + N],
                               dev(buf, torch.bfloat16)[..., d_inner + N:d_inner + 2 * N], dev(D),
                               return_final_state=True, dt_bias=dev(bias), dt_softplus=True, dt_limit=(0.01, 0.5))
    assert y.shape == (b, L, d_inner) and fin.shape == (b, d_inner, N)
    dt = ref.process_dt(dt_raw.numpy(), bias.numpy(), True, (0.01, 0.5))
    xr = x.to(torch.float64).numpy().reshape(b, L, H, P)
    y_ref, f_ref = ref.ssd_via_reference(xr, dt, A.numpy(), B.to(torch.float64).numpy(),
                                         C.to(torch.float64).numpy(), D.numpy().reshape(H, P))
    check("y", y.view(b, L, H, P), y_ref, 1e-2)
    check("final", fin.view(b, H, P, N), f_ref, 1e-2)


def test_ssd_extreme_decay_cuts_segments():
    """Per-step log-decays down to about -100: segments shrink to a few tokens and results stay exact."""
    g = torch.Generator().manual_seed(9)
    b, L, H, P, N = 1, 200, 4, 64, 64
    x = torch.randn(b, L, H, P, generator=g)
    B = torch.randn(b, L, 1, N, generator=g)
    C = torch.randn(b, L, 1, N, generator=g)
    dt = torch.exp(torch.randn(b, L, H, generator=g) * 2.0)          # 0.02 .. 50
    A = torch.tensor([-16.0, -2.0, -0.5, -0.01])
    say("extreme decay")
    y, fin = mh.selective_scan(dev(x), dev(dt), dev(A), dev(B), dev(C), None, return_final_state=True)
    y_ref, f_ref = ref.ssd_direct(x.double().numpy(), dt.double().numpy(), A.double().numpy(),
                                  B.double().numpy(), C.double().numpy())
    check("y", y, y_ref, 1e-4)
    check("final", fin, f_ref, 1e-4)


@pytest.mark.parametrize("N,chunk,init", [(128, 256, False), (64, 128, True), (128, 64, True), (128, 1024, True)])
def test_ssd_extreme_decay_bf16_multipass(N, chunk, init):
    """bf16 I/O with per-step log-decays from about -0.01 to below -100 per head: a 64-token segment whose decay
    range exceeds the factorisation bound is scanned in several token ranges, the state renormalised at each
    range start.  Several chunks (look-back over predecessor states, or entering states past the look-back
    limit at chunk 64), a chunk of 11 segments (several decay blocks), a partial last segment and an optional
    initial state."""
    g = torch.Generator().manual_seed(N + chunk)
    b, L, H, P = 2, 650, 8, 64
    x = torch.randn(b, L, H, P, generator=g).to(torch.bfloat16)
    B = torch.randn(b, L, 1, N, generator=g).to(torch.bfloat16)
    C = torch.randn(b, L, 1, N, generator=g).to(torch.bfloat16)
    dt = torch.exp(torch.randn(b, L, H, generator=g) * 2.0)          # 0.02 .. 50
    A = torch.tensor([-16.0, -2.0, -0.5, -0.01, -4.0, -1.0, -0.1, -8.0])
    h0 = torch.randn(b, H, P, N, generator=g) if init else None
    say(f"extreme decay bf16 N={N} chunk={chunk} init={init}")
    y, fin = mh.selective_scan(dev(x, torch.bfloat16), dev(dt), dev(A), dev(B, torch.bfloat16),
                               dev(C, torch.bfloat16), None, return_final_state=True, chunk_size=chunk,
                               initial_state=dev(h0))
    y_ref, f_ref = ref.ssd_direct(x.double().numpy(), dt.double().numpy(), A.double().numpy(),
                                  B.double().numpy(), C.double().numpy(),
                                  initial_state=None if h0 is None else h0.double().numpy())
    check("y", y, y_ref, 1e-2)
    check("final", fin, f_ref, 1e-2)


@pytest.mark.parametrize("dtype,L,H,N,chunk", [(torch.bfloat16, 1000, 8, 128, 256), (torch.float32, 333, 4, 64, None),
                                               (torch.float32, 200, 2, 128, 64)])
def test_ssd_output_gate_vs_oracle(dtype, L, H, N, chunk):
    """Fused z-gate y * silu(z) (mamba2.py:337-338), z a strided slice of a wider buffer as in_proj gives it;
    partial last segments, several chunks, both the prefetched (bf16) and the at-store (fp32) gate loads."""
    g = torch.Generator().manual_seed(L + H)
    b, P = 2, 64
    d_inner = H * P
    x = torch.randn(b, L, H, P, generator=g).to(dtype)
    xz = torch.randn(b, L, 2 * d_inner, generator=g).to(dtype)      # [x' | z]: z is the second half
    B = torch.randn(b, L, 1, N, generator=g).to(dtype)
    C = torch.randn(b, L, 1, N, generator=g).to(dtype)
    dt = torch.rand(b, L, H, generator=g) * 0.2 + 0.01
    A = -torch.exp(torch.rand(H, generator=g) * 2.0)
    D = torch.randn(H, generator=g)
    zd = dev(xz, dtype)[..., d_inner:]
    say(f"output gate {dtype} L={L} H={H} N={N} chunk={chunk}")
    y, fin = mh.selective_scan(dev(x, dtype), dev(dt), dev(A), dev(B, dtype), dev(C, dtype), dev(D),
                               return_final_state=True, chunk_size=chunk, z=zd.reshape(b, L, H, P))
    y3 = mh.selective_scan(dev(x, dtype).reshape(b, L, d_inner), dev(dt), dev(A), dev(B, dtype), dev(C, dtype),
                           dev(D), chunk_size=chunk, z=zd)
    torch.cuda.synchronize()
    y_ref, f_ref = ref.ssd_direct(x.double().numpy(), dt.double().numpy(), A.double().numpy(), B.double().numpy(),
                                  C.double().numpy(), D.double().numpy())
    zr = xz[..., d_inner:].double().numpy().reshape(b, L, H, P)
    check("gated y", y, y_ref * (zr / (1.0 + np.exp(-zr))), TOL[dtype])
    check("final (not gated)", fin, f_ref, TOL[dtype])
    assert torch.equal(y3.view(b, L, H, P), y)


@pytest.mark.parametrize("N,G,dtype,h0,gate,dmode", [
    (16, 1, torch.bfloat16, False, False, "head"),       # the reference's scan fixture (tests/test_mamba2.py:22-30)
    (8, 1, torch.float32, True, False, "head"),          # its per-seqlen case (tests/test_mamba2.py:74-80)
    (32, 2, torch.float32, True, True, "channel"),       # the debug preset's d_state
    (96, 1, torch.bfloat16, True, False, None),          # padded to 128
    (256, 1, torch.bfloat16, True, True, "head"),        # two halves, B / C halves read in place
    (256, 2, torch.float32, True, True, "channel"),      # two halves through the workspace
    (200, 1, torch.float32, False, False, "head"),       # two halves, the second padded
], ids=lambda v: str(v).replace("torch.", ""))
def test_ssd_composed_dstate_vs_oracle(N, G, dtype, h0, gate, dmode):
    """dstate outside the kernels' 64 / 128 tiles: zero-padded or split into 128-column halves by the C ABI.
    y (gated or not), the final state and an initial state against the direct float64 recurrence."""
    g = torch.Generator().manual_seed(N * 7 + G)
    b, L, H, P = 2, 203, 4, 64
    x = torch.randn(b, L, H, P, generator=g).to(dtype)
    B = torch.randn(b, L, G, N, generator=g).to(dtype)
    C = torch.randn(b, L, G, N, generator=g).to(dtype)
    dt = torch.rand(b, L, H, generator=g) * 0.2 + 0.01
    A = -torch.exp(torch.rand(H, generator=g) * 2.0)
    D = None if dmode is None else torch.randn(H if dmode == "head" else H * P, generator=g)
    s0 = 0.3 * torch.randn(b, H, P, N, generator=g) if h0 else None
    z = torch.randn(b, L, H, P, generator=g).to(dtype) if gate else None
    say(f"composed dstate N={N} G={G} {dtype} h0={h0} gate={gate} D={dmode}")
    y, fin = mh.selective_scan(dev(x, dtype), dev(dt), dev(A), dev(B, dtype), dev(C, dtype), dev(D),
                               return_final_state=True, initial_state=dev(s0), z=dev(z, dtype), chunk_size=64)
    torch.cuda.synchronize()
    y_ref, f_ref = ref.ssd_direct(x.double().numpy(), dt.double().numpy(), A.double().numpy(), B.double().numpy(),
                                  C.double().numpy(), None if D is None else D.double().numpy(),
                                  initial_state=None if s0 is None else s0.double().numpy())
    if gate:
        zr = z.double().numpy()
        y_ref = y_ref * (zr / (1.0 + np.exp(-zr)))
    check("y", y, y_ref, TOL[dtype])
    check("final", fin, f_ref, TOL[dtype])
    assert fin.shape == (b, H, P, N)


def test_ssd_empty_sequence():
    h0 = torch.randn(1, 4, 64, 64, device="cuda")
    x = torch.zeros(1, 0, 4, 64, device="cuda")
    y, fin = mh.selective_scan(x, torch.zeros(1, 0, 4, device="cuda"), -torch.ones(4, device="cuda"),
                               torch.zeros(1, 0, 1, 64, device="cuda"), torch.zeros(1, 0, 1, 64, device="cuda"),
                               None, return_final_state=True, initial_state=h0)
    assert y.shape == (1, 0, 4, 64)
    assert torch.equal(fin, h0)


def test_ssd2_full_size_properties():
    """Benchmark shape ssd2 (b2 L4096 H64 P64 N128, bf16)."""
    inp = W.ssd_inputs(W.SSD2)
    say("ssd2 full: run")
    y, fin = run(inp, torch.bfloat16)
    # exact linearity: doubling x doubles every intermediate exactly (powers of two)
    inp2 = dict(inp, x=inp["x"] * 2)
    y2, fin2 = run(inp2, torch.bfloat16)
    say("ssd2 full: linearity")
    assert torch.equal(y2, y * 2) and torch.equal(fin2, fin * 2)
    # chunk-length invariance
    y3, fin3 = run(inp, torch.bfloat16, chunk=1024)
    check("chunk 1024 vs auto y", y3, host(y), 1e-2)
    # each chunking is within ~2e-3 of the float64 oracle (bf16 operands); they need not agree bit for bit
    check("chunk 1024 vs auto final", fin3, host(fin), 1e-2)
    # split-sequence state carry
    half = {k: (v[:, :2048] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
    ya, fa = run(half, torch.bfloat16)
    rest = {k: (v[:, 2048:] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
    rest["initial_state"] = fa.cpu()
    yb, fb = run(rest, torch.bfloat16)
    check("split y", torch.cat([ya, yb], 1), host(y), 1e-2)
    check("split final", fb, host(fin), 1e-2)
    # leading slice against the oracle (y is causal)
    n = 512
    arr = {k: (None if v is None else v.to(torch.float64).numpy()) for k, v in inp.items()}
    y_ref, _ = ref.ssd_chunked(arr["x"][:, :n], arr["dt"][:, :n], arr["A"], arr["B"][:, :n], arr["C"][:, :n],
                               arr["D"], chunk_size=128)
    check("ssd2 y[:512] vs oracle", y[:, :n], y_ref, 1e-2)
    # trailing slice from the GPU's own carried state
    ya, fa = run({k: (v[:, :-n] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}, torch.bfloat16)
    y_ref, f_ref = ref.ssd_chunked(arr["x"][:, -n:], arr["dt"][:, -n:], arr["A"], arr["B"][:, -n:],
                                   arr["C"][:, -n:], arr["D"], initial_state=host(fa), chunk_size=128)
    check("ssd2 y[-512:] vs oracle", y[:, -n:], y_ref, 1e-2)
    check("ssd2 final vs oracle", fin, f_ref, 1e-2)


def test_ssd4_full_size_properties():
    """Benchmark shape ssd4 (b1 L131072 H128 G8, bf16, initial state), inputs drawn on the GPU."""
    cfg = W.SSD4
    inp = W.ssd_inputs(cfg, device="cuda")
    say("ssd4 full: run")
    y, fin = mh.selective_scan(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"],
                               return_final_state=True, initial_state=inp["initial_state"])
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(fin).all()
    n = 512
    arr = {k: host(v) for k, v in inp.items()}
    y_ref, _ = ref.ssd_chunked(arr["x"][:, :n], arr["dt"][:, :n], arr["A"], arr["B"][:, :n], arr["C"][:, :n],
                               arr["D"], initial_state=arr["initial_state"], chunk_size=128)
    check("ssd4 y[:512] vs oracle", y[:, :n], y_ref, 1e-2)
    L = cfg.seqlen
    ya, fa = mh.selective_scan(inp["x"][:, :L - n], inp["dt"][:, :L - n], inp["A"], inp["B"][:, :L - n],
                               inp["C"][:, :L - n], inp["D"], return_final_state=True,
                               initial_state=inp["initial_state"])
    y_ref, f_ref = ref.ssd_chunked(arr["x"][:, -n:], arr["dt"][:, -n:], arr["A"], arr["B"][:, -n:],
                                   arr["C"][:, -n:], arr["D"], initial_state=host(fa), chunk_size=128)
    check("ssd4 y[-512:] vs oracle", y[:, -n:], y_ref, 1e-2)
    check("ssd4 final vs oracle", fin, f_ref, 1e-2)
    check("ssd4 prefix consistency", ya, host(y[:, :L - n]), 1e-2)
