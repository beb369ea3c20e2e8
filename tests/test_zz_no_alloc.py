"""The no-allocation SSD prefill entry point (mh_ssd_chunk_scan_fwd_noalloc) through the C ABI.

It runs the prefill kernels on the library's static device scratch instead of a caller workspace, so its
outputs must equal those of mh_ssd_chunk_scan_fwd (caller workspace) bit for bit.  Two calls in a row, the
second on a smaller problem (the scratch keeps the first call's contents), each against the workspace entry
point on the same inputs; and the entry point captured in a HIP graph (after one call outside capture on the
device, as the header asks) and replayed, every replay bit-identical to the workspace entry point.
"""

import ctypes as ct

import pytest
import torch

from mamformer_amd import _lib, ops
from mamformer_amd import workloads as W
from tests.gpu_helpers import say

pytestmark = pytest.mark.gpu


def _run(entry, inp, cfg, z=None):
    b, L, H, P, N, G = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate, cfg.ngroups
    y = torch.full((b, L, H, P), float("nan"), device="cuda", dtype=cfg.dtype)
    fin = torch.full((b, H, P, N), float("nan"), device="cuda", dtype=torch.float32)
    a = ops._ssd_args(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], None, False, None,
                      inp["initial_state"], y, fin, None, z)
    ws = None
    if entry == "mh_ssd_chunk_scan_fwd":
        n = ct.c_size_t()
        _lib.call("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n))
        ws = torch.empty(n.value, device="cuda", dtype=torch.uint8)
        a.workspace, a.workspace_bytes = ws.data_ptr(), n.value
    _lib.call(entry, ct.byref(a), ops._stream(y.device))
    torch.cuda.synchronize()
    return y, fin


def _case(cfg, gate):
    inp = W.ssd_inputs(cfg, device="cuda")
    z = torch.randn(inp["x"].shape, device="cuda").to(cfg.dtype) if gate else None
    n = ct.c_size_t()
    a = ops._ssd_args(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], None, False, None,
                      inp["initial_state"], inp["x"], None, None)
    _lib.call("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n))
    say(f"noalloc {cfg.name} b{cfg.batch} L{cfg.seqlen} H{cfg.nheads} N{cfg.dstate} G{cfg.ngroups} "
        f"h0={cfg.init_state} gate={gate} workspace={n.value} of {_lib.NOALLOC_SCRATCH_BYTES}")
    assert n.value <= _lib.NOALLOC_SCRATCH_BYTES
    y0, f0 = _run("mh_ssd_chunk_scan_fwd", inp, cfg, z)
    y1, f1 = _run("mh_ssd_chunk_scan_fwd_noalloc", inp, cfg, z)
    assert torch.isfinite(y0.float()).all() and torch.isfinite(f0).all()
    assert torch.equal(y0, y1), "y differs between the workspace and no-allocation entry points"
    assert torch.equal(f0, f1), "final state differs between the workspace and no-allocation entry points"


def test_noalloc_equals_workspace_entry_two_calls():
    # the headline shape first, then a smaller problem with two groups, an initial state and the gate
    _case(W.SSD2, gate=False)
    _case(W.SSD2.scaled(name="small", seqlen=777, nheads=16, ngroups=2, seed=11, init_state=True), gate=True)


def test_noalloc_under_graph_capture_replays_bit_identical():
    cfg = W.SSD2.scaled(name="graph", seqlen=640, nheads=16, ngroups=2, seed=5, init_state=True)
    inp = W.ssd_inputs(cfg, device="cuda")
    b, L, H, P, N = cfg.batch, cfg.seqlen, cfg.nheads, cfg.headdim, cfg.dstate
    say(f"noalloc graph capture b{b} L{L} H{H} N{N} G{cfg.ngroups}")
    y0, f0 = _run("mh_ssd_chunk_scan_fwd", inp, cfg)
    _run("mh_ssd_chunk_scan_fwd_noalloc", inp, cfg)          # the first call on the device, outside capture
    y = torch.empty((b, L, H, P), device="cuda", dtype=cfg.dtype)
    fin = torch.empty((b, H, P, N), device="cuda", dtype=torch.float32)
    a = ops._ssd_args(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], None, False, None,
                      inp["initial_state"], y, fin, None, None)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            _lib.call("mh_ssd_chunk_scan_fwd_noalloc", ct.byref(a), ops._stream(y.device))
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        y.fill_(float("nan"))
        fin.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say(f"noalloc graph replay {rep}")
        assert torch.equal(y, y0), f"replay {rep}: y differs from the workspace entry point"
        assert torch.equal(fin, f0), f"replay {rep}: final state differs from the workspace entry point"
