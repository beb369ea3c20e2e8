"""C ABI of libmamformer_hip.so on the CPU host: loads, exports every declared symbol,
and rejects bad arguments before any HIP call (no compute is launched here)."""

import ctypes as ct
import re
from pathlib import Path

import pytest
import torch

import mamformer_amd
from mamformer_amd import _lib
from mamformer_amd._lib import SsdBwdArgs, Conv1dArgs, Conv1dBwdArgs, KdaArgs, KdaBwdArgs, SsdArgs, SsuArgs

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "mamformer_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|size_t)\s+(mh_\w+)\s*\(", text, re.M)))


def test_library_loads_and_exports_every_header_symbol():
    h = _lib.lib()
    syms = declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(h, s), s
    assert set(syms) == set(_lib.EXPORTS)
    assert h.mh_abi_version() == _lib.ABI_VERSION


def _good_ssd():
    a = SsdArgs()
    b, L, H, P, N, G = 2, 300, 8, 64, 128, 2
    a.batch, a.seqlen, a.nheads, a.headdim, a.dstate, a.ngroups = b, L, H, P, N, G
    a.dtype = _lib.MH_BF16
    fake = ct.c_void_p(4096)
    a.x = a.B = a.C = a.y = a.dt = a.A = fake
    a.x_stride_h = a.y_stride_h = P
    a.x_stride_l = a.y_stride_l = H * P
    a.x_stride_b = a.y_stride_b = L * H * P
    a.B_stride_l = a.C_stride_l = G * N
    a.B_stride_b = a.C_stride_b = L * G * N
    a.dt_stride_l, a.dt_stride_b = H, L * H
    return a


def _rc(fn, *args):
    return getattr(_lib.lib(), fn)(*args)


def test_ssd_workspace_and_chunk_len():
    a = _good_ssd()
    n = ct.c_size_t()
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    cl = ct.c_int64()
    assert _rc("mh_ssd_chunk_len", ct.byref(a), ct.byref(cl)) == 0
    nch = -(-300 // cl.value)
    # at least the bf16 chunk states (b, nchunks, H, P, N) and the fp32 chunk log-decays (b, H, nchunks)
    assert n.value >= 2 * nch * 8 * 64 * 128 * 2 + 2 * 8 * nch * 4
    a.chunk_len = 128
    assert _rc("mh_ssd_chunk_len", ct.byref(a), ct.byref(cl)) == 0 and cl.value == 128


@pytest.mark.parametrize("field,value,code", [
    ("headdim", 32, -6), ("dstate", 100, -6), ("dstate", 264, -6), ("dtype", 7, -3), ("ngroups", 3, -2), ("batch", 0, -2),
    ("chunk_len", 100, -2), ("x_stride_l", 8 * 64 + 1, -5), ("B_stride_l", 64, -4),
])
def test_ssd_rejects_bad_arguments(field, value, code):
    a = _good_ssd()
    setattr(a, field, value)
    n = ct.c_size_t()
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == code
    assert _lib.lib().mh_last_error()


@pytest.mark.parametrize("N", [8, 16, 32, 96, 200, 256])
def test_ssd_composed_dstate_workspace(N):
    """dstate outside the 64 / 128 tiles is accepted; its workspace holds an inner run's plus the pieces of B, C
    and the states; the no-allocation entry point declines it (MH_ERR_UNSUPPORTED) before any HIP call."""
    a = _good_ssd()
    G, L, b = a.ngroups, a.seqlen, a.batch
    a.dstate = N
    a.B_stride_l = a.C_stride_l = G * N
    a.B_stride_b = a.C_stride_b = L * G * N
    n = ct.c_size_t()
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    ni = 64 if N <= 64 else 128
    a2 = _good_ssd()
    a2.dstate = ni
    a2.B_stride_l = a2.C_stride_l = G * ni
    a2.B_stride_b = a2.C_stride_b = L * G * ni
    n2 = ct.c_size_t()
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a2), ct.byref(n2)) == 0
    assert n.value >= n2.value + 2 * b * L * G * ni * 2       # inner run + B and C pieces (bf16)
    assert _rc("mh_ssd_chunk_scan_fwd_noalloc", ct.byref(a), None) == -6
    assert b"composition" in _lib.lib().mh_last_error()


def test_ssd_rejects_null_and_misaligned_pointers_and_small_workspace():
    a = _good_ssd()
    a.C = None
    assert _rc("mh_ssd_chunk_scan_fwd", ct.byref(a), None) == -1
    a = _good_ssd()
    a.y = ct.c_void_p(4096 + 2)
    assert _rc("mh_ssd_chunk_scan_fwd", ct.byref(a), None) == -5
    a = _good_ssd()
    a.workspace, a.workspace_bytes = ct.c_void_p(8192), 16
    assert _rc("mh_ssd_chunk_scan_fwd", ct.byref(a), None) == -7
    assert b"workspace" in _lib.lib().mh_last_error()
    assert _rc("mh_ssd_chunk_scan_fwd", None, None) == -1


def test_ssd_noalloc_validates_and_rejects_sizes_beyond_its_static_scratch():
    # the 128K shape of the benchmark (b1 L131072 H128 N128 G8) in 4096-token chunks needs more workspace than
    # the scratch
    a = _good_ssd()
    b, L, H, P, N, G = 1, 131072, 128, 64, 128, 8
    a.batch, a.seqlen, a.nheads, a.ngroups, a.chunk_len = b, L, H, G, 4096
    a.x_stride_l = a.y_stride_l = H * P
    a.x_stride_b = a.y_stride_b = L * H * P
    a.B_stride_l = a.C_stride_l = G * N
    a.B_stride_b = a.C_stride_b = L * G * N
    a.dt_stride_l, a.dt_stride_b = H, L * H
    n = ct.c_size_t()
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    assert n.value > _lib.NOALLOC_SCRATCH_BYTES
    assert _rc("mh_ssd_chunk_scan_fwd_noalloc", ct.byref(a), None) == -7
    assert b"static" in _lib.lib().mh_last_error()
    # argument checks come first, exactly as for the workspace entry point
    a = _good_ssd()
    a.C = None
    assert _rc("mh_ssd_chunk_scan_fwd_noalloc", ct.byref(a), None) == -1
    assert _rc("mh_ssd_chunk_scan_fwd_noalloc", None, None) == -1


def test_ssd_and_state_update_validate_the_output_gate():
    a = _good_ssd()
    a.z, a.z_stride_b, a.z_stride_l, a.z_stride_h = ct.c_void_p(4096), a.y_stride_b, a.y_stride_l, a.y_stride_h
    n = ct.c_size_t()
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    a.z = ct.c_void_p(4096 + 8)
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == -5
    a.z = ct.c_void_p(4096)
    a.z_stride_h = 32
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == -4
    a.z_stride_h, a.z_stride_l = 64, 8 * 64 + 4
    assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == -5
    u = _good_ssu()
    u.z, u.z_stride_b = ct.c_void_p(4096), 8 * 64 - 1
    assert _rc("mh_ssd_state_update", ct.byref(u), None) == -4
    assert b"z" in _lib.lib().mh_last_error()


def _good_ssu():
    a = SsuArgs()
    a.batch, a.nheads, a.headdim, a.dstate, a.ngroups = 4, 8, 64, 128, 1
    a.dtype = _lib.MH_BF16
    a.state_in = a.state_out = ct.c_void_p(1 << 20)
    a.x = a.dt = a.A = a.B = a.C = a.y = ct.c_void_p(4096)
    a.x_stride_b = a.y_stride_b = 8 * 64
    a.B_stride_b = a.C_stride_b = 128
    a.dt_stride_b = 8
    return a


@pytest.mark.parametrize("field,value,code", [
    ("dstate", 48, -6), ("ngroups", 3, -2), ("dtype", 5, -3), ("x_stride_b", 10, -4), ("nheads", 0, -2),
])
def test_state_update_rejects_bad_arguments(field, value, code):
    a = _good_ssu()
    setattr(a, field, value)
    assert _rc("mh_ssd_state_update", ct.byref(a), None) == code


def test_state_update_rejects_partial_overlap():
    a = _good_ssu()
    a.state_out = ct.c_void_p((1 << 20) + 4096)
    assert _rc("mh_ssd_state_update", ct.byref(a), None) == -4


def test_kda_rejects_bad_arguments():
    a = KdaArgs()
    a.batch, a.nheads, a.seqlen, a.dk, a.dv = 1, 2, 10, 128, 128
    a.dtype = _lib.MH_BF16
    a.q1 = a.q2 = a.k = a.v = a.o = ct.c_void_p(4096)
    a.dk = 96                             # head sizes 64 and 128 (each of dk, dv) only
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -6
    a.dk, a.dv = 128, 256
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -6
    a.dv = 128
    a.v = None
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -1
    a.v = ct.c_void_p(4096)
    a.dtype = 5
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -3


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 64, 64)
    dt = torch.zeros(1, 64, 1)
    with pytest.raises(RuntimeError, match="no CPU path"):
        mamformer_amd.selective_scan(x, dt, torch.zeros(1), torch.zeros(1, 64, 64), torch.zeros(1, 64, 64), None)
    with pytest.raises(RuntimeError, match="no CPU path"):
        mamformer_amd.linear_attn_scan(*(torch.zeros(1, 1, 4, 128) for _ in range(4)))


def test_chunk_len_auto_choice():
    assert mamformer_amd.ssd_chunk_len(2, 4096, 64, 64, 128, 1) % 64 == 0
    assert mamformer_amd.ssd_chunk_len(1, 131072, 128, 64, 128, 8) == 16384
    assert mamformer_amd.ssd_chunk_len(1, 512, 8, 64, 64, 1, chunk_size=128) == 128


def test_kda_reference_mode_validation():
    a = KdaArgs()
    a.batch, a.nheads, a.seqlen, a.dk, a.dv = 1, 2, 10, 128, 128
    a.dtype = _lib.MH_BF16
    a.mode = _lib.MH_KDA_REFERENCE
    a.q1 = a.k = a.v = a.o = ct.c_void_p(4096)
    a.kernel_dim = 0
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -2          # kernel_dim must be positive
    a.kernel_dim = 128
    a.g = ct.c_void_p(4096)
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -2          # no gate in reference mode
    a.g = None
    a.o2 = ct.c_void_p(4096)
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -1          # o2 without q2
    a.mode = 7
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(a), None) == -6
    g = KdaArgs()
    g.batch, g.nheads, g.seqlen, g.dk, g.dv = 1, 2, 10, 128, 128
    g.dtype = _lib.MH_BF16
    g.q1 = g.k = g.v = g.o = ct.c_void_p(4096)
    g.final_z = ct.c_void_p(4096)
    assert _rc("mh_kda_chunk_scan_fwd", ct.byref(g), None) == -2          # z outputs belong to reference mode


def _good_step():
    a = _lib.KdaStepArgs()
    a.batch, a.nheads, a.dk, a.dv = 2, 4, 128, 128
    a.dtype = _lib.MH_BF16
    a.flags = _lib.MH_KDA_PHI
    a.kernel_dim = 128
    a.q1 = a.q2 = a.k = a.v = a.o = ct.c_void_p(4096)
    a.state = a.z = ct.c_void_p(8192)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("dv", 96, -6), ("dk", 256, -6), ("kernel_dim", 0, -2), ("dtype", 5, -3), ("batch", 0, -2),
    ("state", None, -1), ("z", None, -1), ("q1", None, -1), ("state", 8196, -5),
])
def test_kda_step_rejects_bad_arguments(field, value, code):
    a = _good_step()
    setattr(a, field, ct.c_void_p(value) if field in ("state", "z", "q1") and value is not None else value)
    assert _rc("mh_kda_recurrent_step", ct.byref(a), None) == code


def test_kda_step_o2_needs_q2():
    a = _good_step()
    a.q2 = None
    a.o2 = ct.c_void_p(4096)
    assert _rc("mh_kda_recurrent_step", ct.byref(a), None) == -1


def _good_conv():
    a = Conv1dArgs()
    a.batch, a.seqlen, a.dim, a.width = 2, 50, 256, 4
    a.dtype = _lib.MH_BF16
    fake = ct.c_void_p(4096)
    a.x = a.y = a.weight = fake
    a.x_stride_l = a.y_stride_l = 256
    a.x_stride_b = a.y_stride_b = 50 * 256
    return a


@pytest.mark.parametrize("field,value,code", [
    ("width", 9, -6), ("dim", 12, -6), ("dtype", 5, -3), ("batch", 0, -2), ("conv_state_len", 4, -2),
    ("x_stride_l", 100, -5), ("y_stride_l", 128, -4),
])
def test_conv1d_rejects_bad_arguments(field, value, code):
    a = _good_conv()
    setattr(a, field, value)
    assert _rc("mh_causal_conv1d_fwd", ct.byref(a), None) == code
    assert _lib.lib().mh_last_error()


def test_conv1d_rejects_missing_conv_state():
    a = _good_conv()
    a.conv_state_len = 2
    assert _rc("mh_causal_conv1d_fwd", ct.byref(a), None) == -1


def _good_bwd():
    a = SsdBwdArgs()
    a.fwd = _good_ssd()
    f = a.fwd
    P, H, L, G, N = 64, f.nheads, f.seqlen, f.ngroups, f.dstate
    fake = ct.c_void_p(8192)
    a.dy = a.dx = a.ddt = a.dA = a.dB = a.dC = fake
    a.dy_stride_h = a.dx_stride_h = P
    a.dy_stride_l = a.dx_stride_l = H * P
    a.dy_stride_b = a.dx_stride_b = L * H * P
    a.ddt_stride_l, a.ddt_stride_b = H, L * H
    a.dB_stride_l = a.dC_stride_l = G * N
    a.dB_stride_b = a.dC_stride_b = L * G * N
    return a


def test_ssd_bwd_workspace_and_validation():
    a = _good_bwd()
    n = ct.c_size_t()
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    nseg = -(-300 // 64)
    # entering state and adjoint per segment (bf16), plus the fp32 (b, L, G, N) partial sums of dB and dC
    assert n.value >= 2 * 2 * nseg * 8 * 64 * 128 * 2 + 2 * 2 * 300 * 2 * 128 * 4
    a.fwd.y = None                                       # the forward output is not needed
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    a.fwd.chunk_len = 100                                # ignored: the backward uses 64-token segments
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0


@pytest.mark.parametrize("mutate,code,word", [
    (lambda a: setattr(a.fwd, "z", ct.c_void_p(4096)), -6, b"gate"),
    (lambda a: setattr(a.fwd, "B_stride_l", 0), -6, b"broadcast"),
    (lambda a: setattr(a, "dy", None), -1, b"dy"),
    (lambda a: setattr(a, "dA", None), -1, b"dA"),
    (lambda a: setattr(a.fwd, "D", ct.c_void_p(4096)), -1, b"dD"),
    (lambda a: setattr(a, "dB", ct.c_void_p(8192 + 4)), -5, b"aligned"),
    (lambda a: setattr(a, "dx_stride_h", 32), -4, b"head stride"),
    (lambda a: setattr(a, "dC_stride_l", 64), -4, b"token stride"),
    (lambda a: setattr(a.fwd, "dstate", 100), -6, b"dstate"),
])
def test_ssd_bwd_rejects_bad_arguments(mutate, code, word):
    a = _good_bwd()
    mutate(a)
    n = ct.c_size_t()
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == code
    assert word in _lib.lib().mh_last_error()
    assert _rc("mh_ssd_chunk_scan_bwd", ct.byref(a), None) == code


def test_ssd_bwd_rejects_small_workspace():
    a = _good_bwd()
    a.workspace, a.workspace_bytes = ct.c_void_p(8192), 64
    assert _rc("mh_ssd_chunk_scan_bwd", ct.byref(a), None) == -7
    assert _rc("mh_ssd_chunk_scan_bwd", None, None) == -1


def _good_conv_bwd():
    q = Conv1dBwdArgs()
    q.fwd = _good_conv()
    q.fwd.y = None                                       # the forward output is not an input of the backward
    q.fwd.y_stride_b = q.fwd.y_stride_l = 0
    fake = ct.c_void_p(8192)
    q.dy = q.dx = q.dweight = fake
    q.dy_stride_l = q.dx_stride_l = 256
    q.dy_stride_b = q.dx_stride_b = 50 * 256
    return q


def test_conv1d_bwd_workspace():
    q = _good_conv_bwd()
    n = ct.c_size_t()
    assert _rc("mh_conv1d_bwd_workspace_bytes", ct.byref(q), ct.byref(n)) == 0
    # one fp32 (dweight, dbias) partial per (batch, 32-token run)
    assert n.value == 2 * 2 * 256 * (4 + 1) * 4
    q.fwd.seqlen = 0
    assert _rc("mh_conv1d_bwd_workspace_bytes", ct.byref(q), ct.byref(n)) == 0 and n.value == 0


@pytest.mark.parametrize("mutate,code,word", [
    (lambda q: setattr(q, "dweight", None), -1, b"dweight"),
    (lambda q: setattr(q, "dy", None), -1, b"dy"),
    (lambda q: setattr(q.fwd, "bias", ct.c_void_p(4096)), -1, b"dbias"),
    (lambda q: setattr(q, "dx", ct.c_void_p(8192 + 4)), -5, b"aligned"),
    (lambda q: setattr(q, "dy_stride_l", 100), -5, b"16 bytes"),
    (lambda q: setattr(q, "dx_stride_l", 128), -4, b"token stride"),
    (lambda q: setattr(q.fwd, "width", 9), -6, b"width"),
])
def test_conv1d_bwd_rejects_bad_arguments(mutate, code, word):
    q = _good_conv_bwd()
    mutate(q)
    n = ct.c_size_t()
    assert _rc("mh_conv1d_bwd_workspace_bytes", ct.byref(q), ct.byref(n)) == code
    assert word in _lib.lib().mh_last_error()
    assert _rc("mh_causal_conv1d_bwd", ct.byref(q), None) == code


def test_conv1d_bwd_rejects_small_workspace():
    q = _good_conv_bwd()
    q.workspace, q.workspace_bytes = ct.c_void_p(8192), 64
    assert _rc("mh_causal_conv1d_bwd", ct.byref(q), None) == -7
    assert _rc("mh_causal_conv1d_bwd", None, None) == -1


def _good_kda_bwd(diff=True):
    a = KdaBwdArgs()
    f = a.fwd
    f.batch, f.nheads, f.seqlen, f.dk, f.dv = 2, 4, 300, 128, 128
    f.dtype, f.mode, f.kernel_dim, f.lam = _lib.MH_BF16, _lib.MH_KDA_REFERENCE, 128, 0.8
    fake = ct.c_void_p(4096)
    f.q1 = f.q2 = f.k = f.v = fake
    a.flags = _lib.MH_KDA_BWD_DIFF if diff else 0
    a.do1 = a.dq1 = a.dq2 = a.dk = a.dv = ct.c_void_p(8192)
    return a


def test_kda_bwd_workspace():
    a = _good_kda_bwd()
    n = ct.c_size_t()
    assert _rc("mh_kda_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    # n_t and dn_t per (query, b, h, token), per-(b, h) lambda partial sums (two queries and the baseline), and
    # two adjoint-state sums (128 x 128 + 128) per reverse-walk segment and (b, h) (one segment: 5 chunks)
    assert n.value == (2 * 2 * 8 * 300 + 3 * 8 + 2 * 8 * (128 * 128 + 128)) * 4
    a.fwd.seqlen = 0
    assert _rc("mh_kda_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0


@pytest.mark.parametrize("mutate,code,word", [
    (lambda a: setattr(a.fwd, "mode", _lib.MH_KDA_GATED), -6, b"reference mode"),
    (lambda a: setattr(a, "do1", None), -1, b"do1"),
    (lambda a: setattr(a, "dk", None), -1, b"dk"),
    (lambda a: setattr(a.fwd, "q2", None), -1, b"q2"),
    (lambda a: setattr(a, "do2", ct.c_void_p(4096)), -2, b"do2"),
    (lambda a: setattr(a, "flags", 6), -6, b"flags"),
    (lambda a: setattr(a, "dv", ct.c_void_p(8192 + 8)), -5, b"aligned"),
    (lambda a: setattr(a.fwd, "dk", 96), -6, b"dk"),
])
def test_kda_bwd_rejects_bad_arguments(mutate, code, word):
    a = _good_kda_bwd()
    mutate(a)
    n = ct.c_size_t()
    assert _rc("mh_kda_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == code
    assert word in _lib.lib().mh_last_error()
    assert _rc("mh_kda_chunk_scan_bwd", ct.byref(a), None) == code


def test_kda_bwd_rejects_small_workspace():
    a = _good_kda_bwd(diff=False)
    a.workspace, a.workspace_bytes = ct.c_void_p(8192), 64
    assert _rc("mh_kda_chunk_scan_bwd", ct.byref(a), None) == -7


def test_flag_values_match_the_header():
    """Every MH_* enum value the Python side uses equals the header's."""
    import re
    text = (Path(__file__).resolve().parents[1] / "include" / "mamformer_hip.h").read_text()
    vals = {m.group(1): int(m.group(2)) for m in re.finditer(r"\b(MH_[A-Z0-9_]+)\s*=\s*(-?\d+)", text)}
    for name in ("MH_F32", "MH_BF16", "MH_DT_SOFTPLUS", "MH_DT_LIMIT", "MH_D_PER_CHANNEL", "MH_A_PER_STATE",
                 "MH_DT_PER_CHANNEL", "MH_KDA_GATED", "MH_KDA_REFERENCE", "MH_KDA_PHI", "MH_KDA_BWD_DIFF",
                 "MH_CONV_SILU"):
        assert vals[name] == getattr(_lib, name), name


def test_prefill_rejects_decode_only_flags():
    for flag in (_lib.MH_A_PER_STATE, _lib.MH_DT_PER_CHANNEL):
        a = _good_ssd()
        a.flags = flag
        n = ct.c_size_t()
        assert _rc("mh_ssd_workspace_bytes", ct.byref(a), ct.byref(n)) == -6
        assert b"decode" in _lib.lib().mh_last_error()


def test_state_update_per_channel_dt_needs_a_row_of_steps():
    a = _good_ssu()
    a.flags = _lib.MH_DT_PER_CHANNEL
    a.dt_stride_b = a.nheads                  # one step per head is too short a row for per-channel steps
    assert _rc("mh_ssd_state_update", ct.byref(a), None) == -4


def _good_hs_bwd():
    a = _lib.SsdHsBwdArgs()
    a.fwd = _good_ssd()
    fake = ct.c_void_p(4096)
    a.dhs = a.dx = a.ddt = a.dA = a.dB = fake
    return a


def test_h_states_workspace_and_bwd_validation():
    a = _good_ssd()
    n, nb = ct.c_size_t(), ct.c_size_t()
    assert _rc("mh_ssd_h_states_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    g = _good_hs_bwd()
    assert _rc("mh_ssd_h_states_bwd_workspace_bytes", ct.byref(g), ct.byref(nb)) == 0
    # forward: per-segment state sums (b, nseg, H, N), decays, e^c per (token, head) and the in-segment weights
    # (b, nseg, G, 32, 32); backward: the state sums twice (forward and adjoint), decays, xs per (token, head)
    b, L, H, N, G = 2, 300, 8, 128, 2
    nseg = -(-L // 32)
    assert n.value >= 4 * (b * nseg * H * N + b * nseg * H + b * L * H + b * nseg * G * 32 * 32)
    assert nb.value >= 4 * (2 * b * nseg * H * N + b * nseg * H + b * L * H)
    g.dA = None
    assert _rc("mh_ssd_h_states_bwd", ct.byref(g), None) == -1
    g = _good_hs_bwd()
    g.fwd.dt_bias = ct.c_void_p(4096)            # d_dt_bias required with dt_bias
    assert _rc("mh_ssd_h_states_bwd", ct.byref(g), None) == -1
    assert b"d_dt_bias" in _lib.lib().mh_last_error()
    g = _good_hs_bwd()
    g.fwd.dstate, g.fwd.B_stride_l, g.fwd.C_stride_l = 256, 2 * 256, 2 * 256
    g.fwd.B_stride_b = g.fwd.C_stride_b = 300 * 2 * 256
    assert _rc("mh_ssd_h_states_bwd_workspace_bytes", ct.byref(g), ct.byref(nb)) == -6
    g = _good_hs_bwd()
    g.dx = ct.c_void_p(4100)
    assert _rc("mh_ssd_h_states_bwd", ct.byref(g), None) == -5
    g = _good_hs_bwd()
    g.workspace, g.workspace_bytes = ct.c_void_p(4096), 16
    assert _rc("mh_ssd_h_states_bwd", ct.byref(g), None) == -7
    # dx_rows in place of dx: dx may then be NULL; dx_rows needs 4-byte alignment
    g = _good_hs_bwd()
    g.dx, g.dx_rows = None, ct.c_void_p(4096)
    assert _rc("mh_ssd_h_states_bwd_workspace_bytes", ct.byref(g), ct.byref(nb)) == 0
    g.dx_rows = ct.c_void_p(4098)
    assert _rc("mh_ssd_h_states_bwd_workspace_bytes", ct.byref(g), ct.byref(nb)) == -5
    g.dx_rows = None
    assert _rc("mh_ssd_h_states_bwd_workspace_bytes", ct.byref(g), ct.byref(nb)) == -1


def test_scan_bwd_dx_rows_alignment():
    a = _lib.SsdBwdArgs()
    a.fwd = _good_ssd()
    fake = ct.c_void_p(4096)
    a.dy = a.dx = a.ddt = a.dA = a.dB = a.dC = fake
    b, L, H, P, N, G = 2, 300, 8, 64, 128, 2
    a.dy_stride_h = a.dx_stride_h = P
    a.dy_stride_l = a.dx_stride_l = H * P
    a.dy_stride_b = a.dx_stride_b = L * H * P
    a.ddt_stride_l, a.ddt_stride_b = H, L * H
    a.dB_stride_l = a.dC_stride_l = G * N
    a.dB_stride_b = a.dC_stride_b = L * G * N
    n = ct.c_size_t()
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    a.dx_rows = ct.c_void_p(4096)
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == 0
    a.dx_rows = ct.c_void_p(4097)
    assert _rc("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(n)) == -5


def _good_ref():
    """Arguments of the reference-form scan: (b, L, d_inner) rows as H heads of P channels, one B / C group, dt per
    channel, A per state."""
    a = SsdArgs()
    b, L, H, P, N = 2, 100, 4, 16, 32
    di = H * P
    a.batch, a.seqlen, a.nheads, a.headdim, a.dstate, a.ngroups = b, L, H, P, N, 1
    a.dtype = _lib.MH_BF16
    a.flags = _lib.MH_A_PER_STATE | _lib.MH_DT_PER_CHANNEL
    fake = ct.c_void_p(4096)
    a.x = a.B = a.C = a.y = a.dt = a.A = fake
    a.x_stride_h = a.y_stride_h = P
    a.x_stride_l = a.y_stride_l = a.dt_stride_l = di
    a.x_stride_b = a.y_stride_b = a.dt_stride_b = L * di
    a.B_stride_l = a.C_stride_l = N
    a.B_stride_b = a.C_stride_b = L * N
    return a


def test_ref_scan_bwd_validation_and_workspace():
    g = _lib.SsdRefBwdArgs()
    g.fwd = _good_ref()
    fake = ct.c_void_p(4096)
    g.dy = g.dx = g.ddt = g.dA = g.dB = g.dC = fake
    n = ct.c_size_t()
    assert _rc("mh_ssd_ref_scan_bwd_workspace_bytes", ct.byref(g), ct.byref(n)) == 0
    # the state at every 16th token (b, ceil(L / 16), d_inner, N) fp32 plus the channel-block partials
    b, L, di, N = 2, 100, 64, 32
    assert n.value >= 4 * (b * -(-L // 16) * di * N + 2 * b * L * N + b * N + 2 * b * di)
    g.fwd.z = fake                                   # the gate's backward is mh_silu_gate_bwd
    assert _rc("mh_ssd_ref_scan_bwd_workspace_bytes", ct.byref(g), ct.byref(n)) == -6
    g.fwd.z = None
    g.dA = None
    assert _rc("mh_ssd_ref_scan_bwd", ct.byref(g), None) == -1
    g.dA = fake
    g.fwd.D = fake                                   # dD required with D
    assert _rc("mh_ssd_ref_scan_bwd", ct.byref(g), None) == -1
    g.fwd.D = None
    g.dx = ct.c_void_p(4097)                         # bf16 elements: 2-byte alignment
    assert _rc("mh_ssd_ref_scan_bwd", ct.byref(g), None) == -5
    g.dx = fake
    g.workspace, g.workspace_bytes = fake, 16
    assert _rc("mh_ssd_ref_scan_bwd", ct.byref(g), None) == -7
    g.fwd.flags = 0                                  # the head form is not the reference form
    assert _rc("mh_ssd_ref_scan_bwd_workspace_bytes", ct.byref(g), ct.byref(n)) < 0
    assert b"reference form" in _lib.lib().mh_last_error()
