"""ctypes binding of libmamformer_hip.so (C ABI in include/mamformer_hip.h).

The library is loaded lazily on first use and there is no fallback: if the
shared library is missing or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes as ct
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmamformer_hip.so"

ABI_VERSION = 11

# bytes of the static device scratch behind mh_ssd_chunk_scan_fwd_noalloc (MH_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 64 << 20

MH_F32, MH_BF16 = 0, 1
MH_DT_SOFTPLUS, MH_DT_LIMIT, MH_D_PER_CHANNEL, MH_A_PER_STATE, MH_DT_PER_CHANNEL = 1, 2, 4, 8, 16
MH_KDA_GATED, MH_KDA_REFERENCE = 0, 1
MH_KDA_PHI = 1

ERRORS = {
    -1: "MH_ERR_NULL", -2: "MH_ERR_SHAPE", -3: "MH_ERR_DTYPE", -4: "MH_ERR_STRIDE",
    -5: "MH_ERR_ALIGN", -6: "MH_ERR_UNSUPPORTED", -7: "MH_ERR_WORKSPACE", -8: "MH_ERR_HIP",
}

_i64, _i32, _f32, _vp, _sz = ct.c_int64, ct.c_int32, ct.c_float, ct.c_void_p, ct.c_size_t


class SsdArgs(ct.Structure):
    _fields_ = [
        ("batch", _i64), ("seqlen", _i64), ("nheads", _i64), ("headdim", _i64), ("dstate", _i64),
        ("ngroups", _i64), ("chunk_len", _i64),
        ("dtype", _i32), ("flags", _i32), ("dt_min", _f32), ("dt_max", _f32),
        ("x", _vp), ("x_stride_b", _i64), ("x_stride_l", _i64), ("x_stride_h", _i64),
        ("dt", _vp), ("dt_stride_b", _i64), ("dt_stride_l", _i64),
        ("A", _vp),
        ("B", _vp), ("B_stride_b", _i64), ("B_stride_l", _i64),
        ("C", _vp), ("C_stride_b", _i64), ("C_stride_l", _i64),
        ("D", _vp), ("dt_bias", _vp), ("initial_state", _vp),
        ("y", _vp), ("y_stride_b", _i64), ("y_stride_l", _i64), ("y_stride_h", _i64),
        ("final_state", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("z", _vp), ("z_stride_b", _i64), ("z_stride_l", _i64), ("z_stride_h", _i64),
        ("xsum", _vp),
    ]


class SsdBwdArgs(ct.Structure):
    _fields_ = [
        ("fwd", SsdArgs),
        ("dy", _vp), ("dy_stride_b", _i64), ("dy_stride_l", _i64), ("dy_stride_h", _i64),
        ("d_final_state", _vp),
        ("dx", _vp), ("dx_stride_b", _i64), ("dx_stride_l", _i64), ("dx_stride_h", _i64),
        ("ddt", _vp), ("ddt_stride_b", _i64), ("ddt_stride_l", _i64),
        ("dA", _vp),
        ("dB", _vp), ("dB_stride_b", _i64), ("dB_stride_l", _i64),
        ("dC", _vp), ("dC_stride_b", _i64), ("dC_stride_l", _i64),
        ("dD", _vp), ("d_dt_bias", _vp), ("d_initial_state", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("dx_rows", _vp),
    ]


class SsdHsBwdArgs(ct.Structure):
    _fields_ = [
        ("fwd", SsdArgs),
        ("dhs", _vp), ("dx", _vp), ("ddt", _vp), ("dA", _vp), ("dB", _vp),
        ("d_dt_bias", _vp), ("d_initial_state", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("dx_rows", _vp),
    ]


class SsdRefBwdArgs(ct.Structure):
    _fields_ = [
        ("fwd", SsdArgs),
        ("dy", _vp), ("dhs", _vp), ("d_final_state", _vp),
        ("dx", _vp), ("ddt", _vp), ("dA", _vp), ("dB", _vp), ("dC", _vp), ("dD", _vp),
        ("d_dt_bias", _vp), ("d_initial_state", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
    ]


class SsuArgs(ct.Structure):
    _fields_ = [
        ("batch", _i64), ("nheads", _i64), ("headdim", _i64), ("dstate", _i64), ("ngroups", _i64),
        ("dtype", _i32), ("flags", _i32), ("dt_min", _f32), ("dt_max", _f32),
        ("state_in", _vp), ("state_out", _vp),
        ("x", _vp), ("x_stride_b", _i64),
        ("dt", _vp), ("dt_stride_b", _i64),
        ("A", _vp),
        ("B", _vp), ("B_stride_b", _i64),
        ("C", _vp), ("C_stride_b", _i64),
        ("D", _vp), ("dt_bias", _vp),
        ("y", _vp), ("y_stride_b", _i64),
        ("z", _vp), ("z_stride_b", _i64),
    ]


class KdaArgs(ct.Structure):
    _fields_ = [
        ("batch", _i64), ("nheads", _i64), ("seqlen", _i64), ("dk", _i64), ("dv", _i64),
        ("dtype", _i32), ("mode", _i32), ("kernel_dim", _i32), ("lam", _f32),
        ("lam_per_head", _vp),
        ("q1", _vp), ("q2", _vp), ("k", _vp), ("v", _vp),
        ("g", _vp),
        ("initial_state", _vp), ("initial_z", _vp),
        ("final_state", _vp), ("final_z", _vp),
        ("o", _vp), ("o2", _vp),
    ]


class KdaStepArgs(ct.Structure):
    _fields_ = [
        ("batch", _i64), ("nheads", _i64), ("dk", _i64), ("dv", _i64),
        ("dtype", _i32), ("flags", _i32), ("kernel_dim", _i32), ("lam", _f32),
        ("lam_per_head", _vp),
        ("q1", _vp), ("q2", _vp), ("k", _vp), ("v", _vp),
        ("state", _vp), ("z", _vp), ("o", _vp), ("o2", _vp),
    ]


class KdaBwdArgs(ct.Structure):
    _fields_ = [
        ("fwd", KdaArgs), ("flags", _i32),
        ("do1", _vp), ("do2", _vp),
        ("d_final_state", _vp), ("d_final_z", _vp),
        ("dq1", _vp), ("dq2", _vp), ("dk", _vp), ("dv", _vp),
        ("d_initial_state", _vp), ("d_initial_z", _vp),
        ("d_lam", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
    ]


MH_KDA_BWD_DIFF = 1


class Conv1dArgs(ct.Structure):
    _fields_ = [
        ("batch", _i64), ("seqlen", _i64), ("dim", _i64), ("width", _i64),
        ("dtype", _i32), ("flags", _i32),
        ("x", _vp), ("x_stride_b", _i64), ("x_stride_l", _i64),
        ("weight", _vp), ("bias", _vp),
        ("conv_state", _vp), ("conv_state_len", _i64), ("conv_state_stride_b", _i64), ("conv_state_stride_l", _i64),
        ("y", _vp), ("y_stride_b", _i64), ("y_stride_l", _i64),
    ]


MH_CONV_SILU = 1


class Conv1dBwdArgs(ct.Structure):
    _fields_ = [
        ("fwd", Conv1dArgs),
        ("dy", _vp), ("dy_stride_b", _i64), ("dy_stride_l", _i64),
        ("dx", _vp), ("dx_stride_b", _i64), ("dx_stride_l", _i64),
        ("d_conv_state", _vp), ("d_conv_state_stride_b", _i64), ("d_conv_state_stride_l", _i64),
        ("dweight", _vp), ("dbias", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
    ]

class GateArgs(ct.Structure):
    _fields_ = [
        ("batch", _i64), ("seqlen", _i64), ("nheads", _i64), ("headdim", _i64),
        ("dtype", _i32), ("reserved", _i32),
        ("y", _vp), ("y_stride_b", _i64), ("y_stride_l", _i64), ("y_stride_h", _i64),
        ("z", _vp), ("z_stride_b", _i64), ("z_stride_l", _i64), ("z_stride_h", _i64),
        ("g", _vp), ("g_stride_b", _i64), ("g_stride_l", _i64), ("g_stride_h", _i64),
        ("out", _vp), ("out_stride_b", _i64), ("out_stride_l", _i64), ("out_stride_h", _i64),
        ("dz", _vp), ("dz_stride_b", _i64), ("dz_stride_l", _i64), ("dz_stride_h", _i64),
    ]


# every symbol include/mamformer_hip.h declares
EXPORTS = (
    "mh_abi_version", "mh_last_error",
    "mh_ssd_workspace_bytes", "mh_ssd_chunk_len", "mh_ssd_chunk_scan_fwd", "mh_ssd_chunk_scan_fwd_noalloc",
    "mh_ssd_bwd_workspace_bytes", "mh_ssd_chunk_scan_bwd",
    "mh_ssd_h_states_workspace_bytes", "mh_ssd_h_states",
    "mh_ssd_h_states_bwd_workspace_bytes", "mh_ssd_h_states_bwd",
    "mh_ssd_ref_scan_workspace_bytes", "mh_ssd_ref_scan_fwd",
    "mh_ssd_ref_scan_bwd_workspace_bytes", "mh_ssd_ref_scan_bwd",
    "mh_silu_gate_fwd", "mh_silu_gate_bwd",
    "mh_ssd_state_update",
    "mh_kda_chunk_scan_fwd", "mh_kda_bwd_workspace_bytes", "mh_kda_chunk_scan_bwd",
    "mh_kda_recurrent_step",
    "mh_causal_conv1d_fwd",
    "mh_conv1d_bwd_workspace_bytes", "mh_causal_conv1d_bwd",
)

_lock = threading.Lock()
_lib = None


class MHError(RuntimeError):
    """A C-ABI call returned a nonzero status."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn}: {ERRORS.get(code, code)}: {msg}")
        self.code = code


def lib():
    """Load (once) and return the ctypes handle; raises if the library is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m mamformer_amd.build` "
                    "(there is no CPU fallback for the scan ops)")
            h = ct.CDLL(str(LIB_PATH))
            h.mh_abi_version.restype = ct.c_int
            h.mh_last_error.restype = ct.c_char_p
            h.mh_ssd_workspace_bytes.argtypes = [ct.POINTER(SsdArgs), ct.POINTER(_sz)]
            h.mh_ssd_chunk_len.argtypes = [ct.POINTER(SsdArgs), ct.POINTER(_i64)]
            h.mh_ssd_chunk_scan_fwd.argtypes = [ct.POINTER(SsdArgs), _vp]
            h.mh_ssd_chunk_scan_fwd_noalloc.argtypes = [ct.POINTER(SsdArgs), _vp]
            h.mh_ssd_bwd_workspace_bytes.argtypes = [ct.POINTER(SsdBwdArgs), ct.POINTER(_sz)]
            h.mh_ssd_chunk_scan_bwd.argtypes = [ct.POINTER(SsdBwdArgs), _vp]
            h.mh_ssd_state_update.argtypes = [ct.POINTER(SsuArgs), _vp]
            h.mh_ssd_h_states_workspace_bytes.argtypes = [ct.POINTER(SsdArgs), ct.POINTER(_sz)]
            h.mh_ssd_h_states.argtypes = [ct.POINTER(SsdArgs), _vp, _vp]
            h.mh_ssd_h_states_bwd_workspace_bytes.argtypes = [ct.POINTER(SsdHsBwdArgs), ct.POINTER(_sz)]
            h.mh_ssd_h_states_bwd.argtypes = [ct.POINTER(SsdHsBwdArgs), _vp]
            h.mh_ssd_ref_scan_workspace_bytes.argtypes = [ct.POINTER(SsdArgs), ct.c_int, ct.POINTER(_sz)]
            h.mh_ssd_ref_scan_fwd.argtypes = [ct.POINTER(SsdArgs), _vp, _vp]
            h.mh_ssd_ref_scan_bwd_workspace_bytes.argtypes = [ct.POINTER(SsdRefBwdArgs), ct.POINTER(_sz)]
            h.mh_ssd_ref_scan_bwd.argtypes = [ct.POINTER(SsdRefBwdArgs), _vp]
            h.mh_silu_gate_fwd.argtypes = [ct.POINTER(GateArgs), _vp]
            h.mh_silu_gate_bwd.argtypes = [ct.POINTER(GateArgs), _vp]
            h.mh_kda_chunk_scan_fwd.argtypes = [ct.POINTER(KdaArgs), _vp]
            h.mh_kda_recurrent_step.argtypes = [ct.POINTER(KdaStepArgs), _vp]
            h.mh_kda_bwd_workspace_bytes.argtypes = [ct.POINTER(KdaBwdArgs), ct.POINTER(_sz)]
            h.mh_kda_chunk_scan_bwd.argtypes = [ct.POINTER(KdaBwdArgs), _vp]
            h.mh_causal_conv1d_fwd.argtypes = [ct.POINTER(Conv1dArgs), _vp]
            h.mh_conv1d_bwd_workspace_bytes.argtypes = [ct.POINTER(Conv1dBwdArgs), ct.POINTER(_sz)]
            h.mh_causal_conv1d_bwd.argtypes = [ct.POINTER(Conv1dBwdArgs), _vp]
            for name in ("mh_ssd_workspace_bytes", "mh_ssd_chunk_len", "mh_ssd_chunk_scan_fwd",
                         "mh_ssd_chunk_scan_fwd_noalloc",
                         "mh_ssd_state_update", "mh_kda_chunk_scan_fwd", "mh_kda_recurrent_step",
                         "mh_causal_conv1d_fwd", "mh_conv1d_bwd_workspace_bytes", "mh_causal_conv1d_bwd",
                         "mh_ssd_bwd_workspace_bytes", "mh_ssd_chunk_scan_bwd",
                         "mh_kda_bwd_workspace_bytes", "mh_kda_chunk_scan_bwd",
                         "mh_ssd_h_states_workspace_bytes", "mh_ssd_h_states",
                         "mh_ssd_h_states_bwd_workspace_bytes", "mh_ssd_h_states_bwd",
                         "mh_ssd_ref_scan_workspace_bytes", "mh_ssd_ref_scan_fwd",
                         "mh_ssd_ref_scan_bwd_workspace_bytes", "mh_ssd_ref_scan_bwd",
                         "mh_silu_gate_fwd", "mh_silu_gate_bwd"):
                getattr(h, name).restype = ct.c_int
            ver = h.mh_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH.name} ABI version {ver} != expected {ABI_VERSION}; rebuild")
            _lib = h
    return _lib


def check(fn: str, rc: int):
    if rc != 0:
        msg = lib().mh_last_error().decode(errors="replace")
        raise MHError(fn, rc, msg)


def call(fn: str, *args):
    rc = getattr(lib(), fn)(*args)
    check(fn, rc)
