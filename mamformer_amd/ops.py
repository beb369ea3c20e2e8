"""Scan-path operators with the reference's names, argument order and layouts.

Every op launches hand-written gfx950 HIP kernels through the C ABI
(``libmamformer_hip.so``) on the current torch stream.  There is no CPU or
PyTorch fallback: non-CUDA tensors or a missing library raise.

Reference functions replaced (``R`` = ``mamformer 671b/``):

=====================================  ====================================================================
``selective_scan``                      R/mamformer/layers/mamba2.py:31-67 (``_selective_scan_impl`` :70-130);
                                        differentiable (autograd through ``selective_scan_bwd``)
``selective_scan_bwd``                  the autograd backward of the same scan (trained through in
                                        R/tests/test_mamba2.py:56-71), as one explicit op
``recurrent_step``                      R/mamformer/layers/mamba2.py:407-458 (``Mamba2Block._recurrent_step``)
``selective_state_update``              in-place form of the same decode step (the state is updated in HBM)
``linear_attn_scan``                    gated KDA scan of the benchmark configuration (no reference function);
                                        ``mode="reference"``: the normalised phi-kernel scan below
``linear_attn_scan_pair``               R/mamformer/kernels/triton_ssd.py:260-350 (``triton_linear_attn_scan``)
``linear_attn_scan_single``             R/mamformer/kernels/triton_ssd.py:353-400 (``triton_linear_attn_scan_single``)
``linear_attention_scan``               R/mamformer/layers/kda_diff.py:357-478 (``_linear_attention_scan``)
``linear_attention_recurrent``          R/mamformer/layers/kda_diff.py:564-605 (``_linear_attention_recurrent``)
``linear_attn_step``                    in-place form of the same step (fp32 state and z updated in HBM)
``causal_conv1d``                       R/mamformer/layers/mamba2.py:370-405 (``Mamba2Block._causal_conv1d``)
                                        with the SiLU of mamba2.py:282-283 optionally fused
=====================================  ====================================================================

SSD convention.  The reference's scan uses a per-channel dt and a per-state
A_log (decay exp(-exp(A_log[n]) dt[c])); the kernels implement the Mamba-2
per-head form (decay exp(A_h dt_h), A_h < 0).  The two meet exactly through
the reparameterisation A_log = 0, dt_ref = -A_h dt_h, x_ref = x / -A_h,
D_ref = -A_h D_h (see ``oracle.ssd``).  Channel ``c = h * headdim + p`` so
``x (b, L, d_inner)`` and ``final_state (b, d_inner, N)`` keep the reference
memory layout.
"""

from __future__ import annotations

import ctypes as ct
from typing import Optional

import torch

from . import _lib
from ._lib import SsdArgs, SsdBwdArgs, SsuArgs, KdaArgs, Conv1dArgs, Conv1dBwdArgs

__all__ = ["selective_scan", "selective_scan_reference", "plan_selective_scan_reference", "selective_scan_bwd", "plan_selective_scan_bwd", "selective_state_update", "recurrent_step", "linear_attn_scan",
           "linear_attn_scan_pair", "linear_attn_scan_single", "linear_attention_scan", "diff_lambda",
           "linear_attn_step", "linear_attention_recurrent",
           "ssd_chunk_len", "Plan", "plan_selective_scan", "plan_selective_state_update", "plan_linear_attn_scan",
           "plan_linear_attn_step", "causal_conv1d", "linear_attn_scan_bwd"]

_DT = {torch.float32: _lib.MH_F32, torch.bfloat16: _lib.MH_BF16}


class _Heads64:
    """Head size P of the SSD prefill in the kernels' 64 channels: a head of P = 64 k channels is k heads of 64
    sharing its dt, A, dt_bias and B / C group (the recurrence of each channel depends only on its head's decay
    and the group's B, C), and other sizes are zero-padded to the next multiple of 64 first (a zero channel keeps
    a zero state and a zero output, so it changes nothing else; h_states, a mean over every channel, is rescaled).
    Every map is a view, repeat or pad that autograd differentiates."""

    def __init__(self, H, P):
        if P < 1:
            raise ValueError(f"selective_scan: head size must be positive, got {P}")
        self.H, self.P, self.k = H, P, (P + 63) // 64
        self.Pp = 64 * self.k

    def chan(self, t4):             # (b, L, H, P) -> (b, L, H k, 64)
        b, L = t4.shape[:2]
        if self.Pp != self.P:
            t4 = torch.nn.functional.pad(t4, (0, self.Pp - self.P))
        return t4.reshape(b, L, self.H * self.k, 64)

    def unchan(self, t4):           # (b, L, H k, 64) -> (b, L, H, P)
        b, L = t4.shape[:2]
        return t4.reshape(b, L, self.H, self.Pp)[..., :self.P]

    def state(self, s):             # (b, H, P, N) -> (b, H k, 64, N)
        if self.Pp != self.P:
            s = torch.nn.functional.pad(s, (0, 0, 0, self.Pp - self.P))
        return s.reshape(s.shape[0], self.H * self.k, 64, s.shape[-1])

    def unstate(self, s):           # (b, H k, 64, N) -> (b, H, P, N)
        return s.reshape(s.shape[0], self.H, self.Pp, s.shape[-1])[:, :, :self.P]

    def head(self, v, dim=-1):      # per-head values -> per sub-head
        return None if v is None else v.repeat_interleave(self.k, dim=dim)

    def unhead(self, v):            # gradient per sub-head -> per head (last dim H k)
        return None if v is None else v.reshape(*v.shape[:-1], self.H, self.k).sum(-1)

    def d_vec(self, D):             # D (H,) or (H P,) -> per sub-head or per padded channel
        if D is None:
            return None
        D = D.reshape(-1)
        if D.numel() == self.H:
            return self.head(D)
        D = D.reshape(self.H, self.P)
        if self.Pp != self.P:
            D = torch.nn.functional.pad(D, (0, self.Pp - self.P))
        return D.reshape(-1)

    def d_grad(self, dD, D):        # gradient of d_vec(D) -> gradient of D
        if dD.numel() == self.H * self.k and D.numel() == self.H:
            return self.unhead(dD).reshape(D.shape)
        return dD.reshape(self.H, self.Pp)[:, :self.P].reshape(D.shape)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ct.c_void_p(t.data_ptr())


def _stream(dev: torch.device):
    return ct.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _require_cuda(name, *ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{name}: HIP op needs device tensors (got {t.device}); no CPU path exists")
    devs = {t.device for t in ts if t is not None}
    if len(devs) > 1:
        raise RuntimeError(f"{name}: tensors on different devices {devs}")


def _f32c(t: Optional[torch.Tensor]):
    if t is None:
        return None
    return t.to(torch.float32).contiguous()


def _inner_contig(t: torch.Tensor, ndim_inner: int = 1) -> torch.Tensor:
    """Make the innermost `ndim_inner` dims contiguous and 16-byte aligned rows (copy if needed)."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and (ndim_inner == 1 or t.stride(-2) == t.shape[-1])
    ok = ok and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-ndim_inner])
    return t if ok else t.contiguous()


def _ssd_args(x4, dt, A, B4, C4, D, dt_bias, dt_softplus, dt_limit, initial_state, y4, final_state, chunk_size,
              z4=None, xsum=None):
    b, L, H, P = x4.shape
    G, N = B4.shape[2], B4.shape[3]
    a = SsdArgs()
    a.batch, a.seqlen, a.nheads, a.headdim, a.dstate, a.ngroups = b, L, H, P, N, G
    a.chunk_len = int(chunk_size or 0)
    a.dtype = _DT[x4.dtype]
    flags = 0
    if dt_softplus:
        flags |= _lib.MH_DT_SOFTPLUS
    if dt_limit is not None:
        flags |= _lib.MH_DT_LIMIT
        a.dt_min, a.dt_max = float(dt_limit[0]), float(dt_limit[1])
    if D is not None and D.numel() == H * P and H * P != H:
        flags |= _lib.MH_D_PER_CHANNEL
    a.flags = flags
    a.x, a.x_stride_b, a.x_stride_l, a.x_stride_h = _ptr(x4), x4.stride(0), x4.stride(1), x4.stride(2)
    a.dt, a.dt_stride_b, a.dt_stride_l = _ptr(dt), dt.stride(0), dt.stride(1)
    a.A = _ptr(A)
    a.B, a.B_stride_b, a.B_stride_l = _ptr(B4), B4.stride(0), B4.stride(1)
    a.C, a.C_stride_b, a.C_stride_l = _ptr(C4), C4.stride(0), C4.stride(1)
    a.D, a.dt_bias, a.initial_state = _ptr(D), _ptr(dt_bias), _ptr(initial_state)
    a.y, a.y_stride_b, a.y_stride_l, a.y_stride_h = _ptr(y4), y4.stride(0), y4.stride(1), y4.stride(2)
    a.final_state = _ptr(final_state)
    if z4 is not None:
        a.z, a.z_stride_b, a.z_stride_l, a.z_stride_h = _ptr(z4), z4.stride(0), z4.stride(1), z4.stride(2)
    a.xsum = _ptr(xsum)
    return a


def ssd_chunk_len(batch, seqlen, nheads, headdim, dstate, ngroups, dtype=torch.bfloat16, chunk_size=None):
    """State-passing chunk length the kernels will use for these sizes (auto when chunk_size is None)."""
    a = SsdArgs()
    a.batch, a.seqlen, a.nheads, a.headdim, a.dstate, a.ngroups = batch, seqlen, nheads, headdim, dstate, ngroups
    a.chunk_len = int(chunk_size or 0)
    a.dtype = _DT[dtype]
    # dummy, aligned, non-null pointers and consistent strides (validation only)
    fake = ct.c_void_p(256)
    a.x = a.B = a.C = a.y = a.dt = a.A = fake
    a.x_stride_h = a.y_stride_h = headdim
    a.x_stride_l = a.y_stride_l = nheads * headdim
    a.x_stride_b = a.y_stride_b = seqlen * nheads * headdim
    a.B_stride_l = a.C_stride_l = ngroups * dstate
    a.B_stride_b = a.C_stride_b = seqlen * ngroups * dstate
    out = ct.c_int64()
    _lib.call("mh_ssd_chunk_len", ct.byref(a), ct.byref(out))
    return out.value


class Plan:
    """A validated launch of one op on fixed device buffers.

    Calling the plan re-runs the op on the same buffers (inputs may be
    overwritten in place between calls) with no allocation and no Python-side
    checks -- for serving loops, graph capture and benchmarking.  Outputs are
    attributes (``y``, ``final_state``, ``o``...).  The plan keeps every buffer
    it references alive.
    """

    def __init__(self, fn, args, device, keep=(), **outputs):
        self._fn, self._args, self._device, self._keep = fn, args, device, keep
        self.__dict__.update(outputs)

    def __call__(self, stream=None):
        s = _stream(self._device) if stream is None else ct.c_void_p(stream)
        _lib.call(self._fn, ct.byref(self._args), s)
        return self


def plan_selective_scan(*args, **kw):
    """Validate and allocate once; returns a ``Plan`` whose call launches ``selective_scan`` (outputs ``y``,
    ``final_state``)."""
    return selective_scan(*args, _plan_only=True, **kw)


def selective_scan(x, dt, A, B, C, D, return_h_states=False, return_final_state=False, *,
                   chunk_size=None, initial_state=None, dt_bias=None, dt_softplus=False, dt_limit=None, z=None,
                   _plan_only=False):
    """Mamba-2 SSD chunked-scan prefill.  Drop-in for ``selective_scan`` (R/mamformer/layers/mamba2.py:31-67).

    Args (SSD convention; see module docstring):
        x: (b, L, H*P) like the reference, or (b, L, H, P); fp32 or bf16.  The kernels run heads of P = 64
            channels; a head of 64 k channels runs as k of them, other head sizes zero-padded to the next
            multiple of 64 (``_Heads64``).
        dt: (b, L, H) per-head step sizes (positive unless ``dt_softplus``).
        A: (H,) per-head decay rates, A <= 0.
        B, C: (b, L, N) (one group, as the reference) or (b, L, G, N); dtype of x.
        D: (H,), (H*P,) or None.
        return_h_states: also return h_states (b, L, N), the per-token mean of the state over the
            H*P channels (mamba2.py:114-116); computed by ``mh_ssd_h_states`` from the state's channel sums,
            which need one scalar per (token, head) (see ``_h_states``).
        return_final_state: also return the state after the last token,
            shaped (b, H*P, N) for 3-D x (the reference's (b, d_inner, d_state)) or (b, H, P, N).
        chunk_size: state-passing chunk length (multiple of 64); None picks it from the shape.
        initial_state: (b, H*P, N) / (b, H, P, N) fp32 state before the first token (prefill of a cached
            sequence); the reference scan always starts from zero (mamba2.py:101).
        dt_bias, dt_softplus, dt_limit: dt <- clamp(softplus(dt + dt_bias), *dt_limit) inside the kernel.
        z: optional gate shaped like x: y <- y * silu(z) applied as y is stored -- the z-gate that
            ``Mamba2Block.forward`` applies right after the scan (mamba2.py:337-338).  h_states and the
            final state are not gated.
    Returns y (like x), or a tuple in the reference's order (y, h_states, final_state) (mamba2.py:121-130).
    """
    if return_h_states and _plan_only:
        raise ValueError("plan_selective_scan: return_h_states is not planned (call selective_scan)")
    _require_cuda("selective_scan", x, dt, A, B, C, D, initial_state, dt_bias, z)
    if x.dtype not in _DT:
        raise TypeError(f"selective_scan: x dtype {x.dtype} not supported (float32, bfloat16)")
    if B.dtype != x.dtype or C.dtype != x.dtype:
        raise TypeError("selective_scan: B and C must have the dtype of x")
    if dt.dim() != 3:
        raise ValueError(f"selective_scan: dt must be (b, L, H), got {tuple(dt.shape)}")
    b, L, H = dt.shape
    if x.dim() == 3:
        if x.shape[0] != b or x.shape[1] != L or x.shape[2] % H:
            raise ValueError(f"selective_scan: x {tuple(x.shape)} incompatible with dt {tuple(dt.shape)}")
        P = x.shape[2] // H
        x4 = x.view(b, L, H, P) if x.stride(-1) == 1 else x.contiguous().view(b, L, H, P)
    elif x.dim() == 4:
        P = x.shape[3]
        if tuple(x.shape[:3]) != (b, L, H):
            raise ValueError(f"selective_scan: x {tuple(x.shape)} incompatible with dt {tuple(dt.shape)}")
        x4 = x
    else:
        raise ValueError("selective_scan: x must be (b, L, H*P) or (b, L, H, P)")
    B4 = B.unsqueeze(2) if B.dim() == 3 else B
    C4 = C.unsqueeze(2) if C.dim() == 3 else C
    if B4.shape[:2] != (b, L) or C4.shape != B4.shape:
        raise ValueError(f"selective_scan: B {tuple(B.shape)} / C {tuple(C.shape)} incompatible with dt")
    G, N = B4.shape[2], B4.shape[3]
    if A.shape != (H,):
        raise ValueError(f"selective_scan: A must be (H,) = ({H},), got {tuple(A.shape)}")
    if D is not None and D.numel() not in (H, H * P):
        raise ValueError(f"selective_scan: D must have H or H*P entries, got {tuple(D.shape)}")
    if dt_bias is not None and dt_bias.numel() != H:
        raise ValueError(f"selective_scan: dt_bias must have H = {H} entries")
    if initial_state is not None and initial_state.numel() != b * H * P * N:
        raise ValueError(f"selective_scan: initial_state must hold b*H*P*N = {b * H * P * N} values")
    if z is not None and (z.shape != x.shape or z.dtype != x.dtype):
        raise ValueError(f"selective_scan: z must have the shape and dtype of x, got {tuple(z.shape)} {z.dtype}")
    if P != 64:
        # the kernels run heads of 64 channels: split (or pad and split) and map the outputs back
        if _plan_only:
            raise ValueError("plan_selective_scan: headdim must be 64 (selective_scan takes other head sizes)")
        hm = _Heads64(H, P)
        out = selective_scan(
            hm.chan(x4), hm.head(dt, 2), hm.head(A), B4, C4, hm.d_vec(D), return_h_states, return_final_state,
            chunk_size=chunk_size, dt_bias=hm.head(dt_bias), dt_softplus=dt_softplus, dt_limit=dt_limit,
            initial_state=None if initial_state is None else hm.state(initial_state.reshape(b, H, P, N)),
            z=None if z is None else hm.chan(z.reshape(b, L, H, P)))
        out = list(out) if isinstance(out, tuple) else [out]
        res = [hm.unchan(out[0]).reshape(x.shape)]
        if return_h_states:
            res.append(out[1] * (hm.Pp / P) if hm.Pp != P else out[1])
        if return_final_state:
            fin = hm.unstate(out[-1])
            res.append(fin.reshape(b, H * P, N) if x.dim() == 3 else fin)
        return res[0] if len(res) == 1 else tuple(res)
    x4 = _inner_contig(x4)
    B4 = _inner_contig(B4, 2)
    C4 = _inner_contig(C4, 2)
    dt32 = dt.to(torch.float32)
    if dt32.stride(-1) != 1:
        dt32 = dt32.contiguous()
    A32, D32, bias32 = _f32c(A), _f32c(D.reshape(-1) if D is not None else None), _f32c(dt_bias)
    h0 = None
    if initial_state is not None:
        h0 = initial_state.reshape(b, H, P, N).to(torch.float32).contiguous()
    z4 = None
    if z is not None:
        if z.dim() == 3:
            z4 = z.view(b, L, H, P) if z.stride(-1) == 1 else z.contiguous().view(b, L, H, P)
        else:
            z4 = z
        z4 = _inner_contig(z4)
    # with h_states, the scan also writes the sums of x over each half of a head, which h_states then reads
    # instead of x (headdim 64; the forward and the h_states backward take them)
    xsum = torch.empty((b, L, H, 2), device=x.device, dtype=torch.float32) if (return_h_states and P == 64) else None
    if not _plan_only and torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (x4, dt32, A32, B4, C4, D32, bias32, h0, z4)):
        cfg = (dt_softplus, dt_limit, chunk_size, xsum)
        if return_h_states:
            y4, fin, hs = _SelectiveScanHsFn.apply(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg)
        else:
            y4, fin = _SelectiveScanFn.apply(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg)
        if z4 is not None:
            y4 = _GateFn.apply(y4, z4)
        out = [y4.reshape(x.shape) if x.dim() == 3 else y4]
        if return_h_states:
            out.append(hs)
        if return_final_state:
            out.append(fin.reshape(b, H * P, N) if x.dim() == 3 else fin)
        return out[0] if len(out) == 1 else tuple(out)
    y4 = torch.empty((b, L, H, P), device=x.device, dtype=x.dtype)
    fin = torch.empty((b, H, P, N), device=x.device, dtype=torch.float32) if return_final_state else None
    args = _ssd_args(x4, dt32, A32, B4, C4, D32, bias32, dt_softplus, dt_limit, h0, y4, fin, chunk_size, z4,
                     None if _plan_only else xsum)
    nbytes = ct.c_size_t()
    _lib.call("mh_ssd_workspace_bytes", ct.byref(args), ct.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 16), device=x.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = _ptr(ws), nbytes.value
    y = y4.view(x.shape) if x.dim() == 3 else y4
    if fin is not None and x.dim() == 3:
        fin_out = fin.view(b, H * P, N)
    else:
        fin_out = fin
    plan = Plan("mh_ssd_chunk_scan_fwd", args, x.device,
                keep=(x4, dt32, A32, B4, C4, D32, bias32, h0, y4, fin, ws, z4), y=y, final_state=fin_out)
    if _plan_only:
        return plan
    plan()
    out = [y]
    if return_h_states:
        out.append(_h_states(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, chunk_size, xsum=xsum))
    if return_final_state:
        out.append(fin_out)
    return out[0] if len(out) == 1 else tuple(out)


def _scan_fwd(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg):
    dt_softplus, dt_limit, chunk_size = cfg[:3]
    xsum = cfg[3] if len(cfg) > 3 else None
    b, L, H, P = x4.shape
    N = B4.shape[3]
    y4 = torch.empty((b, L, H, P), device=x4.device, dtype=x4.dtype)
    fin = torch.empty((b, H, P, N), device=x4.device, dtype=torch.float32)
    args = _ssd_args(x4, dt32, A32, B4, C4, D32, bias32, dt_softplus, dt_limit, h0, y4, fin, chunk_size, None,
                     xsum)
    nbytes = ct.c_size_t()
    _lib.call("mh_ssd_workspace_bytes", ct.byref(args), ct.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 16), device=x4.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = _ptr(ws), nbytes.value
    _lib.call("mh_ssd_chunk_scan_fwd", ct.byref(args), _stream(x4.device))
    return y4, fin


def _scan_bwd(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg, dy4, dfin, need_dh0, plan_only=False, dx_rows=None):
    dt_softplus, dt_limit = cfg[0], cfg[1]
    b, L, H, P = x4.shape
    G, N = B4.shape[2], B4.shape[3]
    dev = x4.device
    if dy4 is None:
        dy4 = torch.zeros((b, L, H, P), device=dev, dtype=x4.dtype)
    dy4 = _inner_contig(dy4.to(x4.dtype))
    if dy4.stride(2) < P:                 # a broadcast gradient (e.g. of a sum over heads): the kernels need
        dy4 = dy4.contiguous()            # each head's row of P values in its own place
    dfin = None if dfin is None else dfin.reshape(b, H, P, N).to(torch.float32).contiguous()
    dx = torch.empty((b, L, H, P), device=dev, dtype=x4.dtype)
    ddt = torch.empty((b, L, H), device=dev, dtype=torch.float32)
    dA = torch.empty((H,), device=dev, dtype=torch.float32)
    dB = torch.empty((b, L, G, N), device=dev, dtype=x4.dtype)
    dC = torch.empty((b, L, G, N), device=dev, dtype=x4.dtype)
    dD = torch.empty_like(D32) if D32 is not None else None
    dbias = torch.empty((H,), device=dev, dtype=torch.float32) if bias32 is not None else None
    dh0 = torch.empty((b, H, P, N), device=dev, dtype=torch.float32) if need_dh0 else None
    a = SsdBwdArgs()
    a.fwd = _ssd_args(x4, dt32, A32, B4, C4, D32, bias32, dt_softplus, dt_limit, h0, x4, None, 64)
    a.fwd.y = None
    a.dy, a.dy_stride_b, a.dy_stride_l, a.dy_stride_h = _ptr(dy4), dy4.stride(0), dy4.stride(1), dy4.stride(2)
    a.d_final_state = _ptr(dfin)
    a.dx, a.dx_stride_b, a.dx_stride_l, a.dx_stride_h = _ptr(dx), dx.stride(0), dx.stride(1), dx.stride(2)
    a.ddt, a.ddt_stride_b, a.ddt_stride_l = _ptr(ddt), ddt.stride(0), ddt.stride(1)
    a.dA = _ptr(dA)
    a.dB, a.dB_stride_b, a.dB_stride_l = _ptr(dB), dB.stride(0), dB.stride(1)
    a.dC, a.dC_stride_b, a.dC_stride_l = _ptr(dC), dC.stride(0), dC.stride(1)
    a.dD, a.d_dt_bias, a.d_initial_state = _ptr(dD), _ptr(dbias), _ptr(dh0)
    a.dx_rows = _ptr(dx_rows)
    nbytes = ct.c_size_t()
    _lib.call("mh_ssd_bwd_workspace_bytes", ct.byref(a), ct.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 16), device=dev, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = _ptr(ws), nbytes.value
    if plan_only:
        return Plan("mh_ssd_chunk_scan_bwd", a, dev,
                    keep=(x4, dt32, A32, B4, C4, D32, h0, bias32, dy4, dfin, ws),
                    dx=dx, ddt=ddt, dA=dA, dB=dB, dC=dC, dD=dD, d_initial_state=dh0, d_dt_bias=dbias)
    _lib.call("mh_ssd_chunk_scan_bwd", ct.byref(a), _stream(dev))
    return dx, ddt, dA, dB, dC, dD, dh0, dbias


class _SelectiveScanFn(torch.autograd.Function):
    """Autograd node of the HIP scan: forward = the prefill kernels, backward = ``mh_ssd_chunk_scan_bwd``."""

    @staticmethod
    def forward(ctx, x4, dt32, A32, B4, C4, D32, h0, bias32, cfg):
        y4, fin = _scan_fwd(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg)
        ctx.save_for_backward(x4, dt32, A32, B4, C4, D32, h0, bias32)
        ctx.cfg = cfg
        return y4, fin

    @staticmethod
    def backward(ctx, dy4, dfin):
        x4, dt32, A32, B4, C4, D32, h0, bias32 = ctx.saved_tensors
        need_dh0 = h0 is not None and ctx.needs_input_grad[6]
        dx, ddt, dA, dB, dC, dD, dh0, dbias = _scan_bwd(x4, dt32, A32, B4, C4, D32, h0, bias32, ctx.cfg, dy4,
                                                        dfin, need_dh0)
        return dx, ddt, dA, dB, dC, dD, dh0, dbias, None


class _SelectiveScanHsFn(torch.autograd.Function):
    """The scan with h_states (``selective_scan(..., return_h_states=True)`` under autograd, mamba2.py:114-116):
    forward = the prefill kernels (which also write the per-head sums of x) and ``mh_ssd_h_states``; backward =
    the h_states gradient first, its gradient w.r.t. x as one fp32 value per (token, head) row
    (``mh_ssd_h_states_bwd`` with ``dx_rows``), then ``mh_ssd_chunk_scan_bwd``, which adds those rows to its dx as
    it stores it, so the two gradients w.r.t. x meet without a separate pass over dx.  The remaining gradients
    (dt, A, B, dt_bias, the initial state) of the two outputs are added here."""

    @staticmethod
    def forward(ctx, x4, dt32, A32, B4, C4, D32, h0, bias32, cfg):
        y4, fin = _scan_fwd(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg)
        hs = _h_states_fwd(x4, dt32, A32, B4, h0, bias32, cfg[0], cfg[1], cfg[3])
        ctx.save_for_backward(x4, dt32, A32, B4, C4, D32, h0, bias32)
        ctx.cfg = cfg
        ctx.set_materialize_grads(False)
        return y4, fin, hs

    @staticmethod
    def backward(ctx, dy4, dfin, dhs):
        x4, dt32, A32, B4, C4, D32, h0, bias32 = ctx.saved_tensors
        cfg = ctx.cfg
        need_dh0 = h0 is not None and ctx.needs_input_grad[6]
        if dhs is None:
            dx, ddt, dA, dB, dC, dD, dh0, dbias = _scan_bwd(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg, dy4,
                                                            dfin, need_dh0)
            return dx, ddt, dA, dB, dC, dD, dh0, dbias, None
        xr, ddt_h, dA_h, dB_h, dh0_h, dbias_h = _h_states_bwd_blocks(dhs, x4, dt32, A32, B4, h0, bias32, cfg[0],
                                                                     cfg[1], cfg[3], rows=True)
        if dy4 is None and dfin is None:            # only h_states reaches the loss
            b, L, H, P = x4.shape
            dx = xr[..., None].expand(b, L, H, P).to(x4.dtype)
            dC = torch.zeros_like(C4)
            dD = None if D32 is None else torch.zeros_like(D32)
            return (dx, ddt_h, dA_h, dB_h, dC, dD, dh0_h if need_dh0 else None, dbias_h, None)
        dx, ddt, dA, dB, dC, dD, dh0, dbias = _scan_bwd(x4, dt32, A32, B4, C4, D32, h0, bias32, cfg, dy4, dfin,
                                                        need_dh0, dx_rows=xr)
        dh0 = dh0 + dh0_h if need_dh0 else None
        dbias = None if dbias is None else dbias + dbias_h
        return dx, ddt + ddt_h, dA + dA_h, dB + dB_h, dC, dD, dh0, dbias, None


def _gate_args(y4, z4, out, g=None, dz=None):
    b, L, H, P = y4.shape
    a = _lib.GateArgs()
    a.batch, a.seqlen, a.nheads, a.headdim = b, L, H, P
    a.dtype = _DT[y4.dtype]
    for name, t in (("y", y4), ("z", z4), ("out", out), ("g", g), ("dz", dz)):
        if t is not None:
            setattr(a, name, _ptr(t))
            setattr(a, name + "_stride_b", t.stride(0))
            setattr(a, name + "_stride_l", t.stride(1))
            setattr(a, name + "_stride_h", t.stride(2))
    return a


class _GateFn(torch.autograd.Function):
    """The block's output gate y * silu(z) (R/mamformer/layers/mamba2.py:337-338) on the training path, where the
    ungated y is kept for the backward: one fused pass forward (``mh_silu_gate_fwd``) and one backward
    (``mh_silu_gate_bwd``: dy = g silu(z), dz = g y silu'(z)) instead of torch's separate element-wise kernels."""

    @staticmethod
    def forward(ctx, y4, z4):
        y4c = _inner_contig(y4)
        out = torch.empty(y4.shape, device=y4.device, dtype=y4.dtype)
        _lib.call("mh_silu_gate_fwd", ct.byref(_gate_args(y4c, z4, out)), _stream(y4.device))
        ctx.save_for_backward(y4c, z4)
        return out

    @staticmethod
    def backward(ctx, g):
        y4, z4 = ctx.saved_tensors
        g = _inner_contig(g.to(y4.dtype))
        if any(s < 0 for s in g.stride()) or g.stride(2) < y4.shape[3]:
            g = g.contiguous()
        dy = torch.empty(y4.shape, device=y4.device, dtype=y4.dtype)
        dz = torch.empty(y4.shape, device=y4.device, dtype=y4.dtype)
        _lib.call("mh_silu_gate_bwd", ct.byref(_gate_args(y4, z4, dy, g, dz)), _stream(y4.device))
        return dy, dz


def plan_selective_scan_bwd(*args, **kw):
    """Validate and allocate once; returns a ``Plan`` whose call launches ``selective_scan_bwd`` into the same
    gradient buffers (attributes ``dx``, ``ddt``, ``dA``, ``dB``, ``dC``, ``dD``, ``d_initial_state``,
    ``d_dt_bias``, shaped as the kernels write them)."""
    return selective_scan_bwd(*args, _plan_only=True, **kw)


def selective_scan_bwd(dy, x, dt, A, B, C, D=None, *, d_final_state=None, initial_state=None, dt_bias=None,
                       dt_softplus=False, dt_limit=None, _plan_only=False):
    """Gradients of ``<dy, y> + <d_final_state, final_state>`` for ``y, final_state = selective_scan(x, dt, A, B,
    C, D, initial_state=..., dt_bias=..., dt_softplus=..., dt_limit=...)`` -- the backward PyTorch autograd runs
    through the reference's scan (mamba2.py:70-130; R/tests/test_mamba2.py:56-71), on the GPU.

    Shapes as ``selective_scan`` (x and dy (b, L, H*P) or (b, L, H, P)); ``dy`` None means zero.
    Returns a dict with dx (like x), ddt (b, L, H) fp32 w.r.t. the raw dt (through bias / softplus / clamp),
    dA (H,), dB, dC (like B, C), dD (like D, when D is given), d_dt_bias (H,) when dt_bias is given and
    d_initial_state (like initial_state, or (b, H, P, N) when none was given: the gradient w.r.t. a zero one).
    """
    _require_cuda("selective_scan_bwd", dy, x, dt, A, B, C, D, d_final_state, initial_state, dt_bias)
    if x.dtype not in _DT or B.dtype != x.dtype or C.dtype != x.dtype:
        raise TypeError("selective_scan_bwd: x, B, C must share one dtype (float32 or bfloat16)")
    b, L, H = dt.shape
    if x.dim() == 3:
        P = x.shape[2] // H
        x4 = x.reshape(b, L, H, P)
    else:
        P = x.shape[3]
        x4 = x
    B4 = B.unsqueeze(2) if B.dim() == 3 else B
    C4 = C.unsqueeze(2) if C.dim() == 3 else C
    N = B4.shape[3]
    if A.shape != (H,):
        raise ValueError(f"selective_scan_bwd: A must be (H,) = ({H},), got {tuple(A.shape)}")
    if D is not None and D.numel() not in (H, H * P):
        raise ValueError(f"selective_scan_bwd: D must have H or H*P entries, got {tuple(D.shape)}")
    if P != 64:
        # heads of 64 channels, as in selective_scan; the gradients of the shared per-head values are summed
        if _plan_only:
            raise ValueError("plan_selective_scan_bwd: headdim must be 64 (selective_scan_bwd takes other head sizes)")
        hm = _Heads64(H, P)
        r = selective_scan_bwd(
            None if dy is None else hm.chan(dy.reshape(b, L, H, P)), hm.chan(x4), hm.head(dt, 2), hm.head(A), B4,
            C4, hm.d_vec(D), dt_softplus=dt_softplus, dt_limit=dt_limit, dt_bias=hm.head(dt_bias),
            d_final_state=None if d_final_state is None else hm.state(d_final_state.reshape(b, H, P, N)),
            initial_state=None if initial_state is None else hm.state(initial_state.reshape(b, H, P, N)))
        dh0 = hm.unstate(r["d_initial_state"])
        out = {"dx": hm.unchan(r["dx"]).reshape(x.shape), "ddt": hm.unhead(r["ddt"]), "dA": hm.unhead(r["dA"]),
               "dB": r["dB"].reshape(B.shape), "dC": r["dC"].reshape(C.shape),
               "d_initial_state": dh0 if initial_state is None else dh0.reshape(initial_state.shape)}
        if D is not None:
            out["dD"] = hm.d_grad(r["dD"], D)
        if dt_bias is not None:
            out["d_dt_bias"] = hm.unhead(r["d_dt_bias"]).reshape(dt_bias.shape)
        return out
    x4 = _inner_contig(x4)
    B4, C4 = _inner_contig(B4, 2), _inner_contig(C4, 2)
    dt32 = dt.to(torch.float32)
    if dt32.stride(-1) != 1:
        dt32 = dt32.contiguous()
    A32, D32, bias32 = _f32c(A), _f32c(D.reshape(-1) if D is not None else None), _f32c(dt_bias)
    h0 = None if initial_state is None else initial_state.reshape(b, H, P, N).to(torch.float32).contiguous()
    dy4 = None if dy is None else dy.reshape(b, L, H, P)
    with torch.no_grad():
        res = _scan_bwd(x4, dt32, A32, B4, C4, D32, h0, bias32, (dt_softplus, dt_limit, None), dy4, d_final_state,
                        True, plan_only=_plan_only)
    if _plan_only:
        return res
    dx, ddt, dA, dB, dC, dD, dh0, dbias = res
    out = {"dx": dx.reshape(x.shape), "ddt": ddt, "dA": dA, "dB": dB.reshape(B.shape), "dC": dC.reshape(C.shape),
           "d_initial_state": dh0 if initial_state is None else dh0.reshape(initial_state.shape)}
    if D is not None:
        out["dD"] = dD.reshape(D.shape)
    if dt_bias is not None:
        out["d_dt_bias"] = dbias.reshape(dt_bias.shape)
    return out


def _h_states(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, chunk_size, xsum=None):
    """h_states[b, t, n] = mean over (h, p) of the state h_t[h, p, n] (mamba2.py:114-116), without autograd.

    Computed by ``mh_ssd_h_states`` (the channel sums of the state follow a recurrence with one scalar input per
    (token, head), sum_p x); under autograd ``_SelectiveScanHsFn`` computes it together with the scan.
    """
    return _h_states_fwd(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum)


_HS_MAXH = 128    # heads the h_states kernels hold at once (forward and backward)
_HS_BWD_MAXN = 128  # state columns of the h_states backward kernel


def _head_blocks(H, G):
    """Blocks [h0, h1) of at most 128 heads that never split a group unless a group alone has more than 128 heads
    (then it is cut into pieces of at most 128).  h_states is a sum over heads, so blocks combine linearly."""
    hpg = H // G
    out = []
    if hpg <= _HS_MAXH:
        k = _HS_MAXH // hpg
        for g0 in range(0, G, k):
            out.append((g0 * hpg, min(G, g0 + k) * hpg))
    else:
        for g in range(G):
            for h0 in range(g * hpg, (g + 1) * hpg, _HS_MAXH):
                out.append((h0, min(h0 + _HS_MAXH, (g + 1) * hpg)))
    return out


def _h_block_args(x4, dt32, A32, B4, h0, bias32, h0_, h1_):
    """The inputs restricted to heads [h0_, h1_) and their groups (B / C groups as a contiguous slice)."""
    H, G = x4.shape[2], B4.shape[2]
    hpg = H // G
    g0, g1 = h0_ // hpg, (h1_ - 1) // hpg + 1
    return (x4[:, :, h0_:h1_], dt32[:, :, h0_:h1_], A32[h0_:h1_].contiguous(), B4[:, :, g0:g1].contiguous(),
            None if h0 is None else h0[:, h0_:h1_].contiguous(),
            None if bias32 is None else bias32[h0_:h1_].contiguous(), g0, g1)


def _h_states_fwd(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum=None):
    """h_states by ``mh_ssd_h_states`` (reading the prefill's sums of x, ``xsum``, when given); more than 128 heads
    run as head blocks whose fp32 h_states are combined with weights H_block / H (the mean over (h, p) is linear
    in the heads)."""
    H = x4.shape[2]
    if H <= _HS_MAXH:
        return _h_states_kernel(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum)
    x32, B32 = x4.to(torch.float32), B4.to(torch.float32)
    acc = None
    for h0_, h1_ in _head_blocks(H, B4.shape[2]):
        xb, db, ab, bb, h0b, biasb, _, _ = _h_block_args(x32, dt32, A32, B32, h0, bias32, h0_, h1_)
        part = _h_states_kernel(xb, db, ab, bb, h0b, biasb, dt_softplus, dt_limit) * ((h1_ - h0_) / H)
        acc = part if acc is None else acc + part
    return acc.to(x4.dtype)


def _h_states_kernel(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum=None):
    b, L, H, P = x4.shape
    N = B4.shape[3]
    hs = torch.empty((b, L, N), device=x4.device, dtype=x4.dtype)
    args = _ssd_args(x4, dt32, A32, B4, B4, None, bias32, dt_softplus, dt_limit, h0, x4, None, 64, None, xsum)
    nbytes = ct.c_size_t()
    _lib.call("mh_ssd_h_states_workspace_bytes", ct.byref(args), ct.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 16), device=x4.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = _ptr(ws), nbytes.value
    _lib.call("mh_ssd_h_states", ct.byref(args), _ptr(hs), _stream(x4.device))
    return hs


def _h_states_bwd_kernel(ghs, x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum=None, rows=False):
    """Gradients of <ghs, h_states> by ``mh_ssd_h_states_bwd``: (dx, ddt, dA, dB, d h0, d dt_bias); with ``rows``
    the gradient w.r.t. x as its one value per (token, head), (b, L, H) fp32, instead of dx."""
    b, L, H, P = x4.shape
    G, N = B4.shape[2], B4.shape[3]
    dev = x4.device
    ghs = ghs.to(x4.dtype).contiguous()
    dx = None if rows else torch.empty((b, L, H, P), device=dev, dtype=x4.dtype)
    dxr = torch.empty((b, L, H), device=dev, dtype=torch.float32) if rows else None
    ddt = torch.empty((b, L, H), device=dev, dtype=torch.float32)
    dA = torch.empty((H,), device=dev, dtype=torch.float32)
    dB = torch.empty((b, L, G, N), device=dev, dtype=B4.dtype)
    dh0 = None if h0 is None else torch.empty((b, H, P, N), device=dev, dtype=torch.float32)
    dbias = None if bias32 is None else torch.empty((H,), device=dev, dtype=torch.float32)
    a = _lib.SsdHsBwdArgs()
    a.fwd = _ssd_args(x4, dt32, A32, B4, B4, None, bias32, dt_softplus, dt_limit, h0, x4, None, 64, None, xsum)
    a.dhs, a.dx, a.ddt, a.dA, a.dB = _ptr(ghs), _ptr(dx), _ptr(ddt), _ptr(dA), _ptr(dB)
    a.d_dt_bias, a.d_initial_state, a.dx_rows = _ptr(dbias), _ptr(dh0), _ptr(dxr)
    nbytes = ct.c_size_t()
    _lib.call("mh_ssd_h_states_bwd_workspace_bytes", ct.byref(a), ct.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 16), device=dev, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = _ptr(ws), nbytes.value
    _lib.call("mh_ssd_h_states_bwd", ct.byref(a), _stream(dev))
    return (dxr if rows else dx), ddt, dA, dB, dh0, dbias


def _h_states_bwd_blocks(ghs, x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum=None, rows=False):
    """``mh_ssd_h_states_bwd`` for any head count and dstate: the state columns separate (column n of h_states
    depends on B[..., n] alone; dx, ddt, dA and d dt_bias are sums over columns, dB and d h0 per column), so
    dstate > 128 runs as column pieces of at most 128; the heads enter h_states as a sum, so more than 128 heads
    run as head blocks, each with the gradient scaled by H_block / H (its h_states is a mean over its own heads).
    Every piece is the dedicated kernel; pieces combine in a fixed order (deterministic).  With ``rows`` the
    gradient w.r.t. x comes as its one fp32 value per (token, head), (b, L, H)."""
    b, L, H, P = x4.shape
    G, N = B4.shape[2], B4.shape[3]
    if N > _HS_BWD_MAXN:
        outs = []
        for n0 in range(0, N, _HS_BWD_MAXN):
            n1 = min(N, n0 + _HS_BWD_MAXN)
            outs.append(_h_states_bwd_blocks(ghs[..., n0:n1], x4, dt32, A32, B4[..., n0:n1].contiguous(),
                                             None if h0 is None else h0[..., n0:n1].contiguous(), bias32,
                                             dt_softplus, dt_limit, xsum, rows))
        dx = sum(o[0].to(torch.float32) for o in outs)
        dx = dx if rows else dx.to(x4.dtype)
        ddt = sum(o[1] for o in outs)
        dA = sum(o[2] for o in outs)
        dB = torch.cat([o[3] for o in outs], dim=-1)
        dh0 = None if h0 is None else torch.cat([o[4] for o in outs], dim=-1)
        dbias = None if bias32 is None else sum(o[5] for o in outs)
        return dx, ddt, dA, dB, dh0, dbias
    if H <= _HS_MAXH:
        return _h_states_bwd_kernel(ghs, x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, xsum, rows)
    dev = x4.device
    dx = torch.empty((b, L, H) if rows else (b, L, H, P), device=dev, dtype=torch.float32 if rows else x4.dtype)
    ddt = torch.empty((b, L, H), device=dev, dtype=torch.float32)
    dA = torch.empty((H,), device=dev, dtype=torch.float32)
    dB = torch.zeros((b, L, G, N), device=dev, dtype=torch.float32)
    dh0 = None if h0 is None else torch.empty((b, H, P, N), device=dev, dtype=torch.float32)
    dbias = None if bias32 is None else torch.empty((H,), device=dev, dtype=torch.float32)
    g32 = ghs.to(torch.float32)
    for h0_, h1_ in _head_blocks(H, G):
        xb, db, ab, bb, h0b, biasb, g0, g1 = _h_block_args(x4, dt32, A32, B4, h0, bias32, h0_, h1_)
        r = _h_states_bwd_kernel(g32 * ((h1_ - h0_) / H), xb, db, ab, bb, h0b, biasb, dt_softplus, dt_limit,
                                 rows=rows)
        dx[:, :, h0_:h1_] = r[0]
        ddt[:, :, h0_:h1_] = r[1]
        dA[h0_:h1_] = r[2]
        dB[:, :, g0:g1] += r[3].to(torch.float32)
        if dh0 is not None:
            dh0[:, h0_:h1_] = r[4]
        if dbias is not None:
            dbias[h0_:h1_] = r[5]
    return dx, ddt, dA, dB.to(B4.dtype), dh0, dbias


def _h_states_swap(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, chunk_size, grad=False):
    """h_states by a second run of the prefill kernels on a swapped problem: an independent second formulation
    (the tests check the dedicated kernels and their gradient against it at full size).

    The channel sum of the state is itself an SSD output once the roles of x and B are swapped: with
    heads h' = (h, q) over the two 64-wide halves q of the state dimension n, headdim' = 64 (n' = n - 64q),
    x'_t[h', n'] = B_t[g(h), 64q + n'], one group per original head with B'_t[h, p] = x_t[h, p]
    (dstate' = P), C' = 1, D' = 0, and the same dt and A per head, the recurrence gives
    h'_t[h', n', p] = h_t[h, p, 64q + n'], so y'_t[h', n'] = sum_p h_t[h, p, 64q + n'].  The same kernels
    compute it; the mean over heads is a reduction over the head axis.

    ``grad``: through the autograd node of the scan (backward = ``mh_ssd_chunk_scan_bwd`` of the swapped
    problem, with C' materialised as ones since the backward reads no broadcast C); the gathers and repeats
    of B, dt, A, dt_bias and h0 carry their gradients back to the caller's tensors.
    """
    b, L, H, P = x4.shape
    G, N = B4.shape[2], B4.shape[3]
    if P != 64:
        raise NotImplementedError("selective_scan: return_h_states needs headdim 64")
    if N % 64:                            # zero-padded state columns beyond N stay zero
        pad = 64 - N % 64
        B4 = torch.nn.functional.pad(B4, (0, pad))
        h0 = None if h0 is None else torch.nn.functional.pad(h0, (0, pad))
        hs = _h_states_swap(x4, dt32, A32, B4, h0, bias32, dt_softplus, dt_limit, chunk_size, grad)
        return hs[..., :N]
    Q = N // 64
    gidx = torch.arange(H, device=x4.device) // (H // G)
    xs = B4[:, :, gidx, :].reshape(b, L, H * Q, 64).contiguous()                # x'
    Bs = x4 if (x4.stride(-1) == 1 and x4.stride(-2) == P) else x4.contiguous()  # B' (g' = h, n' = p)
    Cs = torch.ones((1, 1, H, P), device=x4.device, dtype=x4.dtype).expand(b, L, H, P)
    dts = dt32.repeat_interleave(Q, dim=-1)
    As = A32.repeat_interleave(Q)
    bias_s = bias32.repeat_interleave(Q) if bias32 is not None else None
    h0s = None
    if h0 is not None:
        h0s = h0.view(b, H, P, Q, 64).permute(0, 1, 3, 4, 2).reshape(b, H * Q, 64, P).contiguous()
    if grad:
        Cs = torch.ones((b, L, H, P), device=x4.device, dtype=x4.dtype)
        ys, _ = _SelectiveScanFn.apply(xs, dts, As, Bs, Cs, None, h0s, bias_s, (dt_softplus, dt_limit, chunk_size))
        return (ys.reshape(b, L, H, N).to(torch.float32).sum(dim=2) / float(H * P)).to(x4.dtype)
    ys = torch.empty((b, L, H * Q, 64), device=x4.device, dtype=x4.dtype)
    args = _ssd_args(xs, dts, As, Bs, Cs, None, bias_s, dt_softplus, dt_limit, h0s, ys, None, chunk_size)
    nbytes = ct.c_size_t()
    _lib.call("mh_ssd_workspace_bytes", ct.byref(args), ct.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 16), device=x4.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = _ptr(ws), nbytes.value
    _lib.call("mh_ssd_chunk_scan_fwd", ct.byref(args), _stream(x4.device))
    hs = ys.view(b, L, H, N).to(torch.float32).sum(dim=2) / float(H * P)
    return hs.to(x4.dtype)


def _conv_args(x, w, bc, cs, silu):
    b, L, Dm = x.shape
    a = Conv1dArgs()
    a.batch, a.seqlen, a.dim, a.width = b, L, Dm, w.shape[1]
    a.dtype = _DT[x.dtype]
    a.flags = _lib.MH_CONV_SILU if silu else 0
    a.x, a.x_stride_b, a.x_stride_l = _ptr(x), x.stride(0), x.stride(1)
    a.weight, a.bias = _ptr(w), _ptr(bc)
    if cs is not None and cs.shape[1] > 0:
        a.conv_state, a.conv_state_len = _ptr(cs), cs.shape[1]
        a.conv_state_stride_b, a.conv_state_stride_l = cs.stride(0), cs.stride(1)
    return a


def _conv_fwd(xc, w, bc, cs, silu):
    y = torch.empty(xc.shape, device=xc.device, dtype=xc.dtype)
    a = _conv_args(xc, w, bc, cs, silu)
    a.y, a.y_stride_b, a.y_stride_l = _ptr(y), y.stride(0), y.stride(1)
    _lib.call("mh_causal_conv1d_fwd", ct.byref(a), _stream(xc.device))
    return y


def _conv_bwd(dy, xc, w, bc, cs, silu, need_dcs):
    dy = _inner_contig(dy.to(xc.dtype))
    dx = torch.empty(xc.shape, device=xc.device, dtype=xc.dtype)
    dcs = torch.empty(cs.shape, device=xc.device, dtype=xc.dtype) if (need_dcs and cs is not None) else None
    dw = torch.empty(w.shape, device=xc.device, dtype=torch.float32)
    db = torch.empty(w.shape[0], device=xc.device, dtype=torch.float32) if bc is not None else None
    q = Conv1dBwdArgs()
    q.fwd = _conv_args(xc, w, bc, cs, silu)
    q.dy, q.dy_stride_b, q.dy_stride_l = _ptr(dy), dy.stride(0), dy.stride(1)
    q.dx, q.dx_stride_b, q.dx_stride_l = _ptr(dx), dx.stride(0), dx.stride(1)
    if dcs is not None:
        q.d_conv_state, q.d_conv_state_stride_b, q.d_conv_state_stride_l = _ptr(dcs), dcs.stride(0), dcs.stride(1)
    q.dweight, q.dbias = _ptr(dw), _ptr(db)
    n = ct.c_size_t()
    _lib.call("mh_conv1d_bwd_workspace_bytes", ct.byref(q), ct.byref(n))
    ws = torch.empty(max(n.value, 16), device=xc.device, dtype=torch.uint8)
    q.workspace, q.workspace_bytes = _ptr(ws), ws.numel()
    _lib.call("mh_causal_conv1d_bwd", ct.byref(q), _stream(xc.device))
    return dx, dw, db, dcs


class _CausalConv1dFn(torch.autograd.Function):
    """Autograd node of the HIP conv: forward = ``mh_causal_conv1d_fwd``, backward = ``mh_causal_conv1d_bwd``."""

    @staticmethod
    def forward(ctx, xc, w, bc, cs, silu):
        y = _conv_fwd(xc, w, bc, cs, silu)
        ctx.save_for_backward(xc, w, bc, cs)
        ctx.silu = silu
        return y

    @staticmethod
    def backward(ctx, dy):
        xc, w, bc, cs = ctx.saved_tensors
        dx, dw, db, dcs = _conv_bwd(dy, xc, w, bc, cs, ctx.silu, ctx.needs_input_grad[3])
        return dx, dw, db, dcs, None


def causal_conv1d(x, weight, bias=None, conv_state=None, *, silu=False):
    """Causal depthwise conv1d over channels-last x (b, L, D) on the GPU (+ SiLU when ``silu``).

    ``Mamba2Block._causal_conv1d`` counterpart (R/mamformer/layers/mamba2.py:370-405): weight (D, 1, K) or
    (D, K) as ``nn.Conv1d(D, D, K, groups=D)`` holds it, optional bias (D,); ``conv_state`` (b, S_c, D) with
    S_c <= K-1 are the cached raw inputs prepended on the incremental path (:388-390).  Returns y (b, L, D)
    in the dtype of x (fp32 accumulation).  Differentiable in x, weight, bias and conv_state (backward
    ``mh_causal_conv1d_bwd``, what autograd forms through the reference's conv + SiLU when the block trains).
    """
    _require_cuda("causal_conv1d", x, weight, bias, conv_state)
    if x.dim() != 3:
        raise ValueError("causal_conv1d: x must be (b, L, D)")
    if x.dtype not in _DT:
        raise TypeError(f"causal_conv1d: x dtype {x.dtype} not supported (float32, bfloat16)")
    b, L, Dm = x.shape
    w = weight.reshape(Dm, -1).to(torch.float32).contiguous()
    K = w.shape[1]
    xc = _inner_contig(x)
    bc = _f32c(bias.reshape(-1)) if bias is not None else None
    cs = None
    if conv_state is not None and conv_state.shape[1] > 0:
        if conv_state.dim() != 3 or conv_state.shape[0] != b or conv_state.shape[2] != Dm:
            raise ValueError("causal_conv1d: conv_state must be (b, S_c, D)")
        if conv_state.shape[1] > K - 1:
            conv_state = conv_state[:, -(K - 1):] if K > 1 else conv_state[:, :0]
        cs = _inner_contig(conv_state.to(x.dtype))
    if cs is not None and cs.shape[1] == 0:
        cs = None
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (xc, w, bc, cs)):
        return _CausalConv1dFn.apply(xc, w, bc, cs, silu)
    return _conv_fwd(xc, w, bc, cs, silu)


def plan_selective_state_update(*args, **kw):
    """``Plan`` of ``selective_state_update`` on fixed buffers (output ``y``; the state is updated per call)."""
    return selective_state_update(*args, _plan_only=True, **kw)


def selective_state_update(state, x, dt, A, B, C, D=None, *, dt_bias=None, dt_softplus=True, dt_limit=None,
                           out_state=None, z=None, A_per_state=False, _plan_only=False):
    """One-token SSD state update on the GPU, in place by default.

    state (b, H, P, N) fp32 (updated in place unless ``out_state`` is given);
    x (b, H, P); dt (b, H) raw, or (b, H, P) one step per channel (``dt_softplus``/``dt_bias``/``dt_limit``
    applied in the kernel, as the decode path of mamba2.py:293 does before the step; dt_bias then (H*P,));
    A (H,), or with ``A_per_state`` (N,) one decay rate per state column; B, C (b, N) or (b, G, N);
    D (H,), (H, P) or None; optional gate z (b, H, P) like x: y <- y * silu(z) (mamba2.py:337-338).
    Returns y (b, H, P).  Semantics of ``Mamba2Block._recurrent_step`` (R/mamformer/layers/mamba2.py:431-458);
    with per-channel dt and per-state A it is the reference's own parameterisation.
    """
    _require_cuda("selective_state_update", state, x, dt, A, B, C, D, dt_bias, out_state, z)
    if state.dim() != 4 or state.dtype != torch.float32:
        raise ValueError("selective_state_update: state must be (b, H, P, N) float32")
    b, H, P, N = state.shape
    if x.shape != (b, H, P):
        raise ValueError(f"selective_state_update: x must be {(b, H, P)}, got {tuple(x.shape)}")
    if x.dtype not in _DT or B.dtype != x.dtype or C.dtype != x.dtype:
        raise TypeError("selective_state_update: x, B, C must share a dtype in (float32, bfloat16)")
    B3 = B.unsqueeze(1) if B.dim() == 2 else B
    C3 = C.unsqueeze(1) if C.dim() == 2 else C
    if B3.shape[0] != b or B3.shape[2] != N or C3.shape != B3.shape:
        raise ValueError("selective_state_update: B/C must be (b, N) or (b, G, N)")
    G = B3.shape[1]
    dt_chan = dt.dim() == 3
    if dt.shape != ((b, H, P) if dt_chan else (b, H)):
        raise ValueError(f"selective_state_update: dt must be {(b, H)} or {(b, H, P)}")
    if not state.is_contiguous():
        raise ValueError("selective_state_update: state must be contiguous (it is updated in place)")
    xs = x if (x.stride(-1) == 1 and x.stride(-2) == P) else x.contiguous()
    Bs = B3 if (B3.stride(-1) == 1 and B3.stride(-2) == N) else B3.contiguous()
    Cs = C3 if (C3.stride(-1) == 1 and C3.stride(-2) == N) else C3.contiguous()
    if A.numel() != (N if A_per_state else H):
        raise ValueError(f"selective_state_update: A must have {'N' if A_per_state else 'H'} entries")
    if D is not None and D.numel() not in (H, H * P):
        raise ValueError("selective_state_update: D must have H or H*P entries")
    if dt_bias is not None and dt_bias.numel() != (H * P if dt_chan else H):
        raise ValueError(f"selective_state_update: dt_bias must have one entry per {'channel' if dt_chan else 'head'}")
    if H % G:
        raise ValueError("selective_state_update: nheads must be a multiple of ngroups")
    dt32 = dt.to(torch.float32)
    if dt32.stride(-1) != 1 or (dt_chan and dt32.stride(-2) != P):
        dt32 = dt32.contiguous()
    A32, D32, bias32 = _f32c(A), _f32c(D.reshape(-1) if D is not None else None), _f32c(dt_bias)
    dst = state if out_state is None else out_state
    if dst is not state and (dst.shape != state.shape or dst.dtype != torch.float32 or not dst.is_contiguous()):
        raise ValueError("selective_state_update: out_state must match state")
    zs = None
    if z is not None:
        if z.shape != (b, H, P) or z.dtype != x.dtype:
            raise ValueError(f"selective_state_update: z must be {(b, H, P)} in the dtype of x")
        zs = z if (z.stride(-1) == 1 and z.stride(-2) == P) else z.contiguous()
    y = torch.empty((b, H, P), device=x.device, dtype=x.dtype)
    a = SsuArgs()
    a.batch, a.nheads, a.headdim, a.dstate, a.ngroups = b, H, P, N, G
    a.dtype = _DT[x.dtype]
    flags = _lib.MH_DT_SOFTPLUS if dt_softplus else 0
    if dt_limit is not None:
        flags |= _lib.MH_DT_LIMIT
        a.dt_min, a.dt_max = float(dt_limit[0]), float(dt_limit[1])
    if D32 is not None and D32.numel() == H * P and P != 1:
        flags |= _lib.MH_D_PER_CHANNEL
    if A_per_state:
        flags |= _lib.MH_A_PER_STATE
    if dt_chan:
        flags |= _lib.MH_DT_PER_CHANNEL
    a.flags = flags
    a.state_in, a.state_out = _ptr(state), _ptr(dst)
    a.x, a.x_stride_b = _ptr(xs), xs.stride(0)
    a.dt, a.dt_stride_b = _ptr(dt32), dt32.stride(0)
    a.A = _ptr(A32)
    a.B, a.B_stride_b = _ptr(Bs), Bs.stride(0)
    a.C, a.C_stride_b = _ptr(Cs), Cs.stride(0)
    a.D, a.dt_bias = _ptr(D32), _ptr(bias32)
    a.y, a.y_stride_b = _ptr(y), y.stride(0)
    if zs is not None:
        a.z, a.z_stride_b = _ptr(zs), zs.stride(0)
    plan = Plan("mh_ssd_state_update", a, x.device, keep=(state, dst, xs, dt32, A32, Bs, Cs, D32, bias32, zs), y=y)
    if _plan_only:
        return plan
    plan()
    return y


def recurrent_step(x, dt, B, C, h_prev, A, D, *, dt_bias=None, dt_softplus=False, dt_limit=None, z=None):
    """``Mamba2Block._recurrent_step`` counterpart (R/mamformer/layers/mamba2.py:407-458), per-head form.

    x (b, seqlen, H*P) -- only the last token is used (:435-438); dt (b, seqlen, H)
    (already softplus'ed, as at mamba2.py:293, unless ``dt_softplus``); B, C (b, seqlen, N)
    or (b, seqlen, G, N); h_prev (b, H*P, N) or None (zeros, :448-449); A (H,); D (H,) or (H*P,).
    Optional gate z (b, seqlen, H*P) (last token used): y_t <- y_t * silu(z_t) (mamba2.py:337-338).
    Returns (y_t (b, 1, H*P), h_t (b, H*P, N)) -- a new state tensor, as the reference returns.
    """
    b, _, d_inner = x.shape
    H = dt.shape[-1]
    P = d_inner // H
    Bl = B[:, -1]
    Cl = C[:, -1]
    N = Bl.shape[-1]
    if h_prev is None:
        state = torch.zeros((b, H, P, N), device=x.device, dtype=torch.float32)
    else:
        state = h_prev.reshape(b, H, P, N).to(torch.float32)
    out = torch.empty((b, H, P, N), device=x.device, dtype=torch.float32)
    zl = z[:, -1].reshape(b, H, P) if z is not None else None
    y = selective_state_update(state.contiguous(), x[:, -1].reshape(b, H, P), dt[:, -1], A, Bl, Cl, D,
                               dt_bias=dt_bias, dt_softplus=dt_softplus, dt_limit=dt_limit, out_state=out, z=zl)
    return y.reshape(b, 1, d_inner), out.view(b, d_inner, N)


def recurrent_step_reference(x, dt, B, C, h_prev, A_log, D):
    """``Mamba2Block._recurrent_step`` (R/mamformer/layers/mamba2.py:407-458) in the reference's own
    parameterisation, on the GPU: a decay rate per state column and a step per channel,
        a[c, n] = exp(-exp(A_log[n]) dt[c]),  h[c, n] <- a[c, n] h[c, n] + dt[c] x[c] B[n],
        y[c] = sum_n C[n] h[c, n] + D[c] x[c].
    x, dt (b, seqlen, d_inner) -- only the last token is used (:435-438), dt already positive (the block
    applies softplus before the call); B, C (b, seqlen, N); h_prev (b, d_inner, N) or None (zeros,
    :448-449); A_log (N,) unclamped (:441-443); D (d_inner,).  Returns (y_t (b, 1, d_inner) in the dtype of x,
    h_t (b, d_inner, N) float32), a new state as the reference returns.
    """
    b, _, d_inner = x.shape
    N = B.shape[-1]
    P = next(p for p in (64, 32, 16, 8, 4, 2, 1) if d_inner % p == 0)    # channels per kernel row group
    H = d_inner // P
    if h_prev is None:
        state = torch.zeros((b, H, P, N), device=x.device, dtype=torch.float32)
    else:
        state = h_prev.reshape(b, H, P, N).to(torch.float32).contiguous()
    out = torch.empty((b, H, P, N), device=x.device, dtype=torch.float32)
    A = -torch.exp(A_log.to(torch.float32))
    y = selective_state_update(state, x[:, -1].reshape(b, H, P), dt[:, -1].reshape(b, H, P), A, B[:, -1],
                               C[:, -1], D, dt_softplus=False, out_state=out, A_per_state=True)
    return y.reshape(b, 1, d_inner), out.view(b, d_inner, N)


def selective_scan_reference(x, dt, A, B, C, D, return_h_states=False, return_final_state=False, *,
                             initial_state=None, dt_bias=None, dt_softplus=False, dt_limit=None, z=None,
                             _plan_only=False):
    """``selective_scan`` (R/mamformer/layers/mamba2.py:31-130) in the reference's own parameterisation, on the GPU:
    a decay rate per state column and a step size per channel,
        h_t[c, n] = exp(-exp(clamp(A[n], -5, 5)) dt_t[c]) h_{t-1}[c, n] + dt_t[c] x_t[c] B_t[n],
        y_t[c] = sum_n C_t[n] h_t[c, n] + D[c] x_t[c].
    Same arguments and return order as the reference: x, dt (b, L, d_inner) (dt already positive, as the block's
    softplus leaves it; ``dt_softplus`` / ``dt_bias`` / ``dt_limit`` apply the prologue in-kernel instead), A the
    log-rates A_log (N,) clamped to [-5, 5] as in :87, B, C (b, L, N), D (d_inner,) or None.  Returns y, or a tuple
    (y, h_states (b, L, N) in the dtype of x, final_state (b, d_inner, N) float32) as requested (:121-130).
    ``initial_state`` (b, d_inner, N) seeds the state (the reference starts at zero); ``z`` (b, L, d_inner) applies
    the block's gate y * silu(z) (mamba2.py:337-338), in the kernel without autograd.  x / B / C / z bf16 or fp32
    (y in that dtype), state and arithmetic fp32.  Differentiable: under autograd the backward is
    ``mh_ssd_ref_scan_bwd`` (A_log's gradient passes through the clamp and the exponential in torch) and the gate's
    ``mh_silu_gate_bwd``."""
    _require_cuda("selective_scan_reference", x, dt, A, B, C, D, initial_state, dt_bias, z)
    if x.dim() != 3 or dt.shape != x.shape:
        raise ValueError("selective_scan_reference: x and dt must be (batch, seqlen, d_inner)")
    b, L, di = x.shape
    if B.dim() == 4:
        B, C = B.squeeze(2), C.squeeze(2)
    N = A.shape[0]
    if B.shape != (b, L, N) or C.shape != (b, L, N):
        raise ValueError(f"selective_scan_reference: B and C must be (batch, seqlen, {N})")
    if x.dtype not in _DT:
        raise TypeError(f"selective_scan_reference: unsupported dtype {x.dtype}")
    P = next(p for p in (64, 32, 16) if di % p == 0) if di % 16 == 0 else None
    if P is None:
        raise ValueError("selective_scan_reference: d_inner must be a multiple of 16")
    H = di // P
    if D is not None and D.numel() != di:
        raise ValueError("selective_scan_reference: D must have d_inner entries")
    dt32 = _inner_contig(dt.to(torch.float32))
    if dt32.stride(1) % 4 or dt32.stride(0) % 4:
        dt32 = dt32.contiguous()
    rates = (-torch.exp(torch.clamp(A.to(torch.float32), min=-5.0, max=5.0))).contiguous()
    xc = _inner_contig(x)
    Bc = _inner_contig(B.to(x.dtype))
    Cc = _inner_contig(C.to(x.dtype))
    D32 = _f32c(D)
    h0 = None if initial_state is None else initial_state.to(torch.float32).reshape(b, di, N).contiguous()
    bias32 = _f32c(dt_bias)
    zc = None if z is None else _inner_contig(z.to(x.dtype))
    cfg = (dt_softplus, dt_limit, H, P)
    if not _plan_only and torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (xc, dt32, rates, Bc, Cc, D32, h0, bias32, zc)):
        y, hs, fin = _RefScanFn.apply(xc, dt32, rates, Bc, Cc, D32, h0, bias32, cfg, return_h_states)
        if zc is not None:
            y = _GateFn.apply(y.view(b, L, H, P), zc.view(b, L, H, P)).view(b, L, di)
        out = [y] + ([hs] if return_h_states else []) + ([fin] if return_final_state else [])
        return out[0] if len(out) == 1 else tuple(out)
    y = torch.empty((b, L, di), device=x.device, dtype=x.dtype)
    fin = torch.empty((b, di, N), device=x.device, dtype=torch.float32) if return_final_state else None
    hs = torch.empty((b, L, N), device=x.device, dtype=x.dtype) if return_h_states else None
    a = _ref_args(xc, dt32, rates, Bc, Cc, D32, h0, bias32, cfg, y, fin, zc)
    n = ct.c_size_t()
    _lib.call("mh_ssd_ref_scan_workspace_bytes", ct.byref(a), int(return_h_states), ct.byref(n))
    ws = torch.empty(max(n.value, 1), device=x.device, dtype=torch.uint8) if n.value else None
    a.workspace, a.workspace_bytes = _ptr(ws), n.value
    if _plan_only:
        return _RefScanPlan(a, _ptr(hs), x.device, keep=(xc, dt32, rates, Bc, Cc, D32, h0, bias32, zc, ws), y=y,
                            h_states=hs, final_state=fin)
    _lib.call("mh_ssd_ref_scan_fwd", ct.byref(a), _ptr(hs), _stream(x.device))
    out = [y]
    if return_h_states:
        out.append(hs)
    if return_final_state:
        out.append(fin)
    return out[0] if len(out) == 1 else tuple(out)


def _ref_args(xc, dt32, rates, Bc, Cc, D32, h0, bias32, cfg, y, fin, zc):
    """``mh_ssd_args`` of the reference-form scan: (b, L, d_inner) rows seen as H heads of P channels."""
    dt_softplus, dt_limit, H, P = cfg
    b, L, di = xc.shape
    N = rates.shape[0]
    a = _ssd_args(xc.view(b, L, H, P), dt32, rates, Bc.view(b, L, 1, N), Cc.view(b, L, 1, N), None, bias32,
                  dt_softplus, dt_limit, h0, (xc if y is None else y).view(b, L, H, P), fin, None,
                  None if zc is None else zc.view(b, L, H, P))
    flags = a.flags | _lib.MH_A_PER_STATE | _lib.MH_DT_PER_CHANNEL
    if D32 is not None:
        a.D = _ptr(D32)
        if D32.numel() == di:
            flags |= _lib.MH_D_PER_CHANNEL
    a.flags = flags
    # the (b, L, d_inner) rows: strides of the flattened channel axis
    a.x_stride_h = a.y_stride_h = P
    if zc is not None:
        a.z_stride_h = P
    return a


class _RefScanFn(torch.autograd.Function):
    """Autograd node of the reference-form scan: forward ``mh_ssd_ref_scan_fwd`` (y ungated, h_states when asked,
    the final state), backward ``mh_ssd_ref_scan_bwd`` (every gradient, w.r.t. the rates A; torch chains A_log)."""

    @staticmethod
    def forward(ctx, xc, dt32, rates, Bc, Cc, D32, h0, bias32, cfg, want_hs):
        b, L, di = xc.shape
        N = rates.shape[0]
        y = torch.empty((b, L, di), device=xc.device, dtype=xc.dtype)
        fin = torch.empty((b, di, N), device=xc.device, dtype=torch.float32)
        hs = torch.empty((b, L, N), device=xc.device, dtype=xc.dtype) if want_hs else None
        a = _ref_args(xc, dt32, rates, Bc, Cc, D32, h0, bias32, cfg, y, fin, None)
        n = ct.c_size_t()
        _lib.call("mh_ssd_ref_scan_workspace_bytes", ct.byref(a), int(want_hs), ct.byref(n))
        ws = torch.empty(max(n.value, 1), device=xc.device, dtype=torch.uint8) if n.value else None
        a.workspace, a.workspace_bytes = _ptr(ws), n.value
        _lib.call("mh_ssd_ref_scan_fwd", ct.byref(a), _ptr(hs), _stream(xc.device))
        ctx.save_for_backward(xc, dt32, rates, Bc, Cc, D32, h0, bias32)
        ctx.cfg = cfg
        ctx.set_materialize_grads(False)
        return y, hs, fin

    @staticmethod
    def backward(ctx, dy, dhs, dfin):
        xc, dt32, rates, Bc, Cc, D32, h0, bias32 = ctx.saved_tensors
        b, L, di = xc.shape
        N = rates.shape[0]
        dev = xc.device
        g = _lib.SsdRefBwdArgs()
        g.fwd = _ref_args(xc, dt32, rates, Bc, Cc, D32, h0, bias32, ctx.cfg, None, None, None)
        dy = None if dy is None else dy.to(xc.dtype).contiguous()
        dhs = None if dhs is None else dhs.to(xc.dtype).contiguous()
        dfin = None if dfin is None else dfin.to(torch.float32).contiguous()
        dx = torch.empty((b, L, di), device=dev, dtype=xc.dtype)
        ddt = torch.empty((b, L, di), device=dev, dtype=torch.float32)
        dA = torch.empty((N,), device=dev, dtype=torch.float32)
        dB = torch.empty((b, L, N), device=dev, dtype=xc.dtype)
        dC = torch.empty((b, L, N), device=dev, dtype=xc.dtype)
        dD = None if D32 is None else torch.empty_like(D32)
        dbias = None if bias32 is None else torch.empty_like(bias32)
        need_dh0 = h0 is not None and ctx.needs_input_grad[6]
        dh0 = torch.empty((b, di, N), device=dev, dtype=torch.float32) if need_dh0 else None
        g.dy, g.dhs, g.d_final_state = _ptr(dy), _ptr(dhs), _ptr(dfin)
        g.dx, g.ddt, g.dA, g.dB, g.dC = _ptr(dx), _ptr(ddt), _ptr(dA), _ptr(dB), _ptr(dC)
        g.dD, g.d_dt_bias, g.d_initial_state = _ptr(dD), _ptr(dbias), _ptr(dh0)
        n = ct.c_size_t()
        _lib.call("mh_ssd_ref_scan_bwd_workspace_bytes", ct.byref(g), ct.byref(n))
        ws = torch.empty(max(n.value, 16), device=dev, dtype=torch.uint8)
        g.workspace, g.workspace_bytes = _ptr(ws), n.value
        _lib.call("mh_ssd_ref_scan_bwd", ct.byref(g), _stream(dev))
        return dx, ddt, dA, dB, dC, dD, dh0, dbias, None, None


class _RefScanPlan(Plan):
    """``Plan`` of ``mh_ssd_ref_scan_fwd``, whose h_states pointer is an argument of its own."""

    def __init__(self, args, hs_ptr, device, keep=(), **outputs):
        super().__init__("mh_ssd_ref_scan_fwd", args, device, keep, **outputs)
        self._hs = hs_ptr

    def __call__(self, stream=None):
        s = _stream(self._device) if stream is None else ct.c_void_p(stream)
        _lib.call(self._fn, ct.byref(self._args), self._hs, s)
        return self


def plan_selective_scan_reference(*args, **kw):
    """``Plan`` of ``selective_scan_reference`` on fixed buffers (outputs ``y``, ``h_states``, ``final_state``)."""
    return selective_scan_reference(*args, _plan_only=True, **kw)


def plan_linear_attn_scan(*args, **kw):
    """``Plan`` of ``linear_attn_scan`` on fixed buffers (outputs ``o``, ``o2``, ``final_state``, ``final_z``)."""
    return linear_attn_scan(*args, _plan_only=True, **kw)


def diff_lambda(lambda_raw):
    """lambda = min(sigmoid(lambda_raw), 0.99) per head (R/mamformer/layers/kda_diff.py:473-474)."""
    return torch.clamp(torch.sigmoid(lambda_raw.to(torch.float32)), max=0.99)


def linear_attn_scan(q1, q2, k, v, *, g=None, lam=0.8, mode="gated", kernel_dim=None, initial_state=None,
                     initial_z=None, return_final_state=False, pair=False, chunk_size=64, _plan_only=False):
    """KDA linear-attention chunked scan on the GPU, layout (B, H, S, D) as the reference (kda_diff.py:270-273).

    mode="gated" (benchmark operator, no reference function):
        S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,  o_t = q1_t S_t - lam q2_t S_t
        g (B, H, S, dk) fp32 per-channel log-decay or None (no decay); lam a float or (H,) tensor;
        q2 may be None (single query).  Returns o, or (o, final_state (B, H, dk, dv) fp32).
    mode="reference" (the reference's normalised scan, triton_ssd.py:121-181 / kda_diff.py:357-478):
        phi(x) = elu(x) + 1 on the first ``kernel_dim`` channels;  S_t = S_{t-1} + phi(k_t)^T v_t,
        z_t = z_{t-1} + phi(k_t),  o_i,t = phi(q_i,t) S_t / (phi(q_i,t) z_t + 1e-8).
        ``pair=True`` returns (o1, o2) like ``triton_linear_attn_scan``; otherwise the differential
        combination (o1 - lam o2) / (1 - lam + 1e-8) is fused into the kernel and returned as one tensor
        (q2=None: the single-query o1).  ``initial_state`` (B, H, dk, dv) / ``initial_z`` (B, H, dk) seed the
        accumulators (the reference always starts at zero); with ``return_final_state`` the result gains
        (final_state, final_z).
    chunk_size: accepted for API compatibility; the kernels walk segments of <= 64 tokens.
    """
    if mode not in ("gated", "reference"):
        raise ValueError(f"linear_attn_scan: unknown mode {mode!r} (gated, reference)")
    ref_mode = mode == "reference"
    _require_cuda("linear_attn_scan", q1, q2, k, v, g, initial_state, initial_z)
    if q1.dim() != 4:
        raise ValueError("linear_attn_scan: q1 must be (B, H, S, dk)")
    Bb, H, S, dk = q1.shape
    dv = v.shape[-1]
    if k.shape != q1.shape or (q2 is not None and q2.shape != q1.shape) or v.shape[:3] != (Bb, H, S):
        raise ValueError("linear_attn_scan: q1/q2/k must be (B, H, S, dk) and v (B, H, S, dv)")
    if q1.dtype not in _DT or any(t is not None and t.dtype != q1.dtype for t in (q2, k, v)):
        raise TypeError("linear_attn_scan: q1, q2, k, v must share a dtype")
    if ref_mode and g is not None:
        raise ValueError("linear_attn_scan: reference mode has no gate g")
    if pair and (not ref_mode or q2 is None):
        raise ValueError("linear_attn_scan: pair=True needs mode='reference' and two queries")
    q1c, kc, vc = q1.contiguous(), k.contiguous(), v.contiguous()
    q2c = q2.contiguous() if q2 is not None else None
    gc = None
    if g is not None:
        if g.shape != (Bb, H, S, dk):
            raise ValueError("linear_attn_scan: g must be (B, H, S, dk)")
        gc = g.to(torch.float32).contiguous()
    lam_h = None
    if torch.is_tensor(lam):
        lam_h = lam.to(device=q1.device, dtype=torch.float32).reshape(-1).contiguous()
        if lam_h.numel() != H:
            raise ValueError("linear_attn_scan: per-head lam must have H entries")
        lam_f = 0.0
    else:
        lam_f = float(lam)
    s0 = z0 = None
    if initial_state is not None:
        if initial_state.numel() != Bb * H * dk * dv:
            raise ValueError("linear_attn_scan: initial_state must be (B, H, dk, dv)")
        s0 = initial_state.reshape(Bb, H, dk, dv).to(torch.float32).contiguous()
    if initial_z is not None:
        if not ref_mode or initial_z.numel() != Bb * H * dk:
            raise ValueError("linear_attn_scan: initial_z (B, H, dk) is a reference-mode input")
        z0 = initial_z.reshape(Bb, H, dk).to(torch.float32).contiguous()
    if not _plan_only and torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q1c, q2c, kc, vc, gc, lam_h, s0, z0)):
        if not ref_mode:
            raise RuntimeError("linear_attn_scan: the gated operator has no backward (it has no reference "
                               "training path); use mode='reference' or call it under torch.no_grad()")
        cfg = (a_kernel_dim(kernel_dim, dk), pair, return_final_state, lam_f)
        outs = _KdaRefFn.apply(q1c, q2c, kc, vc, lam_h, s0, z0, cfg)
        return outs if len(outs) > 1 else outs[0]
    o = torch.empty((Bb, H, S, dv), device=q1.device, dtype=q1.dtype)
    o2 = torch.empty((Bb, H, S, dv), device=q1.device, dtype=q1.dtype) if pair else None
    fin = torch.empty((Bb, H, dk, dv), device=q1.device, dtype=torch.float32) if return_final_state else None
    finz = (torch.empty((Bb, H, dk), device=q1.device, dtype=torch.float32)
            if (return_final_state and ref_mode) else None)
    a = KdaArgs()
    a.batch, a.nheads, a.seqlen, a.dk, a.dv = Bb, H, S, dk, dv
    a.dtype = _DT[q1.dtype]
    a.mode = _lib.MH_KDA_REFERENCE if ref_mode else _lib.MH_KDA_GATED
    a.kernel_dim = int(kernel_dim) if (ref_mode and kernel_dim is not None) else dk
    a.lam = lam_f
    a.lam_per_head = _ptr(lam_h)
    a.q1, a.q2, a.k, a.v, a.g = _ptr(q1c), _ptr(q2c), _ptr(kc), _ptr(vc), _ptr(gc)
    a.initial_state, a.final_state = _ptr(s0), _ptr(fin)
    a.initial_z, a.final_z = _ptr(z0), _ptr(finz)
    a.o, a.o2 = _ptr(o), _ptr(o2)
    plan = Plan("mh_kda_chunk_scan_fwd", a, q1.device, keep=(q1c, q2c, kc, vc, gc, lam_h, s0, z0),
                o=o, o2=o2, final_state=fin, final_z=finz)
    if _plan_only:
        return plan
    plan()
    out = (o, o2) if pair else (o,)
    if return_final_state:
        out = out + ((fin, finz) if ref_mode else (fin,))
    return out if len(out) > 1 else out[0]


def a_kernel_dim(kernel_dim, dk):
    return int(kernel_dim) if kernel_dim is not None else dk


class _KdaRefFn(torch.autograd.Function):
    """Autograd node of the reference-mode KDA scan: forward = ``mh_kda_chunk_scan_fwd``, backward =
    ``mh_kda_chunk_scan_bwd`` (the gradient autograd forms through kda_diff.py:357-478)."""

    @staticmethod
    def forward(ctx, q1, q2, k, v, lam_h, s0, z0, cfg):
        kd, pair, ret_fin, lam_f = cfg
        res = linear_attn_scan(q1, q2, k, v, mode="reference", kernel_dim=kd, lam=lam_h if lam_h is not None
                               else lam_f, initial_state=s0, initial_z=z0, return_final_state=ret_fin, pair=pair)
        res = res if isinstance(res, tuple) else (res,)
        ctx.save_for_backward(q1, q2, k, v, lam_h, s0, z0)
        ctx.cfg = cfg
        return res

    @staticmethod
    def backward(ctx, *grads):
        q1, q2, k, v, lam_h, s0, z0 = ctx.saved_tensors
        kd, pair, ret_fin, lam_f = ctx.cfg
        n_o = 2 if pair else 1
        g_o = list(grads[:n_o])
        g_fin, g_finz = (grads[n_o], grads[n_o + 1]) if ret_fin else (None, None)
        r = linear_attn_scan_bwd(q1, q2, k, v, kernel_dim=kd, lam=lam_h if lam_h is not None else lam_f,
                                 do1=g_o[0], do2=g_o[1] if pair else None, pair=pair, initial_state=s0,
                                 initial_z=z0, d_final_state=g_fin, d_final_z=g_finz,
                                 need_initial=(ctx.needs_input_grad[5] or ctx.needs_input_grad[6]))
        dlam = r.get("d_lam") if (lam_h is not None and ctx.needs_input_grad[4]) else None
        return (r["dq1"], r.get("dq2"), r["dk"], r["dv"], dlam,
                r.get("d_initial_state") if ctx.needs_input_grad[5] else None,
                r.get("d_initial_z") if ctx.needs_input_grad[6] else None, None)


def linear_attn_scan_bwd(q1, q2, k, v, *, kernel_dim=None, lam=0.8, do1=None, do2=None, pair=False,
                         initial_state=None, initial_z=None, d_final_state=None, d_final_z=None, need_initial=True):
    """Gradients of the reference-mode scan (``linear_attn_scan(..., mode="reference")``) on the GPU.

    Loss = <do1, o1> + <do2, o2> (``pair=True``), <do1, out> for the fused differential output
    out = (o1 - lam o2) / (1 - lam + 1e-8) (two queries, ``pair=False``) or <do1, o1> (single query), plus
    <d_final_state, S_final> + <d_final_z, z_final>.  Shapes as ``linear_attn_scan``; any gradient may be None
    (zero).  Returns a dict: dq1, dq2 (with q2), dk, dv (dtype of q1), d_lam (H,) fp32 for the differential
    output, and with ``need_initial`` d_initial_state (B, H, dk, dv) and d_initial_z (B, H, dk) fp32.
    """
    _require_cuda("linear_attn_scan_bwd", q1, q2, k, v, do1, do2, initial_state, initial_z, d_final_state,
                  d_final_z)
    Bb, H, S, dk = q1.shape
    dv = v.shape[-1]
    if q1.dtype not in _DT or any(t is not None and t.dtype != q1.dtype for t in (q2, k, v)):
        raise TypeError("linear_attn_scan_bwd: q1, q2, k, v must share a dtype")
    if pair and q2 is None:
        raise ValueError("linear_attn_scan_bwd: pair=True needs q2")
    diff = q2 is not None and not pair
    q1c, kc, vc = q1.contiguous(), k.contiguous(), v.contiguous()
    q2c = q2.contiguous() if q2 is not None else None

    def grad_like(t):
        return None if t is None else t.to(q1.dtype).contiguous()

    do1c = grad_like(do1) if do1 is not None else torch.zeros_like(vc)
    do2c = grad_like(do2) if (pair and do2 is not None) else None
    lam_h = None
    if torch.is_tensor(lam):
        lam_h = lam.to(device=q1.device, dtype=torch.float32).reshape(-1).contiguous()
        lam_f = 0.0
    else:
        lam_f = float(lam)

    def f32(t, n):
        if t is None:
            return None
        if t.numel() != n:
            raise ValueError("linear_attn_scan_bwd: state tensors must be (B, H, dk, dv) / (B, H, dk)")
        return t.to(torch.float32).contiguous()

    s0, z0 = f32(initial_state, Bb * H * dk * dv), f32(initial_z, Bb * H * dk)
    dfs, dfz = f32(d_final_state, Bb * H * dk * dv), f32(d_final_z, Bb * H * dk)
    dq1 = torch.empty_like(q1c)
    dq2 = torch.empty_like(q2c) if q2c is not None else None
    dkk, dvv = torch.empty_like(kc), torch.empty_like(vc)
    dS0 = torch.empty((Bb, H, dk, dv), device=q1.device, dtype=torch.float32) if need_initial else None
    dz0 = torch.empty((Bb, H, dk), device=q1.device, dtype=torch.float32) if need_initial else None
    dlam = torch.empty(H, device=q1.device, dtype=torch.float32) if diff else None
    a = _lib.KdaBwdArgs()
    f = a.fwd
    f.batch, f.nheads, f.seqlen, f.dk, f.dv = Bb, H, S, dk, dv
    f.dtype = _DT[q1.dtype]
    f.mode = _lib.MH_KDA_REFERENCE
    f.kernel_dim = a_kernel_dim(kernel_dim, dk)
    f.lam, f.lam_per_head = lam_f, _ptr(lam_h)
    f.q1, f.q2, f.k, f.v = _ptr(q1c), _ptr(q2c), _ptr(kc), _ptr(vc)
    f.initial_state, f.initial_z = _ptr(s0), _ptr(z0)
    a.flags = _lib.MH_KDA_BWD_DIFF if diff else 0
    a.do1, a.do2 = _ptr(do1c), _ptr(do2c)
    a.d_final_state, a.d_final_z = _ptr(dfs), _ptr(dfz)
    a.dq1, a.dq2, a.dk, a.dv = _ptr(dq1), _ptr(dq2), _ptr(dkk), _ptr(dvv)
    a.d_initial_state, a.d_initial_z, a.d_lam = _ptr(dS0), _ptr(dz0), _ptr(dlam)
    n = ct.c_size_t()
    _lib.call("mh_kda_bwd_workspace_bytes", ct.byref(a), ct.byref(n))
    ws = torch.empty(max(n.value, 16), device=q1.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = _ptr(ws), ws.numel()
    _lib.call("mh_kda_chunk_scan_bwd", ct.byref(a), _stream(q1.device))
    res = {"dq1": dq1, "dk": dkk, "dv": dvv}
    if dq2 is not None:
        res["dq2"] = dq2
    if dlam is not None:
        res["d_lam"] = dlam
    if need_initial:
        res["d_initial_state"], res["d_initial_z"] = dS0, dz0
    return res


def linear_attn_scan_pair(q1, q2, k, v, kernel_dim, block_k=128, block_d=128, group_h=0):
    """``triton_linear_attn_scan`` counterpart (R/mamformer/kernels/triton_ssd.py:260-350): raw q1, q2, k, v
    (B, H, S, D) -> (o1, o2) of the phi(x)=elu(x)+1 normalised scan.  ``block_k``/``block_d``/``group_h`` are the
    Triton tiling knobs, accepted and ignored (the HIP kernel's tiling is fixed)."""
    return linear_attn_scan(q1, q2, k, v, mode="reference", kernel_dim=kernel_dim, pair=True)


def linear_attn_scan_single(q, k, v, kernel_dim, block_k=128, block_d=128):
    """``triton_linear_attn_scan_single`` counterpart (triton_ssd.py:353-400): one query stream -> o."""
    return linear_attn_scan(q, None, k, v, mode="reference", kernel_dim=kernel_dim)


def linear_attention_scan(q1, q2, k, v, kernel_dim, lambda_raw):
    """``LinearDiffAttention._linear_attention_scan`` counterpart (R/mamformer/layers/kda_diff.py:357-478):
    the normalised scan of both queries with the differential combination
    (o1 - lam o2) / (1 - lam + 1e-8), lam = min(sigmoid(lambda_raw), 0.99) per head, fused into the kernel.
    Starts from a zero state, as the reference does."""
    return linear_attn_scan(q1, q2, k, v, mode="reference", kernel_dim=kernel_dim, lam=diff_lambda(lambda_raw))


def plan_linear_attn_step(*args, **kw):
    """``Plan`` of ``linear_attn_step`` on fixed buffers (output ``o``; state and z are updated per call)."""
    return linear_attn_step(*args, _plan_only=True, **kw)


def linear_attn_step(state, z, q1, q2, k, v, *, lam=0.8, kernel_dim=None, apply_phi=True, pair=False,
                     _plan_only=False):
    """One-token step of the reference-mode scan, updating ``state`` and ``z`` in place (KDA decode).

    state (B, H, dk, dv) fp32 contiguous; z (B, H, dk) or (B, H, dk, 1) fp32 contiguous; q1, q2, k
    (B, H, dk) or (B, H, 1, dk); v (B, H, dv) or (B, H, 1, dv).  ``apply_phi``: q/k are raw and
    phi(x) = elu(x)+1 is applied to their first ``kernel_dim`` channels in the kernel (else they are already
    feature-mapped).  Returns the differential output (o1 - lam o2) / (1 - lam + 1e-8) shaped like v
    (q2=None: o1; ``pair=True``: (o1, o2)).  Semantics of ``_linear_attention_recurrent``
    (R/mamformer/layers/kda_diff.py:564-605) with the cache update of kda_diff.py:329-338.
    """
    _require_cuda("linear_attn_step", state, z, q1, q2, k, v)
    if state.dim() != 4 or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError("linear_attn_step: state must be a contiguous (B, H, dk, dv) float32 tensor")
    Bb, H, dk, dv = state.shape
    if z.dtype != torch.float32 or not z.is_contiguous() or z.numel() != Bb * H * dk:
        raise ValueError("linear_attn_step: z must be a contiguous float32 (B, H, dk[, 1]) tensor")
    if pair and q2 is None:
        raise ValueError("linear_attn_step: pair=True needs q2")
    if q1.dtype not in _DT or any(t is not None and t.dtype != q1.dtype for t in (q2, k, v)):
        raise TypeError("linear_attn_step: q1, q2, k, v must share a dtype")

    def rows(t, d, name):
        if t is None:
            return None
        if t.numel() != Bb * H * d:
            raise ValueError(f"linear_attn_step: {name} must hold B*H*{d} values (one token)")
        return t.reshape(Bb, H, d).contiguous()

    q1c, q2c, kc, vc = rows(q1, dk, "q1"), rows(q2, dk, "q2"), rows(k, dk, "k"), rows(v, dv, "v")
    lam_h = None
    if torch.is_tensor(lam):
        lam_h = lam.to(device=state.device, dtype=torch.float32).reshape(-1).contiguous()
        if lam_h.numel() != H:
            raise ValueError("linear_attn_step: per-head lam must have H entries")
        lam_f = 0.0
    else:
        lam_f = float(lam)
    o = torch.empty((Bb, H, dv), device=state.device, dtype=q1.dtype)
    o2 = torch.empty((Bb, H, dv), device=state.device, dtype=q1.dtype) if pair else None
    a = _lib.KdaStepArgs()
    a.batch, a.nheads, a.dk, a.dv = Bb, H, dk, dv
    a.dtype = _DT[q1.dtype]
    a.flags = _lib.MH_KDA_PHI if apply_phi else 0
    a.kernel_dim = int(kernel_dim) if kernel_dim is not None else dk
    a.lam = lam_f
    a.lam_per_head = _ptr(lam_h)
    a.q1, a.q2, a.k, a.v = _ptr(q1c), _ptr(q2c), _ptr(kc), _ptr(vc)
    a.state, a.z = _ptr(state), _ptr(z)
    a.o, a.o2 = _ptr(o), _ptr(o2)
    plan = Plan("mh_kda_recurrent_step", a, state.device, keep=(state, z, q1c, q2c, kc, vc, lam_h), o=o, o2=o2)
    if _plan_only:
        return plan
    plan()
    shape = v.shape
    return (o.view(shape), o2.view(shape)) if pair else o.view(shape)


def linear_attention_recurrent(q1_phi, q2_phi, k_phi, v, S, z, lambda_raw):
    """``LinearDiffAttention._linear_attention_recurrent`` counterpart (R/mamformer/layers/kda_diff.py:564-605).

    q1_phi, q2_phi, k_phi (B, H, 1, K) already feature-mapped; v (B, H, 1, D); S (B, H, K, D); z (B, H, K, 1).
    Returns the differential output (B, H, 1, D).  As in the reference, S and z are not modified (the step
    runs on float32 copies); ``linear_attn_step`` is the in-place form for a float32 cache.
    """
    S32 = S.to(torch.float32).clone(memory_format=torch.contiguous_format)
    z32 = z.to(torch.float32).clone(memory_format=torch.contiguous_format)
    return linear_attn_step(S32, z32, q1_phi, q2_phi, k_phi, v, lam=diff_lambda(lambda_raw), apply_phi=False)
