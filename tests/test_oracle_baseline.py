"""Pins of the torch-CPU restatements in oracle/baseline.py -- CPU only.

``oracle/baseline.py`` is what ``bench.py`` times as the reference's CPU path, so each of its functions is
checked here against an independent construction:

* ``selective_scan_cpu`` (mamba2.py:84-126) against the direct SSD recurrence over the bridge, and the
  [-5, 5] clamp of A_log against its closed form;
* ``recurrent_step_cpu`` (mamba2.py:441-456) against the float64 ``ref_recurrent_step`` (itself pinned by the
  prefill/decode and bridge checks of test_oracle.py), against the direct SSD form over chained steps from a
  nonzero state, against the one-token closed form, and for the missing clamp (A_log beyond 5);
* ``linear_attention_scan_cpu`` (kda_diff.py:390-478) against the brute-force normalised attention matrix
  (through ``oracle.kda.ref_attention_scan``): float64 inputs keep float64 chunk tensors with an fp32 carry,
  fp32 inputs take the reference's bf16 intermediates; S not a multiple of the chunk, kernel_dim below the
  head size, lambda at the 0.99 clamp, and chunk-size invariance (which pins the S / z carry).

The ``test_planted_*`` tests plant one mistake each in a copy of the function (clamped A_log in the decode
step, a wrong broadcast of dt, a dropped chunk carry, an exclusive cumsum, a missing +1 of the feature map)
and check that the comparisons above catch it.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kda, ssd
from oracle.baseline import bridge, linear_attention_scan_cpu, recurrent_step_cpu, selective_scan_cpu
from tests.conftest import rel_l2

f64 = torch.float64


def t64(a):
    return torch.tensor(np.asarray(a), dtype=f64)


def step_case(rng, b=3, d_inner=12, N=5):
    x = rng.standard_normal((b, d_inner))
    dt = ssd.softplus(rng.standard_normal((b, d_inner)) - 1.0)
    B = rng.standard_normal((b, N))
    C = rng.standard_normal((b, N))
    h = 0.5 * rng.standard_normal((b, d_inner, N))
    A_log = rng.uniform(-1.0, 1.5, N)
    D = rng.standard_normal(d_inner)
    return x, dt, B, C, h, A_log, D


# ----------------------------------------------------------------- selective_scan_cpu

@pytest.mark.parametrize("G", [1, 2])
def test_selective_scan_cpu_matches_direct_ssd(rng, G):
    b, L, H, P, N = 2, 29, 4, 3, 6
    x = rng.standard_normal((b, L, H, P))
    dt = ssd.softplus(rng.standard_normal((b, L, H)) - 1.0)
    A = -np.exp(rng.uniform(0, np.log(8), H))
    Bm = rng.standard_normal((b, L, G, N))
    Cm = rng.standard_normal((b, L, G, N))
    D = rng.standard_normal(H)
    y_dir, h_dir = ssd.ssd_direct(x, dt, A, Bm, Cm, D)
    hpg = H // G
    for g in range(G):
        hs = slice(g * hpg, (g + 1) * hpg)
        x_ref, dt_ref, D_ref = bridge(t64(x[:, :, hs]), t64(dt[:, :, hs]), t64(A[hs]), t64(D[hs]))
        y, h = selective_scan_cpu(x_ref.double(), dt_ref.double(), torch.zeros(N, dtype=f64),
                                  t64(Bm[:, :, g]), t64(Cm[:, :, g]), D_ref.double())
        # the bridge computes in fp32 (bench inputs); the scan itself runs in the dtype it is given
        assert rel_l2(y.numpy().reshape(b, L, hpg, P), y_dir[:, :, hs]) < 1e-6
        assert rel_l2(h.numpy().reshape(b, hpg, P, N), h_dir[:, hs]) < 1e-6


def test_selective_scan_cpu_clamps_A_log(rng):
    """A_log = 7 and -7 act as 5 and -5 (mamba2.py:87): one token, zero state, closed form."""
    b, d_inner, N = 1, 3, 4
    x = rng.standard_normal((b, 2, d_inner))
    dt = np.full((b, 2, d_inner), 0.3)
    B = rng.standard_normal((b, 2, N))
    C = rng.standard_normal((b, 2, N))
    A_log = np.array([7.0, -7.0, 0.5, 4.0])
    y, h = selective_scan_cpu(t64(x), t64(dt), t64(A_log), t64(B), t64(C), torch.zeros(d_inner, dtype=f64))
    a = np.exp(np.clip(A_log, -5, 5))
    h1 = B[:, 0, None, :] * dt[:, 0, :, None] * x[:, 0, :, None]
    h2 = np.exp(-a[None, None, :] * dt[:, 1, :, None]) * h1 + B[:, 1, None, :] * dt[:, 1, :, None] * x[:, 1, :, None]
    assert rel_l2(h.numpy(), h2) < 1e-12
    assert rel_l2(y.numpy()[:, 1], np.sum(C[:, 1, None, :] * h2, -1)) < 1e-12


# ----------------------------------------------------------------- recurrent_step_cpu

def test_recurrent_step_cpu_matches_float64_oracle(rng):
    x, dt, B, C, h, A_log, D = step_case(rng)
    y, hn = recurrent_step_cpu(t64(x), t64(dt), t64(B), t64(C), t64(h), t64(A_log), t64(D))
    y_ref, h_ref = ssd.ref_recurrent_step(x[:, None], dt[:, None], B[:, None], C[:, None], h, A_log, D)
    assert rel_l2(y.numpy(), y_ref[:, 0]) < 1e-13
    assert rel_l2(hn.numpy(), h_ref) < 1e-13


def test_recurrent_step_cpu_fp32_inputs(rng):
    x, dt, B, C, h, A_log, D = step_case(rng, b=4, d_inner=64, N=16)
    t32 = lambda a: torch.tensor(np.asarray(a), dtype=torch.float32)
    y, hn = recurrent_step_cpu(t32(x), t32(dt), t32(B), t32(C), t32(h), t32(A_log), t32(D))
    y_ref, h_ref = ssd.ref_recurrent_step(x[:, None], dt[:, None], B[:, None], C[:, None], h, A_log, D)
    assert rel_l2(y.numpy(), y_ref[:, 0]) < 1e-6
    assert rel_l2(hn.numpy(), h_ref) < 1e-6


def test_recurrent_step_cpu_chained_equals_direct_ssd_from_state(rng):
    """Steps through the bridge (A_log = 0, dt_ref = -A dt, x_ref = x / -A, D_ref = -A D) from a nonzero state
    h0 reproduce the direct SSD recurrence token by token, and its final state."""
    b, L, H, P, N = 2, 9, 3, 4, 5
    x = rng.standard_normal((b, L, H, P))
    dt = ssd.softplus(rng.standard_normal((b, L, H)) - 1.0)
    A = -np.exp(rng.uniform(0, np.log(8), H))
    Bm = rng.standard_normal((b, L, 1, N))
    Cm = rng.standard_normal((b, L, 1, N))
    D = rng.standard_normal(H)
    h0 = 0.3 * rng.standard_normal((b, H, P, N))
    y_dir, h_dir = ssd.ssd_direct(x, dt, A, Bm, Cm, D, initial_state=h0)
    x_ref, dt_ref, D_ref = bridge(t64(x), t64(dt), t64(A), t64(D))
    h = t64(h0).reshape(b, H * P, N)
    ys = []
    for t in range(L):
        y, h = recurrent_step_cpu(x_ref[:, t].double(), dt_ref[:, t].double(), t64(Bm[:, t, 0]), t64(Cm[:, t, 0]),
                                  h, torch.zeros(N, dtype=f64), D_ref.double())
        ys.append(y)
    y = torch.stack(ys, 1).numpy().reshape(b, L, H, P)
    assert rel_l2(y, y_dir) < 1e-6
    assert rel_l2(h.numpy().reshape(b, H, P, N), h_dir) < 1e-6


def test_recurrent_step_cpu_one_token_closed_form(rng):
    """From a zero state: h = dt x B^T, y = (C . B) dt x + D x."""
    x, dt, B, C, _, A_log, D = step_case(rng)
    h0 = np.zeros((x.shape[0], x.shape[1], B.shape[1]))
    y, hn = recurrent_step_cpu(t64(x), t64(dt), t64(B), t64(C), t64(h0), t64(A_log), t64(D))
    h_cf = dt[:, :, None] * x[:, :, None] * B[:, None, :]
    y_cf = np.sum(C * B, -1)[:, None] * dt * x + D[None] * x
    assert rel_l2(hn.numpy(), h_cf) < 1e-13
    assert rel_l2(y.numpy(), y_cf) < 1e-13


def test_recurrent_step_cpu_does_not_clamp_A_log(rng):
    """The decode step takes exp(A_log) as is (mamba2.py:441-443): A_log = 6 decays by exp(-e^6 dt)."""
    x, dt, B, C, h, _, D = step_case(rng, N=3)
    dt = 0.02 * dt                      # small steps, so that e^6 and the clamped e^5 decay differently
    A_log = np.array([6.0, -6.0, 0.0])
    _, hn = recurrent_step_cpu(t64(x), t64(dt), t64(B), t64(C), t64(h), t64(A_log), t64(D))
    a = np.exp(A_log)
    h_cf = np.exp(-a[None, None, :] * dt[:, :, None]) * h + dt[:, :, None] * x[:, :, None] * B[:, None, :]
    assert rel_l2(hn.numpy(), h_cf) < 1e-13


def _step_planted_clamp(x_t, dt_t, B_t, C_t, h_prev, A_log, D):
    A_disc = torch.exp(-torch.exp(torch.clamp(A_log, -5.0, 5.0)).unsqueeze(0) * dt_t.unsqueeze(-1))
    h_t = A_disc * h_prev + (B_t.unsqueeze(1) * dt_t.unsqueeze(-1)) * x_t.unsqueeze(-1)
    return (C_t.unsqueeze(1) * h_t).sum(-1) + D * x_t, h_t


def _step_planted_broadcast(x_t, dt_t, B_t, C_t, h_prev, A_log, D):
    # dt broadcast along the state axis instead of the channel axis (both are (b, d_inner) vs (b, N) mixed up)
    A_disc = torch.exp(-torch.exp(A_log).unsqueeze(0) * dt_t.unsqueeze(-1))
    h_t = A_disc * h_prev + (B_t.unsqueeze(1) * dt_t[:, :B_t.shape[1]].unsqueeze(1)) * x_t.unsqueeze(-1)
    return (C_t.unsqueeze(1) * h_t).sum(-1) + D * x_t, h_t


def test_planted_clamp_in_decode_step_is_caught(rng):
    x, dt, B, C, h, _, D = step_case(rng, N=3)
    dt = 0.02 * dt
    A_log = np.array([6.0, -6.0, 0.0])
    _, hp = _step_planted_clamp(t64(x), t64(dt), t64(B), t64(C), t64(h), t64(A_log), t64(D))
    _, h_ref = ssd.ref_recurrent_step(x[:, None], dt[:, None], B[:, None], C[:, None], h, A_log, D)
    assert rel_l2(hp.numpy(), h_ref) > 1e-3


def test_planted_dt_broadcast_is_caught(rng):
    x, dt, B, C, h, A_log, D = step_case(rng)
    yp, hp = _step_planted_broadcast(t64(x), t64(dt), t64(B), t64(C), t64(h), t64(A_log), t64(D))
    y_ref, h_ref = ssd.ref_recurrent_step(x[:, None], dt[:, None], B[:, None], C[:, None], h, A_log, D)
    assert rel_l2(hp.numpy(), h_ref) > 1e-2 and rel_l2(yp.numpy(), y_ref[:, 0]) > 1e-2


# ----------------------------------------------------------------- linear_attention_scan_cpu

LAM_RAW = np.array([-1.0, 0.4, 2.5, 5.5])          # sigmoid(5.5) > 0.99: the clamped head


def kda_case(rng, B=2, H=4, S=150, D=32, scale=1.0):
    mk = lambda: rng.standard_normal((B, H, S, D)) * scale
    return mk(), mk(), mk(), mk()


def per_head(out, ref):
    return max(rel_l2(out[:, h], ref[:, h]) for h in range(ref.shape[1]))


@pytest.mark.parametrize("S,K,chunk", [(150, 32, 64), (150, 20, 64), (37, 32, 64), (64, 32, 16)])
def test_linear_attention_scan_cpu_float64_matches_attention_matrix(rng, S, K, chunk):
    """Float64 inputs keep float64 chunk tensors (the carry is fp32): every head, the clamped one included, to 1e-5."""
    q1, q2, k, v = kda_case(rng, S=S)
    out = linear_attention_scan_cpu(t64(q1), t64(q2), t64(k), t64(v), K, t64(LAM_RAW), chunk_size=chunk).numpy()
    ref = kda.ref_attention_scan(q1, q2, k, v, K, LAM_RAW)
    # the brute-force attention-matrix form, independently of ref_attention_scan's recurrence
    lam = kda.diff_lambda(LAM_RAW)[None, :, None, None]
    o1 = kda.ref_attention_matrix(q1, k, v, K)
    o2 = kda.ref_attention_matrix(q2, k, v, K)
    brute = (o1 - lam * o2) / (1.0 - lam + 1e-8)
    assert per_head(ref, brute) < 1e-10
    assert per_head(out, ref) < 1e-5


def test_linear_attention_scan_cpu_fp32_inputs_bf16_intermediates(rng):
    """fp32 inputs take the reference's bf16 intermediates (kda_diff.py:398).  With lambda ~ 0 the output is o1
    alone: every head to 1e-2.  With the differential output the bf16 rounding of o1 and o2 is scaled by
    c = 1 / (1 - lambda) (1.4 to 100 over LAM_RAW): each head within 6e-3 c of the exact value.  And bf16 makes a
    difference (the intermediates are not fp32)."""
    q1, q2, k, v = kda_case(rng, S=130, D=64, scale=0.5)
    t32 = lambda a: torch.tensor(a, dtype=torch.float32)
    off = np.full(4, -40.0)
    o1 = linear_attention_scan_cpu(t32(q1), t32(q2), t32(k), t32(v), 64, t32(off)).numpy()
    r1, _, _, _ = kda.ref_scan_pair(q1, q2, k, v, 64)
    assert per_head(o1, r1) < 1e-2
    out = linear_attention_scan_cpu(t32(q1), t32(q2), t32(k), t32(v), 64, t32(LAM_RAW)).numpy()
    ref = kda.ref_attention_scan(q1, q2, k, v, 64, LAM_RAW)
    c = 1.0 / (1.0 - kda.diff_lambda(LAM_RAW))
    for h in range(4):
        assert rel_l2(out[:, h], ref[:, h]) < 6e-3 * c[h], h
    exact = linear_attention_scan_cpu(t64(q1), t64(q2), t64(k), t64(v), 64, t64(LAM_RAW)).numpy()
    assert rel_l2(out[:, 0], exact[:, 0]) > 1e-4


def test_linear_attention_scan_cpu_chunk_invariant(rng):
    """Chunks of 1, 7, 64 and the whole sequence give the same output: the S / z carry between chunks is exact."""
    q1, q2, k, v = kda_case(rng, S=100)
    outs = [linear_attention_scan_cpu(t64(q1), t64(q2), t64(k), t64(v), 32, t64(LAM_RAW), chunk_size=c).numpy()
            for c in (1, 7, 64, 100)]
    for o in outs[1:]:
        assert per_head(o, outs[0]) < 1e-6


def _scan_planted(q1, q2, k, v, K, lambda_raw, chunk_size, mistake):
    """A copy of linear_attention_scan_cpu's recurrence with one planted mistake (float64 throughout)."""
    B, H, S, Dd = q1.shape
    phi = lambda x: F.elu(x[..., :K]) + (0.0 if mistake == "no_plus_one" else 1.0)
    q1p, q2p, kp = phi(q1), phi(q2), phi(k)
    Sst = torch.zeros(B, H, K, Dd, dtype=f64)
    z = torch.zeros(B, H, K, dtype=f64)
    o1s, o2s = [], []
    for s0 in range(0, S, chunk_size):
        s1 = min(S, s0 + chunk_size)
        kc, vc = kp[:, :, s0:s1], v[:, :, s0:s1]
        kv = kc.unsqueeze(-1) * vc.unsqueeze(-2)
        kv_cum = torch.cumsum(kv, 2) + Sst.unsqueeze(2)
        k_cum = torch.cumsum(kc, 2) + z.unsqueeze(2)
        if mistake == "exclusive":
            kv_cum = kv_cum - kv
            k_cum = k_cum - kc
        for qp, acc in ((q1p, o1s), (q2p, o2s)):
            qc = qp[:, :, s0:s1]
            num = torch.einsum("bhck,bhckd->bhcd", qc, kv_cum)
            den = torch.einsum("bhck,bhck->bhc", qc, k_cum)
            acc.append(num / (den.unsqueeze(-1) + 1e-8))
        if mistake != "no_carry":
            Sst = Sst + kv.sum(2)
            z = z + kc.sum(2)
    o1, o2 = torch.cat(o1s, 2), torch.cat(o2s, 2)
    lam = torch.clamp(torch.sigmoid(lambda_raw).view(1, H, 1, 1), max=0.99)
    return (o1 - lam * o2) / (1.0 - lam + 1e-8)


@pytest.mark.parametrize("mistake", ["no_carry", "exclusive", "no_plus_one"])
def test_planted_kda_scan_mistakes_are_caught(rng, mistake):
    q1, q2, k, v = kda_case(rng, S=150)
    ref = kda.ref_attention_scan(q1, q2, k, v, 32, LAM_RAW)
    good = _scan_planted(t64(q1), t64(q2), t64(k), t64(v), 32, t64(LAM_RAW), 64, None).numpy()
    bad = _scan_planted(t64(q1), t64(q2), t64(k), t64(v), 32, t64(LAM_RAW), 64, mistake).numpy()
    assert per_head(good, ref) < 1e-10
    assert per_head(bad, ref) > 1e-3
