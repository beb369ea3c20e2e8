"""Pins of the CPU oracle (oracle/ssd.py, oracle/kda.py) -- CPU only.

No check below restates the formula it tests: each compares two independent
constructions (reference recurrence through the bridge vs. direct SSD form vs.
explicit semiseparable matrix vs. chunked form), a closed form, or an
invariant, chosen so that a dropped term, a wrong sign/index or a transposed
operand fails (the ``test_planted_*`` tests plant such mistakes in copies of
the oracle and check that the pins catch them).
"""

import numpy as np
import pytest

from oracle import kda, ssd
from tests.conftest import rel_l2


def ssd_case(rng, b=2, L=23, H=4, P=3, N=5, G=2, h0=False, D_per_channel=False):
    x = rng.standard_normal((b, L, H, P))
    dt = ssd.softplus(rng.standard_normal((b, L, H)) - 1.0)
    A = -np.exp(rng.uniform(0, np.log(8), H))
    B = rng.standard_normal((b, L, G, N))
    C = rng.standard_normal((b, L, G, N))
    D = rng.standard_normal((H, P)) if D_per_channel else rng.standard_normal(H)
    s0 = 0.3 * rng.standard_normal((b, H, P, N)) if h0 else None
    return x, dt, A, B, C, D, s0


# ----------------------------------------------------------------- SSD

@pytest.mark.parametrize("G,dpc", [(1, False), (2, True), (4, False)])
def test_bridge_matches_direct_ssd(rng, G, dpc):
    x, dt, A, B, C, D, _ = ssd_case(rng, G=G, D_per_channel=dpc)
    y_ref, h_ref = ssd.ssd_via_reference(x, dt, A, B, C, D)
    y_dir, h_dir = ssd.ssd_direct(x, dt, A, B, C, D)
    assert rel_l2(y_ref, y_dir) < 1e-12
    assert rel_l2(h_ref, h_dir) < 1e-12


def test_bridge_with_initial_state_uses_reference_decode(rng):
    x, dt, A, B, C, D, s0 = ssd_case(rng, h0=True)
    y_ref, h_ref = ssd.ssd_via_reference(x, dt, A, B, C, D, initial_state=s0)
    y_dir, h_dir = ssd.ssd_direct(x, dt, A, B, C, D, initial_state=s0)
    assert rel_l2(y_ref, y_dir) < 1e-12
    assert rel_l2(h_ref, h_dir) < 1e-12


def test_direct_matches_semiseparable_matrix(rng):
    x, dt, A, B, C, D, _ = ssd_case(rng, b=1, L=11, H=2, P=2, N=3, G=1)
    y_dir, _ = ssd.ssd_direct(x, dt, A, B, C, D)
    y_mat = ssd.ssd_semiseparable(x, dt, A, B, C, D)
    assert rel_l2(y_dir, y_mat) < 1e-12


@pytest.mark.parametrize("Q", [1, 3, 8, 64])
def test_chunked_matches_direct_any_chunk(rng, Q):
    x, dt, A, B, C, D, s0 = ssd_case(rng, L=37, h0=True)
    y_dir, h_dir = ssd.ssd_direct(x, dt, A, B, C, D, initial_state=s0)
    y_chk, h_chk = ssd.ssd_chunked(x, dt, A, B, C, D, initial_state=s0, chunk_size=Q)
    assert rel_l2(y_chk, y_dir) < 1e-12
    assert rel_l2(h_chk, h_dir) < 1e-12


def test_single_token_closed_form(rng):
    x, dt, A, B, C, D, _ = ssd_case(rng, L=1, G=1)
    y, h = ssd.ssd_via_reference(x, dt, A, B, C, D)
    cb = np.einsum("bn,bn->b", C[:, 0, 0], B[:, 0, 0])
    expect_y = cb[:, None, None] * dt[:, 0, :, None] * x[:, 0] + D[None, :, None] * x[:, 0]
    assert rel_l2(y[:, 0], expect_y) < 1e-12
    expect_h = dt[:, 0, :, None, None] * x[:, 0, :, :, None] * B[:, 0, 0][:, None, None, :]
    assert rel_l2(h, expect_h) < 1e-12


def test_reference_constant_decay_closed_form(rng):
    """The reference test's dt=1, A_log=0 case (tests/test_mamba2.py:73-84): decay e^-1 per step."""
    b, L, d, N = 2, 33, 32, 8
    x = rng.standard_normal((b, L, d))
    B = rng.standard_normal((b, L, N))
    C = rng.standard_normal((b, L, N))
    y = ssd.ref_selective_scan(x, np.ones((b, L, d)), np.zeros(N), B, C, np.ones(d))
    cb = np.einsum("btn,bsn->bts", C, B)
    t = np.arange(L)
    dec = np.where(t[:, None] >= t[None, :], np.exp(-(t[:, None] - t[None, :]).astype(float)), 0.0)
    expect = np.einsum("bts,bsd->btd", cb * dec[None], x) + x
    assert rel_l2(y, expect) < 1e-12


def test_no_decay_is_cumulative_sum(rng):
    x, dt, _, B, C, D, _ = ssd_case(rng, G=1)
    A = np.zeros(x.shape[2])
    y, _ = ssd.ssd_direct(x, dt, A, B, C, D)
    cb = np.einsum("btn,bsn->bts", C[:, :, 0], B[:, :, 0])
    L = x.shape[1]
    mask = np.tril(np.ones((L, L)))
    expect = np.einsum("bts,bsh,bshp->bthp", cb * mask, dt, x) + D[None, None, :, None] * x
    assert rel_l2(y, expect) < 1e-12


def test_zero_B_gives_skip_only(rng):
    x, dt, A, B, C, D, _ = ssd_case(rng)
    y, h = ssd.ssd_via_reference(x, dt, A, np.zeros_like(B), C, D)
    assert rel_l2(y, D[None, None, :, None] * x) < 1e-14
    assert np.abs(h).max() == 0


def test_linearity_in_x_and_h0(rng):
    x, dt, A, B, C, _, s0 = ssd_case(rng, h0=True)
    x2 = rng.standard_normal(x.shape)
    s1 = rng.standard_normal(s0.shape)
    ya, ha = ssd.ssd_direct(x, dt, A, B, C, None, initial_state=s0)
    yb, hb = ssd.ssd_direct(x2, dt, A, B, C, None, initial_state=s1)
    yc, hc = ssd.ssd_direct(2 * x - 3 * x2, dt, A, B, C, None, initial_state=2 * s0 - 3 * s1)
    assert rel_l2(yc, 2 * ya - 3 * yb) < 1e-12
    assert rel_l2(hc, 2 * ha - 3 * hb) < 1e-12


def test_prefill_then_decode_equals_longer_prefill(rng):
    """State carry: prefill L-m tokens, then m reference decode steps == prefill of L tokens."""
    x, dt, A, B, C, D, s0 = ssd_case(rng, L=20, h0=True)
    y_full, h_full = ssd.ssd_via_reference(x, dt, A, B, C, D, initial_state=s0)
    m = 5
    y_pre, h = ssd.ssd_via_reference(x[:, :-m], dt[:, :-m], A, B[:, :-m], C[:, :-m], D, initial_state=s0)
    ys = [y_pre]
    for t in range(x.shape[1] - m, x.shape[1]):
        # the decode path takes raw dt and applies softplus; feed an exact inverse of softplus
        raw = np.log(np.expm1(dt[:, t]))
        yt, h = ssd.state_update_via_reference(h, x[:, t], raw, A, B[:, t], C[:, t], D, dt_softplus=True)
        ys.append(yt[:, None])
    assert rel_l2(np.concatenate(ys, 1), y_full) < 1e-10
    assert rel_l2(h, h_full) < 1e-10


def test_state_update_bridge_matches_direct(rng):
    b, H, P, N, G = 3, 4, 5, 6, 2
    s0 = rng.standard_normal((b, H, P, N))
    x = rng.standard_normal((b, H, P))
    dt = rng.standard_normal((b, H))
    A = -np.exp(rng.uniform(0, 2, H))
    B = rng.standard_normal((b, G, N))
    C = rng.standard_normal((b, G, N))
    D = rng.standard_normal(H)
    bias = rng.standard_normal(H)
    ya, sa = ssd.state_update_via_reference(s0, x, dt, A, B, C, D, dt_bias=bias, dt_limit=(0.05, 0.8))
    yb, sb = ssd.state_update_direct(s0, x, dt, A, B, C, D, dt_bias=bias, dt_limit=(0.05, 0.8))
    assert rel_l2(ya, yb) < 1e-12 and rel_l2(sa, sb) < 1e-12
    # one step from a zero state equals the reference scan of length 1 (mamba2.py:101 vs :448-449)
    y1, _ = ssd.state_update_via_reference(np.zeros_like(s0), x, dt, A, B, C, D, dt_softplus=True)
    d = ssd.softplus(dt)
    y2, _ = ssd.ssd_via_reference(x[:, None], d[:, None], A, B[:, None], C[:, None], D)
    assert rel_l2(y1, y2[:, 0]) < 1e-12


def test_softplus_matches_torch_definition():
    import torch
    v = np.linspace(-30, 30, 601)
    assert np.allclose(ssd.softplus(v), torch.nn.functional.softplus(torch.tensor(v)).numpy(), rtol=1e-12, atol=0)


# ----------------------------------------------------------------- planted mistakes (mutation checks)

def test_planted_transposed_BC_is_caught(rng):
    x, dt, A, B, C, D, _ = ssd_case(rng, b=1, L=9, H=2, P=2, N=3, G=1)
    y_bad, _ = ssd.ssd_direct(x, dt, A, C, B, D)          # B and C swapped
    y_mat = ssd.ssd_semiseparable(x, dt, A, B, C, D)
    assert rel_l2(y_bad, y_mat) > 1e-3


def test_planted_sign_error_is_caught(rng):
    x, dt, A, B, C, D, _ = ssd_case(rng, b=1, L=9, H=2, P=2, N=3, G=1)
    y_bad, _ = ssd.ssd_direct(x, dt, -A, B, C, D)         # growth instead of decay
    y_mat = ssd.ssd_semiseparable(x, dt, A, B, C, D)
    assert rel_l2(y_bad, y_mat) > 1e-3


def test_planted_off_by_one_decay_is_caught(rng):
    """Exclusive instead of inclusive decay (decay applied after the input) changes y."""
    x, dt, A, B, C, D, _ = ssd_case(rng, b=1, L=9, H=2, P=2, N=3, G=1)
    b, L, H, P = x.shape
    h = np.zeros((b, H, P, B.shape[-1]))
    y = np.zeros_like(x)
    for t in range(L):
        h = h + dt[:, t, :, None, None] * x[:, t, :, :, None] * B[:, t, 0][:, None, None, :]
        y[:, t] = np.einsum("bhpn,bn->bhp", h, C[:, t, 0]) + D[None, :, None] * x[:, t]
        h = np.exp(A[None, :] * dt[:, t])[:, :, None, None] * h
    assert rel_l2(y, ssd.ssd_semiseparable(x, dt, A, B, C, D)) > 1e-3


def test_planted_dropped_skip_is_caught(rng):
    x, dt, A, B, C, D, _ = ssd_case(rng)
    y_ref, _ = ssd.ssd_via_reference(x, dt, A, B, C, D)
    y_bad, _ = ssd.ssd_direct(x, dt, A, B, C, None)
    assert rel_l2(y_bad, y_ref) > 1e-3


# ----------------------------------------------------------------- KDA gated

def kda_case(rng, Bb=2, H=3, S=19, K=6, V=5, gate=True, s0=False):
    q1 = rng.standard_normal((Bb, H, S, K)) * 0.5
    q2 = rng.standard_normal((Bb, H, S, K)) * 0.5
    k = rng.standard_normal((Bb, H, S, K)) * 0.5
    v = rng.standard_normal((Bb, H, S, V))
    g = np.log(1.0 / (1.0 + np.exp(-rng.standard_normal((Bb, H, S, K))))) / 2.0 if gate else None
    S0 = rng.standard_normal((Bb, H, K, V)) if s0 else None
    return q1, q2, k, v, g, S0


def test_gated_recurrent_matches_closed_form(rng):
    q1, q2, k, v, g, S0 = kda_case(rng, s0=True)
    o_r, s_r = kda.gated_recurrent(q1, q2, k, v, g, 0.8, S0)
    o_c, s_c = kda.gated_closed_form(q1, q2, k, v, g, 0.8, S0)
    assert rel_l2(o_r, o_c) < 1e-12 and rel_l2(s_r, s_c) < 1e-12


@pytest.mark.parametrize("Q", [1, 4, 16, 64])
def test_gated_chunked_matches_recurrent(rng, Q):
    q1, q2, k, v, g, S0 = kda_case(rng, S=37, s0=True)
    o_r, s_r = kda.gated_recurrent(q1, q2, k, v, g, 0.8, S0)
    o_c, s_c = kda.gated_chunked(q1, q2, k, v, g, 0.8, S0, chunk_size=Q)
    assert rel_l2(o_c, o_r) < 1e-12 and rel_l2(s_c, s_r) < 1e-12


def test_gated_without_decay_is_causal_linear_attention(rng):
    q1, q2, k, v, _, _ = kda_case(rng, gate=False)
    o, _ = kda.gated_recurrent(q1, q2, k, v, None, 0.8)
    qe = q1 - 0.8 * q2
    S = k.shape[2]
    a = np.einsum("bhtk,bhsk->bhts", qe, k) * np.tril(np.ones((S, S)))
    assert rel_l2(o, np.einsum("bhts,bhsv->bhtv", a, v)) < 1e-12


def test_gated_lambda_zero_is_single_query(rng):
    q1, q2, k, v, g, _ = kda_case(rng)
    o0, _ = kda.gated_recurrent(q1, q2, k, v, g, 0.0)
    o1, _ = kda.gated_recurrent(q1, np.zeros_like(q2), k, v, g, 0.5)
    assert rel_l2(o0, o1) < 1e-14


def test_planted_exclusive_gate_is_caught(rng):
    """Reading the state before adding k_t v_t (exclusive) differs from the inclusive operator."""
    q1, q2, k, v, g, _ = kda_case(rng)
    o_ref, _ = kda.gated_closed_form(q1, q2, k, v, g, 0.8)
    Bb, H, S, K = k.shape
    st = np.zeros((Bb, H, K, v.shape[-1]))
    o = np.zeros_like(o_ref)
    for t in range(S):
        o[:, :, t] = np.einsum("bhk,bhkv->bhv", q1[:, :, t] - 0.8 * q2[:, :, t], st)
        st = np.exp(g[:, :, t, :, None]) * st + k[:, :, t, :, None] * v[:, :, t, None, :]
    assert rel_l2(o, o_ref) > 1e-3


# ----------------------------------------------------------------- KDA reference mode

def test_reference_pair_matches_attention_matrix(rng):
    q1, q2, k, v, _, _ = kda_case(rng, K=6, V=5, gate=False)
    o1, o2, _, _ = kda.ref_scan_pair(q1, q2, k, v, kernel_dim=4)
    assert rel_l2(o1, kda.ref_attention_matrix(q1, k, v, 4)) < 1e-12
    assert rel_l2(o2, kda.ref_attention_matrix(q2, k, v, 4)) < 1e-12


def test_reference_constant_values_pass_through(rng):
    q1, q2, k, _, _, _ = kda_case(rng, gate=False)
    c = rng.standard_normal(5)
    v = np.broadcast_to(c, q1.shape[:3] + (5,))
    o1, _, _, _ = kda.ref_scan_pair(q1, q2, k, v, kernel_dim=6)
    assert np.allclose(o1, c, rtol=1e-6, atol=0)


def test_reference_recurrent_step_continues_scan(rng):
    q1, q2, k, v, _, _ = kda_case(rng, S=9, gate=False)
    lam_raw = rng.standard_normal(q1.shape[1])
    K = 4
    o1, o2, S8, z8 = kda.ref_scan_pair(q1[:, :, :8], q2[:, :, :8], k[:, :, :8], v[:, :, :8], K)
    out, Sn, zn = kda.ref_attention_recurrent(kda.feature_map(q1[:, :, 8:], K), kda.feature_map(q2[:, :, 8:], K),
                                              kda.feature_map(k[:, :, 8:], K), v[:, :, 8:], S8, z8[..., None],
                                              lam_raw)
    full = kda.ref_attention_scan(q1, q2, k, v, K, lam_raw)
    assert rel_l2(out[:, :, 0], full[:, :, 8]) < 1e-12
    _, _, S9, z9 = kda.ref_scan_pair(q1, q2, k, v, K)
    assert rel_l2(Sn, S9) < 1e-12 and rel_l2(zn[..., 0], z9) < 1e-12


def test_feature_map_is_elu_plus_one():
    import torch
    x = np.linspace(-5, 5, 101)
    expect = torch.nn.functional.elu(torch.tensor(x)).numpy() + 1.0
    assert np.allclose(kda.feature_map(x, 101), expect, rtol=1e-12, atol=1e-15)


def test_diff_lambda_clamp():
    lam = kda.diff_lambda(np.array([-10.0, 0.0, 10.0]))
    assert np.allclose(lam, [1 / (1 + np.exp(10)), 0.5, 0.99])


# ----------------------------------------------------------------- conv1d and h_states

@pytest.mark.parametrize("K", [1, 2, 4])
def test_causal_conv1d_matches_numpy_convolve(rng, K):
    """Causal depthwise conv == per-channel np.convolve with the flipped kernel (cross-correlation), truncated."""
    x = rng.standard_normal((2, 11, 6))
    w = rng.standard_normal((6, 1, K))
    bias = rng.standard_normal(6)
    out = ssd.ref_causal_conv1d(x, w, bias)
    exp = np.stack([np.stack([np.convolve(x[b, :, d], w[d, 0, ::-1])[:11] + bias[d] for d in range(6)], -1)
                    for b in range(2)])
    assert np.abs(out - exp).max() < 1e-12


def test_causal_conv1d_cache_equals_longer_sequence(rng):
    """With the cached raw rows prepended, the outputs equal the tail of the conv over the whole sequence;
    a cache shorter than K-1 rows behaves as a zero-padded one (mamba2.py:355, :388-402)."""
    x = rng.standard_normal((2, 9, 4))
    w = rng.standard_normal((4, 1, 4))
    full = ssd.ref_causal_conv1d(x, w)
    tail = ssd.ref_causal_conv1d(x[:, 6:], w, conv_state=x[:, 3:6])
    assert np.abs(tail - full[:, 6:]).max() < 1e-12
    short = ssd.ref_causal_conv1d(x[:, 2:], w, conv_state=x[:, :2])
    assert np.abs(short - full[:, 2:]).max() < 1e-12


def test_planted_unflipped_conv_kernel_is_caught(rng):
    x = rng.standard_normal((1, 8, 3))
    w = rng.standard_normal((3, 1, 3))
    good = ssd.ref_causal_conv1d(x, w)
    bad = ssd.ref_causal_conv1d(x, w[:, :, ::-1])
    assert rel_l2(bad, good) > 1e-2


@pytest.mark.parametrize("G", [1, 2])
def test_h_states_bridge_matches_direct(rng, G):
    """h_states through the reference recurrence (bridge, mean over each group's channels, combined) equals
    the direct per-token mean of the SSD state; the last row is the mean of the final state."""
    x, dt, A, B, C, D, _ = ssd_case(rng, G=G)
    y, fin, hs = ssd.ssd_via_reference(x, dt, A, B, C, D, return_h_states=True)
    hs2 = ssd.ssd_h_states(x, dt, A, B)
    assert rel_l2(hs, hs2) < 1e-12
    assert np.abs(hs[:, -1] - fin.mean(axis=(1, 2))).max() < 1e-12
