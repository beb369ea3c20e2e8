"""Shared helpers of the GPU parity tests (not collected by pytest)."""

import sys

import numpy as np
import torch

TOL = {torch.bfloat16: 1e-2, torch.float32: 1e-4}


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def dev(a, dtype=torch.float32):
    if a is None:
        return None
    t = torch.as_tensor(np.asarray(a)) if not torch.is_tensor(a) else a
    return t.to(device="cuda", dtype=dtype)


def host(t):
    return t.detach().to(torch.float64).cpu().numpy()


def rel_l2(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref.ravel())
    return np.linalg.norm((out - ref).ravel()) / den if den > 0 else np.linalg.norm(out.ravel())


def check(name, out, ref, tol):
    out = host(out) if torch.is_tensor(out) else np.asarray(out)
    assert np.isfinite(out).all(), f"{name}: non-finite output"
    e = rel_l2(out, ref)
    m = np.abs(out - np.asarray(ref)).max() if out.size else 0.0
    say(f"{name}: rel_l2={e:.3e} max_abs={m:.3e} tol={tol:.0e}")
    assert e <= tol, f"{name}: rel_l2 {e:.3e} > {tol:.0e}"
    return e


def check_per_head(name, out, ref, tol, axis=1):
    """check() on every head separately (heads along `axis`): outputs whose scale differs by orders of magnitude
    between heads (the differential output's 1 / (1 - lambda)) cannot hide one head's error in another's norm."""
    out = host(out) if torch.is_tensor(out) else np.asarray(out)
    ref = np.asarray(ref)
    return max(check(f"{name}[head {i}]", np.take(out, i, axis=axis), np.take(ref, i, axis=axis), tol)
               for i in range(out.shape[axis]))


def lambda_term_scale(dout, o1, o2, lambda_raw):
    """Per head, c^2 sigma'(lambda_raw) sum |dout . (o1 - o2)| (c = 1 / (1 - lambda + 1e-8)): the summed magnitude
    of the terms whose (cancelling) sum is d lambda_raw.  Zero for a head past the 0.99 clamp."""
    lr = np.asarray(lambda_raw, np.float64)
    sg = 1.0 / (1.0 + np.exp(-lr))
    lam = np.minimum(sg, 0.99)
    c = 1.0 / (1.0 - lam + 1e-8)
    terms = np.abs(np.asarray(dout, np.float64) * (np.asarray(o1) - np.asarray(o2))).sum(axis=(0, 2, 3))
    return c ** 2 * sg * (1.0 - sg) * (sg <= 0.99) * terms


def check_lambda_bound(name, out, ref, scale, tol):
    """|out_h - ref_h| <= tol * scale_h for every head: the lambda gradient sums c^2 dout . (o1 - o2), which a
    random dout makes cancel to ~1/sqrt(terms) of its magnitude, so the bound is relative to the terms' summed
    magnitude (lambda_term_scale) rather than to the cancelled value."""
    out = host(out) if torch.is_tensor(out) else np.asarray(out)
    err = np.abs(out - np.asarray(ref))
    for h in range(out.shape[0]):
        r = err[h] / scale[h] if scale[h] > 0 else err[h]
        say(f"{name}[head {h}]: |err|={err[h]:.3e} value={ref[h]:.3e} term scale={scale[h]:.3e} ratio={r:.3e} "
            f"tol={tol:.0e}")
        assert r <= tol, f"{name}[head {h}]: |err| / term scale {r:.3e} > {tol:.0e}"
