"""Shared helpers for the GPU parity tests (inputs, oracle calls, tolerances)."""
import numpy as np
import torch

from oracle import cheby_ema as O
from orthossm_amd.synthetic import make_inputs

# fp32 tolerance of the spec: 1e-5 relative.  Checked two ways: normalised by
# the largest reference magnitude, and elementwise with an absolute floor.
RTOL = 1e-5
ATOL = 1e-6


def assert_close_fp32(got, want, rtol=RTOL, atol=ATOL, what="out"):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    both_nan = np.isnan(got) & np.isnan(want)
    g, w = np.where(both_nan, 0.0, got), np.where(both_nan, 0.0, want)
    assert not np.isnan(g).any(), f"{what}: NaN where the oracle has a number"
    err = np.abs(g - w)
    bad = err > rtol * np.abs(w) + atol
    if bad.any():
        i = np.unravel_index(np.argmax(err - rtol * np.abs(w)), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} elements off; worst at {i}: "
                             f"got {g[i]!r} want {w[i]!r}; max rel {O.rel_err(g, w):.3e}")
    assert O.rel_err(g, w) <= rtol, f"{what}: max-normalised error {O.rel_err(g, w):.3e}"


def inputs(B, S, H, hd, K=8, seed=0, dynamic=False, dtype=torch.float32):
    return make_inputs(B, S, H * hd, H, K, seed=seed, dynamic=dynamic, dtype=dtype)


def to_dev(inp, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}


def oracle_forward(inp, **kw):
    g = inp.get("g")
    return O.forward(inp["x"].double().numpy(), inp["coeffs"].numpy(), inp["damping"].numpy(),
                     inp["lam"].numpy(), g=None if g is None else g.numpy(), **kw)


def oracle_ttt(inp, **kw):
    g = inp.get("g")
    return O.ttt_grad(inp["x"].double().numpy(), inp["coeffs"].numpy(), inp["damping"].numpy(),
                      inp["lam"].numpy(), g=None if g is None else g.numpy(), **kw)


def oracle_backward(inp, grad_out, **kw):
    g = inp.get("g")
    return O.backward(inp["x"].double().numpy(), inp["coeffs"].numpy(), inp["damping"].numpy(),
                      inp["lam"].numpy(), np.asarray(grad_out, dtype=np.float64),
                      g=None if g is None else g.numpy(), **kw)


# Gradient tolerance of the spec: 1e-3 relative.  Checked normalised by the
# largest reference magnitude and elementwise with a floor of 1e-4 of it.
GRAD_RTOL = 1e-3


def assert_close_grad(got, want, rtol=GRAD_RTOL, what="grad"):
    want = np.asarray(want, dtype=np.float64)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    assert_close_fp32(got, want, rtol=rtol, atol=1e-4 * scale + 1e-30, what=what)


def compare_v10(out, cn, mn, want):
    """The full path (out, coeffs, momentum) against oracle/v10_full.py's
    (out, coeffs, momentum).  out holds bf16 values: equal except where fp32
    and float64 rounding of s land on two sides of a bf16 rounding boundary
    (one bf16 ulp).  A Lion sign that rounding decides (|interp| ~ 1e-7)
    moves one coefficient by 2 lr ss_k, so a tiny fraction of coefficient
    and momentum elements may differ."""
    wo, wc, wm = want
    o = out.cpu().numpy().astype(np.float64)
    diff = np.abs(o - wo)
    assert np.nanmax(np.where(np.isnan(wo), 0, diff)) <= 2e-2, "out beyond 2e-2"
    assert (diff > 1e-6).mean() <= 1e-3, f"{(diff > 1e-6).mean():.4f} of out differ"
    for got, w, what in ((cn, wc, "coeffs"), (mn, wm, "momentum")):
        g = got.cpu().numpy().astype(np.float64)
        both = np.isnan(g) & np.isnan(w)
        d = np.abs(np.where(both, 0, g) - np.where(both, 0, w))
        assert not np.isnan(d).any(), f"{what}: NaN mismatch"
        assert (d > 1e-5 * (1 + np.abs(w))).mean() <= 1e-3, f"{what}: {(d > 1e-5).sum()} elements off"
