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


# The C restatement of the float64 oracle (oracle/cheby_ema_c.c, built by
# oracle/build.py from build()), for full-size batch rows.  Pinned against
# the numpy oracle in tests/test_oracle_c.py.
_ORACLE_C = None


def oracle_c():
    global _ORACLE_C
    if _ORACLE_C is None:
        import ctypes
        import os
        from oracle import build as ob
        if not os.path.exists(ob.LIB):
            ob.build()   # gcc, about a second (build() normally made it already)
        lib = ctypes.CDLL(ob.LIB)
        P, L, D_, I = ctypes.c_void_p, ctypes.c_long, ctypes.c_double, ctypes.c_int
        common = [P, L, L, L, L, L, P, L, L, P, P, P, L, L, D_, D_, D_, P, I, I]
        lib.osm_oracle_forward_row.argtypes = common + [P, P]
        lib.osm_oracle_forward_row.restype = I
        lib.osm_oracle_ttt_row.argtypes = common + [I, D_, P, P, P]
        lib.osm_oracle_ttt_row.restype = I
        _ORACLE_C = lib
    return _ORACLE_C


def _c_row_args(inp, b, lam_shift, lam_min, lam_max, ema_init, clamp_out, nan_policy):
    """(argument list, keep-alive list, S, D) of one batch row for the C oracle."""
    x = np.ascontiguousarray(inp["x"][b].float().numpy())
    S, D = x.shape
    c = np.ascontiguousarray(inp["coeffs"][b].numpy().astype(np.float32))
    H, K, hd = c.shape
    damp = np.ascontiguousarray(np.asarray(inp["damping"], dtype=np.float32))
    lam = np.ascontiguousarray(np.asarray(inp["lam"], dtype=np.float32))
    g = inp.get("g")
    gp, g_ss, g_sh = None, 0, 0
    if g is not None:
        g = np.ascontiguousarray(np.broadcast_to(np.asarray(g, dtype=np.float32), (inp["x"].shape[0], S, H))[b])
        gp, g_ss, g_sh = g.ctypes.data, H, 1
    init = None if ema_init is None else np.ascontiguousarray(np.asarray(ema_init, np.float64).reshape(-1, D)[b])
    args = [x.ctypes.data, S, D, H, K, D, c.ctypes.data, K * hd, hd, damp.ctypes.data, lam.ctypes.data, gp, g_ss,
            g_sh, lam_shift, lam_min, lam_max, None if init is None else init.ctypes.data, 1 if clamp_out else 0,
            1 if nan_policy == "zero_u" else 0]
    return args, [x, c, damp, lam, g, init], S, D


def oracle_c_forward_row(inp, b, *, lam_shift=0.004, lam_min=0.9, lam_max=0.9999, ema_init=None, clamp_out=True,
                         nan_policy="zero_z"):
    """(out [S,D], ema_final [D]) of batch row b, float64, by the C oracle."""
    args, keep, S, D = _c_row_args(inp, b, lam_shift, lam_min, lam_max, ema_init, clamp_out, nan_policy)
    out = np.empty((S, D))
    fin = np.empty(D)
    assert oracle_c().osm_oracle_forward_row(*args, out.ctypes.data, fin.ctypes.data) == 0
    del keep
    return out, fin


def oracle_c_ttt_row(inp, b, *, n_total, target="x", lam_shift=0.004, lam_min=0.9, lam_max=0.9999, ema_init=None,
                     clamp_out=True, nan_policy="zero_z"):
    """(G [H,K,hd], out [S,D], ema_final [D]) of batch row b by the C oracle,
    with the mean of the loss over n_total = B (S-1) D elements (the whole
    batch's), so G is directly the row's part of the batch gradient."""
    args, keep, S, D = _c_row_args(inp, b, lam_shift, lam_min, lam_max, ema_init, clamp_out, nan_policy)
    H, K, hd = inp["coeffs"].shape[1:]
    G = np.empty((H, K, hd))
    out = np.empty((S, D))
    fin = np.empty(D)
    scale = 2.0 / n_total if n_total > 0 else 0.0
    rc = oracle_c().osm_oracle_ttt_row(*args, 1 if target == "softsign" else 0, scale, G.ctypes.data,
                                        out.ctypes.data, fin.ctypes.data)
    assert rc == 0, rc
    del keep
    return G, out, fin
