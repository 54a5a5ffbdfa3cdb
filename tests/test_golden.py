"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture (a change to the oracle that
moves its outputs fails here).  GPU: the HIP path through the C ABI matches
the fixtures to the spec tolerances."""
import glob
import os

import numpy as np
import pytest
import torch

from helpers import assert_close_fp32, assert_close_grad
from oracle import cheby_ema as O
from oracle import v10_full as V

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    assert {"fwd_static.npz", "fwd_dynamic.npz", "fwd_k5_specials.npz", "ttt_x.npz",
            "ttt_softsign_dynamic.npz", "bwd_static.npz", "v10_full.npz"} <= names


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_oracle_reproduces_fixture(path):
    f = load(path)
    if "coeffs_new" in f:
        out, c, m = V.v10_full(f["x"], f["coeffs"].astype(np.float64), f["momentum"].astype(np.float64),
                               n_heads=int(f["n_heads"]), chunk_size=256)
        for got, k in ((out, "out"), (c, "coeffs_new"), (m, "momentum_new")):
            np.testing.assert_allclose(got, f[k], rtol=1e-12, atol=1e-15)
        return
    kw = dict(g=f.get("g"), ema_init=f.get("ema_init"))
    x = f["x"].astype(np.float64)
    if "grad_x" in f:
        got = O.backward(x, f["coeffs"], f["damping"], f["lam"], f["grad_out"].astype(np.float64),
                         ema_init=f["ema_init"], grad_state=f["grad_state"].astype(np.float64))
        for g_, k in zip(got, ("grad_x", "grad_coeffs", "grad_init")):
            np.testing.assert_allclose(g_, f[k], rtol=1e-12, atol=1e-15)
    if "grad" in f:
        G, out, fin = O.ttt_grad(x, f["coeffs"], f["damping"], f["lam"], target=str(f["target"]), **kw)
        np.testing.assert_allclose(G, f["grad"], rtol=1e-12, atol=1e-15)
    else:
        out, fin = O.forward(x, f["coeffs"], f["damping"], f["lam"], **kw)
    np.testing.assert_allclose(out, f["out"], rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(fin, f["ema_final"], rtol=1e-12, atol=1e-15)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_hip_path_matches_fixture(dev, path):
    from orthossm_amd import cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt
    from orthossm_amd.ops import v10_chunked_ttt

    f = load(path)
    if "coeffs_new" in f:
        x, c, m = (torch.from_numpy(f[k]).to(dev) for k in ("x", "coeffs", "momentum"))
        out, cn, mn = v10_chunked_ttt(x, c, m, n_heads=int(f["n_heads"]), chunk_size=256)
        torch.cuda.synchronize()
        # out holds bf16 values: equal but for rare one-ulp rounding flips
        d = np.abs(out.cpu().numpy() - f["out"])
        assert d.max() <= 2e-2 and (d > 1e-6).mean() <= 1e-3
        for got, k in ((cn, "coeffs_new"), (mn, "momentum_new")):
            e = np.abs(got.cpu().numpy() - f[k])
            assert (e > 1e-5 * (1 + np.abs(f[k]))).mean() <= 1e-3, k
        return
    t = {k: torch.from_numpy(v).to(dev) for k, v in f.items()
         if k in ("x", "coeffs", "damping", "lam", "g", "ema_init")}
    if "grad" in f:
        out, grad, fin = cheby_ema_ttt(t["x"], t["coeffs"], t["damping"], t["lam"], g=t.get("g"),
                                       ema_init=t.get("ema_init"), target=str(f["target"]), return_state=True)
        torch.cuda.synchronize()
        assert O.rel_err(grad.cpu().numpy(), f["grad"]) <= 1e-3
    else:
        out, fin = cheby_ema_forward(t["x"], t["coeffs"], t["damping"], t["lam"], g=t.get("g"),
                                     ema_init=t.get("ema_init"), return_state=True)
        torch.cuda.synchronize()
    if "grad_x" in f:
        go, gs = (torch.from_numpy(f[k]).to(dev) for k in ("grad_out", "grad_state"))
        gx, gc, gi = cheby_ema_backward(t["x"], t["coeffs"], t["damping"], t["lam"], out, go, grad_state=gs,
                                        need_init=True)
        torch.cuda.synchronize()
        for got, k in ((gx, "grad_x"), (gc, "grad_coeffs"), (gi, "grad_init")):
            assert_close_grad(got.cpu(), f[k], what=k)
    assert_close_fp32(out.cpu(), f["out"])
    assert_close_fp32(fin.cpu(), f["ema_final"], what="ema_final")
