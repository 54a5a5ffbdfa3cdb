"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture (a change to the oracle that
moves its outputs fails here).  GPU: the HIP path through the C ABI matches
the fixtures to the spec tolerances."""
import glob
import os

import numpy as np
import pytest
import torch

from helpers import assert_close_fp32
from oracle import cheby_ema as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    assert {"fwd_static.npz", "fwd_dynamic.npz", "fwd_k5_specials.npz", "ttt_x.npz",
            "ttt_softsign_dynamic.npz"} <= names


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_oracle_reproduces_fixture(path):
    f = load(path)
    kw = dict(g=f.get("g"), ema_init=f.get("ema_init"))
    x = f["x"].astype(np.float64)
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
    from orthossm_amd import cheby_ema_forward, cheby_ema_ttt

    f = load(path)
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
    assert_close_fp32(out.cpu(), f["out"])
    assert_close_fp32(fin.cpu(), f["ema_final"], what="ema_final")
