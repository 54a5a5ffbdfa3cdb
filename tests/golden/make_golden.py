"""Writes the golden fixtures of this directory from the float64 oracle.

    python tests/golden/make_golden.py

The reference ships no vectors for this path, so these fixtures freeze the
oracle's outputs (itself pinned by tests/test_oracle.py and
tests/test_oracle_v10.py) on small seeded inputs: forward, TTT gradient,
backward and the full path.  tests/test_golden.py checks the oracle still reproduces them (CPU)
and that the HIP path matches them (GPU).  Inputs are stored in float32 (what
the kernels read), outputs in float64.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import cheby_ema as O  # noqa: E402
from oracle import v10_full as V  # noqa: E402
from orthossm_amd.synthetic import make_inputs  # noqa: E402

CASES = {
    # name: (B, S, H, hd, K, dynamic, seed, extras)
    "fwd_static": (2, 160, 2, 32, 8, False, 1, {"init": True}),
    "fwd_dynamic": (1, 200, 2, 32, 8, True, 2, {}),
    "fwd_k5_specials": (1, 100, 2, 32, 5, False, 3, {"specials": True}),
    "ttt_x": (1, 150, 2, 32, 8, False, 4, {"ttt": "x", "init": True}),
    "ttt_softsign_dynamic": (1, 120, 2, 32, 8, True, 5, {"ttt": "softsign"}),
    "bwd_static": (2, 140, 2, 32, 8, False, 6, {"bwd": True, "init": True}),
    "v10_full": (2, 600, 2, 16, 8, False, 7, {"v10": True}),
}


def build(name):
    B, S, H, hd, K, dyn, seed, ex = CASES[name]
    inp = make_inputs(B, S, H * hd, H, K, seed=seed, dynamic=dyn)
    x = inp["x"].numpy().astype(np.float32)
    if ex.get("specials"):
        x[0, 5, :4] = [np.nan, np.inf, -np.inf, 0.0]
        x[0, 6, :3] = [3e38, -3e38, 1e-42]
    arrays = {"x": x, "coeffs": inp["coeffs"].numpy(), "damping": inp["damping"].numpy(),
              "lam": inp["lam"].numpy()}
    if dyn:
        arrays["g"] = inp["g"].numpy()
    if ex.get("init"):
        arrays["ema_init"] = (np.random.default_rng(seed).random((B, H * hd)) - 0.5).astype(np.float32)
    kw = dict(g=arrays.get("g"), ema_init=arrays.get("ema_init"))
    x64 = arrays["x"].astype(np.float64)
    if ex.get("v10"):
        # the full path: 3 chunks of 256 (the last partial), LUT series, Lion
        rng = np.random.default_rng(seed)
        arrays["momentum"] = (rng.standard_normal(arrays["coeffs"].shape) * 0.01).astype(np.float32)
        out, c_new, m_new = V.v10_full(arrays["x"], arrays["coeffs"].astype(np.float64),
                                       arrays["momentum"].astype(np.float64), n_heads=H, chunk_size=256)
        arrays.update(out=out, coeffs_new=c_new, momentum_new=m_new, n_heads=np.array(H))
        del arrays["damping"], arrays["lam"]
        return arrays
    if ex.get("bwd"):
        rng = np.random.default_rng(seed)
        arrays["grad_out"] = rng.standard_normal(x.shape).astype(np.float32)
        arrays["grad_state"] = rng.standard_normal((B, H * hd)).astype(np.float32)
        out, fin = O.forward(x64, arrays["coeffs"], arrays["damping"], arrays["lam"], **kw)
        gx, gc, gi = O.backward(x64, arrays["coeffs"], arrays["damping"], arrays["lam"],
                                arrays["grad_out"].astype(np.float64), ema_init=arrays["ema_init"],
                                grad_state=arrays["grad_state"].astype(np.float64))
        arrays.update(out=out, ema_final=fin, grad_x=gx, grad_coeffs=gc, grad_init=gi)
        return arrays
    if "ttt" in ex:
        G, out, fin = O.ttt_grad(x64, arrays["coeffs"], arrays["damping"], arrays["lam"], target=ex["ttt"], **kw)
        arrays["grad"] = G
        arrays["target"] = np.array(ex["ttt"])
    else:
        out, fin = O.forward(x64, arrays["coeffs"], arrays["damping"], arrays["lam"], **kw)
    arrays["out"] = out
    arrays["ema_final"] = fin
    return arrays


if __name__ == "__main__":
    for name in CASES:
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **build(name))
        print("wrote", path, os.path.getsize(path), "bytes")
