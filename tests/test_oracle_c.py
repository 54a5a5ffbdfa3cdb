"""The C restatement of the float64 oracle (oracle/cheby_ema_c.c), used for
full-size batch rows, against the numpy oracle it restates (itself pinned by
chebval, lfilter, closed forms, autograd and finite differences in
tests/test_oracle.py), row by row: forward output and final state, TTT
gradient, on random small cases crossing static and dynamic lambda, both
NaN policies, the clamp on and off, an initial state, 1 to 16 coefficients,
both TTT targets, and NaN / +-Inf / huge / subnormal values in x."""
import numpy as np
import pytest
import torch

from helpers import oracle_c_forward_row, oracle_c_ttt_row
from oracle import cheby_ema as O
from orthossm_amd.synthetic import make_inputs


def _case(seed):
    r = np.random.default_rng(seed)
    H = int(r.choice([1, 2, 3, 8]))
    hd = int(r.choice([1, 5, 16, 24]))
    B = int(r.integers(1, 3))
    S = int(r.choice([1, 2, 7, 300, 1001]))
    K = int(r.integers(1, 17))
    dyn = bool(r.integers(0, 2))
    inp = make_inputs(B, S, H * hd, H, K, seed=seed, dynamic=dyn)
    inp["coeffs"] = inp["coeffs"] * float(r.choice([1.0, 5.0]))
    inp["lam"] = torch.tensor(r.uniform(0.5, 0.9995, H), dtype=torch.float32)
    inp["damping"] = torch.tensor(r.uniform(0.3, 1.2, H), dtype=torch.float32)
    x = inp["x"].clone()
    if S > 5:
        flat = x.view(-1)
        idx = r.choice(flat.numel(), size=min(12, flat.numel()), replace=False)
        vals = [float("nan"), float("inf"), -float("inf"), 3e38, -3e38, 1e-40, 0.0, -0.0]
        for i, j in enumerate(idx):
            flat[j] = vals[i % len(vals)]
    inp["x"] = x
    kw = dict(
        ema_init=r.uniform(-1, 1, (B, H * hd)) if r.integers(0, 2) else None,
        clamp_out=bool(r.integers(0, 2)),
        nan_policy=str(r.choice(["zero_z", "zero_u"])),
    )
    return inp, kw


def _close(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN pattern differs"
    g, w = np.nan_to_num(got), np.nan_to_num(want)
    np.testing.assert_allclose(g, w, rtol=1e-12, atol=1e-14 * max(1.0, float(np.max(np.abs(w)))), err_msg=what)


@pytest.mark.parametrize("seed", range(24))
def test_forward_rows_match_the_numpy_oracle(seed):
    inp, kw = _case(seed)
    g = inp.get("g")
    want_out, want_fin = O.forward(inp["x"].double().numpy(), inp["coeffs"].numpy(), inp["damping"].numpy(),
                                   inp["lam"].numpy(), g=None if g is None else g.numpy(), **kw)
    for b in range(inp["x"].shape[0]):
        out, fin = oracle_c_forward_row(inp, b, **kw)
        _close(out, want_out[b], f"seed {seed} row {b} out")
        _close(fin, want_fin[b], f"seed {seed} row {b} ema_final")


@pytest.mark.parametrize("seed", range(24))
@pytest.mark.parametrize("target", ["x", "softsign"])
def test_ttt_rows_match_the_numpy_oracle(seed, target):
    inp, kw = _case(100 + seed)
    if inp["coeffs"].shape[2] > 8:
        inp["coeffs"] = inp["coeffs"][:, :, :8].contiguous()
    g = inp.get("g")
    B, S, D = inp["x"].shape
    G, want_out, want_fin = O.ttt_grad(inp["x"].double().numpy(), inp["coeffs"].numpy(), inp["damping"].numpy(),
                                       inp["lam"].numpy(), g=None if g is None else g.numpy(), target=target,
                                       ema_init=kw["ema_init"], nan_policy=kw["nan_policy"])
    if not kw["clamp_out"]:
        return   # the numpy TTT oracle always clamps; the C one follows it with clamp_out=1
    for b in range(B):
        Gc, out, fin = oracle_c_ttt_row(inp, b, n_total=B * (S - 1) * D, target=target, ema_init=kw["ema_init"],
                                        nan_policy=kw["nan_policy"])
        _close(out, want_out[b], f"seed {seed} row {b} out")
        _close(fin, want_fin[b], f"seed {seed} row {b} ema_final")
        _close(Gc, G[b], f"seed {seed} row {b} grad")


def test_planted_mistake_is_caught():
    """A wrong sign in the EMA of the numpy side shows as a mismatch."""
    inp, kw = _case(7)
    out, _ = oracle_c_forward_row(inp, 0, **kw)
    g = inp.get("g")
    want, _ = O.forward(inp["x"].double().numpy(), inp["coeffs"].numpy(), inp["damping"].numpy(),
                        -inp["lam"].numpy(), g=None if g is None else g.numpy(), **kw)
    with pytest.raises(AssertionError):
        _close(out, want[0], "planted")
