"""Pins the float64 oracle against library routines, closed forms, brute
force and autograd/finite differences (CPU only).  Each pin is chosen so a
plausible mistake (dropped term, wrong sign or index, transposed operand)
fails it; the mutation tests at the end plant such mistakes and check that
the pins catch them."""
import math

import numpy as np
import pytest
import scipy.signal
import torch
from numpy.polynomial import chebyshev as npcheb

from oracle import cheby_ema as O
from oracle import reference_form as RF

rng = np.random.default_rng(1234)


# ---------------------------------------------------------------- Clenshaw
@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8])
def test_clenshaw_matches_numpy_chebval(K):
    c = rng.standard_normal((50, K))
    u = rng.uniform(-1, 1, size=(50,))
    got = O.clenshaw(c, u)
    want = np.array([npcheb.chebval(u[i], c[i]) for i in range(50)])
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("k", range(8))
def test_clenshaw_unit_coefficient_is_cos_k_theta(k):
    theta = np.linspace(0, np.pi, 101)
    c = np.zeros(8)
    c[k] = 1.0
    np.testing.assert_allclose(O.clenshaw(c, np.cos(theta)), np.cos(k * theta), atol=1e-12)


def test_basis_matches_power_basis_brute_force():
    # T_0..T_7 in the power basis (textbook coefficients).
    power = {
        0: [1], 1: [0, 1], 2: [-1, 0, 2], 3: [0, -3, 0, 4], 4: [1, 0, -8, 0, 8],
        5: [0, 5, 0, -20, 0, 16], 6: [-1, 0, 18, 0, -48, 0, 32], 7: [0, -7, 0, 56, 0, -112, 0, 64],
    }
    u = rng.uniform(-1, 1, size=17)
    T = O.chebyshev_basis(u, 8)
    for k in range(8):
        want = sum(a * u ** i for i, a in enumerate(power[k]))
        np.testing.assert_allclose(T[:, k], want, atol=1e-12)


# ---------------------------------------------------------------- softsign
def test_softsign_special_values():
    x = np.array([0.0, -0.0, 1.0, -3.0, np.inf, -np.inf, 1e-40, 1e30, np.nan])
    u = O.softsign(x)
    np.testing.assert_array_equal(u[:6], [0.0, 0.0, 0.5, -0.75, 1.0, -1.0])
    assert u[6] == pytest.approx(1e-40, rel=1e-12)
    assert u[7] == pytest.approx(1.0, rel=1e-12)
    assert np.isnan(u[8])


def test_forward_k1_is_tanh_of_damped_constant():
    # K=1: p = c_0 regardless of x, so z = tanh(delta*c0): pins damping and tanh.
    B, S, H, hd = 1, 3, 2, 4
    x = rng.standard_normal((B, S, H * hd))
    c = rng.standard_normal((B, H, 1, hd))
    damp = np.array([0.7, 1.3])
    out, _, parts = O.forward(x, c, damp, [0.0, 0.0], return_parts=True)
    want = np.tanh(np.repeat(damp, hd) * c[0, :, 0, :].reshape(-1))
    np.testing.assert_allclose(parts["z"][0, 1], want, rtol=1e-14)
    np.testing.assert_allclose(out[0, 2], want, rtol=1e-14)   # lam = 0: s = z


# ---------------------------------------------------------------- EMA
def test_ema_matches_scipy_lfilter_with_initial_state():
    B, S, H, hd = 2, 300, 3, 4
    x = rng.standard_normal((B, S, H * hd))
    c = rng.standard_normal((B, H, 5, hd)) * 0.5
    lam = np.array([0.9, 0.99, 0.5])
    init = rng.uniform(-0.5, 0.5, size=(B, H * hd))
    out, fin, parts = O.forward(x, c, O.baseline_damping(H), lam, ema_init=init, clamp_out=False,
                                return_parts=True)
    z = parts["z"]
    for b in range(B):
        for d in range(H * hd):
            lm = lam[d // hd]
            y, _ = scipy.signal.lfilter([1 - lm], [1, -lm], z[b, :, d], zi=[lm * init[b, d]])
            np.testing.assert_allclose(out[b, :, d], y, rtol=1e-12, atol=1e-14)
            assert fin[b, d] == pytest.approx(y[-1], rel=1e-12)


def test_ema_closed_forms():
    # z constant: force p = c0 with K=1 and large c0 so z = tanh(...) known.
    S, lam = 200, 0.97
    x = np.zeros((1, S, 4))
    c = np.full((1, 1, 1, 4), 0.3)
    out, _, parts = O.forward(x, c, [1.0], [lam], return_parts=True)
    z = math.tanh(0.3)
    t = np.arange(S)
    np.testing.assert_allclose(out[0, :, 0], z * (1 - lam ** (t + 1)), rtol=1e-12)
    # impulse response: z = 1 at t=0 only -> (1-lam) lam^t.  Use NaN (z=0) elsewhere.
    x2 = np.full((1, S, 4), np.nan)
    x2[0, 0] = 0.0
    c2 = np.full((1, 1, 1, 4), 50.0)   # tanh(50) == 1 in float64
    out2, _ = O.forward(x2, c2, [1.0], [lam])
    np.testing.assert_allclose(out2[0, :, 0], (1 - lam) * lam ** t, rtol=1e-12)


def test_lambda_zero_is_identity_and_clamp_binds_only_outside():
    x = rng.standard_normal((1, 10, 8))
    c = rng.standard_normal((1, 2, 8, 4))
    out, _, parts = O.forward(x, c, [1.0, 1.0], [0.0, 0.0], return_parts=True)
    np.testing.assert_array_equal(out, parts["z"])
    # |ema_init| > 1: the output is clamped, the carried state is not.
    out3, fin3, p3 = O.forward(x[:, :1], c, [1.0, 1.0], [0.999, 0.999], ema_init=np.full((1, 8), 5.0),
                               return_parts=True)
    assert np.all(out3 == 1.0) and np.all(p3["s"] > 4.9) and np.all(fin3 > 4.9)


def test_nan_input_gives_zero_z():
    x = rng.standard_normal((1, 6, 8))
    x[0, 3, 5] = np.nan
    c = rng.standard_normal((1, 2, 8, 4))
    lam = [0.9, 0.8]
    out, _, parts = O.forward(x, c, [1.0, 1.0], lam, return_parts=True)
    assert parts["z"][0, 3, 5] == 0.0
    assert out[0, 3, 5] == pytest.approx(lam[1] * out[0, 2, 5], rel=1e-14)


# ---------------------------------------------------------------- dynamic lambda
def _brute_dynamic(x, c, damp, lam, g, shift, lo, hi, init):
    """Scalar loops with math.* only (independent of numpy vectorisation)."""
    B, S, D = x.shape
    _, H, K, hd = c.shape
    out = np.zeros_like(x)
    fin = np.zeros((B, D))
    for b in range(B):
        for d in range(D):
            h, j = divmod(d, hd)
            s = init[b, d]
            for t in range(S):
                u = x[b, t, d] / (1 + abs(x[b, t, d]))
                T = [1.0, u]
                for _ in range(2, K):
                    T.append(2 * u * T[-1] - T[-2])
                p = sum(c[b, h, k, j] * T[k] for k in range(K))
                z = math.tanh(damp[h] * p)
                lm = min(max(lam[h] + shift * g[b, t, h], lo), hi)
                s = lm * s + (1 - lm) * z
                out[b, t, d] = min(max(s, -1.0), 1.0)
            fin[b, d] = s
    return out, fin


def test_dynamic_lambda_matches_brute_force_and_clamps():
    B, S, H, hd, K = 2, 20, 2, 4, 8
    x = rng.standard_normal((B, S, H * hd))
    c = rng.standard_normal((B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, K, 1)
    g = rng.uniform(-1, 1, size=(B, S, H))
    init = rng.uniform(-0.3, 0.3, size=(B, H * hd))
    lam, damp = np.array([0.95, 0.5]), np.array([1.0, 0.9])
    for shift in (0.004, 0.3):       # 0.3 drives lambda into both clamp bounds
        out, fin = O.forward(x, c, damp, lam, g=g, lam_shift=shift, ema_init=init)
        bo, bf = _brute_dynamic(x, c, damp, lam, g, shift, 0.9, 0.9999, init)
        np.testing.assert_allclose(out, bo, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(fin, bf, rtol=1e-12, atol=1e-14)
    lt = O.lambda_field(lam, B, S, H, g, 0.3, 0.9, 0.9999)
    assert lt.min() == 0.9 and lt.max() == 0.9999


def test_g_broadcast_over_batch():
    g = rng.uniform(-1, 1, size=(5, 2))
    lt = O.lambda_field([0.95, 0.97], 3, 5, 2, g)
    assert lt.shape == (3, 5, 2) and np.all(lt[0] == lt[2])


# ---------------------------------------------------------------- carry
@pytest.mark.parametrize("chunk", [1, 7, 64])
def test_chunked_with_carry_equals_monolithic(chunk):
    B, S, H, hd = 2, 130, 2, 4
    x = rng.standard_normal((B, S, H * hd))
    c = rng.standard_normal((B, H, 8, hd)) * 0.4
    g = rng.uniform(-1, 1, size=(S, H))
    mono, fm = O.forward(x, c, [1.0, 0.9], [0.99, 0.95], g=g)
    ch, fc = O.forward_chunked(x, c, [1.0, 0.9], [0.99, 0.95], chunk, g=g)
    np.testing.assert_allclose(ch, mono, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(fc, fm, rtol=1e-13, atol=1e-15)


# ---------------------------------------------------------------- TTT gradient
@pytest.mark.parametrize("dyn,target", [(False, "x"), (True, "x"), (False, "softsign")])
def test_ttt_adjoint_matches_autograd(dyn, target):
    # own generator: the module-level one's state depends on test order
    r = np.random.default_rng(40 + 2 * dyn + (target == "x"))
    B, S, H, hd, K = 2, 33, 2, 4, 8
    x = r.standard_normal((B, S, H * hd))
    c = r.standard_normal((B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, K, 1)
    g = r.uniform(-1, 1, size=(B, S, H)) if dyn else None
    init = r.uniform(-0.5, 0.5, size=(B, H * hd))
    kw = dict(g=g, lam_shift=0.05, ema_init=init, target=target)
    G, out, fin = O.ttt_grad(x, c, [1.0, 0.8], [0.9, 0.97], **kw)
    Ga, outa, fina = O.ttt_grad_autograd(x, c, [1.0, 0.8], [0.9, 0.97], **kw)
    # adjoint sums and autograd sums round differently: elements that cancel
    # to near zero are compared against the gradient's scale
    np.testing.assert_allclose(G, Ga, rtol=1e-10, atol=1e-12 * np.abs(Ga).max())
    np.testing.assert_allclose(out, outa, rtol=1e-13, atol=1e-15 * np.abs(outa).max())


def test_ttt_gradient_matches_central_finite_differences():
    # Multi-epsilon central differences, median over eps (the method of the
    # reference's gradient checker, gradient_checker.py:154-226).
    B, S, H, hd, K = 1, 12, 1, 4, 8
    x = rng.standard_normal((B, S, H * hd))
    c = rng.standard_normal((B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, K, 1)
    G, _, _ = O.ttt_grad(x, c, [0.9], [0.8])

    def loss(cc):
        out, _ = O.forward(x, cc, [0.9], [0.8])
        return np.mean((out[:, :-1] - x[:, 1:]) ** 2)

    fd = np.zeros_like(c)
    for idx in np.ndindex(c.shape):
        ests = []
        for eps in (1e-4, 3e-5, 1e-5):
            cp, cm = c.copy(), c.copy()
            cp[idx] += eps
            cm[idx] -= eps
            ests.append((loss(cp) - loss(cm)) / (2 * eps))
        fd[idx] = np.median(ests)
    scale = (np.arange(1, K + 1) ** 2).reshape(1, 1, K, 1)
    np.testing.assert_allclose(G * scale, fd, rtol=1e-6, atol=1e-10)


def test_ttt_short_sequence_is_zero():
    G, _, _ = O.ttt_grad(rng.standard_normal((1, 1, 4)), rng.standard_normal((1, 1, 8, 4)), [1.0], [0.9])
    assert np.all(G == 0)


# ---------------------------------------------------------------- backward
def _bwd_case(B, S, H, hd, K, dyn, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((B, S, H * hd))
    c = r.standard_normal((B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, K, 1)
    g = r.uniform(-1, 1, size=(B, S, H)) if dyn else None
    init = r.uniform(-0.5, 0.5, size=(B, H * hd))
    go = r.standard_normal(x.shape)
    gs = r.standard_normal((B, H * hd))
    return x, c, g, init, go, gs


@pytest.mark.parametrize("dyn", [False, True])
@pytest.mark.parametrize("nan_policy", ["zero_z", "zero_u"])
def test_backward_matches_autograd(dyn, nan_policy):
    x, c, g, init, go, gs = _bwd_case(2, 37, 2, 4, 8, dyn, 11)
    x[0, 5, 3] = np.nan
    x[1, 9, 0] = 0.0
    x[1, 10, 6] = np.inf
    kw = dict(g=g, lam_shift=0.05, ema_init=init, grad_state=gs, nan_policy=nan_policy)
    gx, gc, gi = O.backward(x, c, [1.0, 0.8], [0.9, 0.97], go, **kw)
    ax, ac, ai, _ = O.backward_autograd(x, c, [1.0, 0.8], [0.9, 0.97], go, **kw)
    np.testing.assert_allclose(gx, ax, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(gc, ac, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(gi, ai, rtol=1e-10, atol=1e-14)
    assert gx[0, 5, 3] == 0 and gx[1, 9, 0] == 0 and gx[1, 10, 6] == 0


def test_backward_matches_central_finite_differences():
    B, S, H, hd, K = 1, 10, 1, 3, 8
    x, c, _, init, go, gs = _bwd_case(B, S, H, hd, K, False, 12)
    gx, gc, gi = O.backward(x, c, [0.9], [0.8], go, ema_init=init, grad_state=gs)

    def loss(xx, cc, ii):
        out, fin = O.forward(xx, cc, [0.9], [0.8], ema_init=ii)
        return np.sum(out * go) + np.sum(fin * gs)

    def fd(arr, f):
        d = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            ests = []
            for eps in (1e-4, 3e-5, 1e-5):
                ap, am = arr.copy(), arr.copy()
                ap[idx] += eps
                am[idx] -= eps
                ests.append((f(ap) - f(am)) / (2 * eps))
            d[idx] = np.median(ests)
        return d

    np.testing.assert_allclose(gx, fd(x, lambda a: loss(a, c, init)), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(gc, fd(c, lambda a: loss(x, a, init)), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(gi, fd(init, lambda a: loss(x, c, a)), rtol=1e-6, atol=1e-9)


def test_backward_tiny_inputs_pass_no_gradient_to_x():
    x, c, _, _, go, _ = _bwd_case(1, 8, 1, 4, 8, False, 13)
    x[0, 2, :] = [3e-8, -5e-8, 2e-7, -1e-6]
    gx, _, _ = O.backward(x, c, [1.0], [0.9], go)
    ax, _, _, _ = O.backward_autograd(x, c, [1.0], [0.9], go)
    assert gx[0, 2, 0] == 0 and gx[0, 2, 1] == 0 and gx[0, 2, 2] != 0
    np.testing.assert_allclose(gx, ax, rtol=1e-9, atol=1e-14)


def test_backward_mask_gates_the_carried_adjoint():
    # Lane 0 saturates (z = 1 exactly, init = 1): every output sits at the
    # clamp, so the reference's mask zeroes its adjoint, carry included.
    # Autograd of a forward whose state is clamped at 1 - 1e-6 has the same
    # gradient; the plain forward's autograd does not (its grad_init is not 0).
    r = np.random.default_rng(14)
    x = np.full((1, 30, 2), 5.0)
    x[:, 20:] = r.standard_normal((1, 10, 2))
    c = np.zeros((1, 1, 8, 2))
    c[0, 0, 0] = [30.0, 0.3]
    c[0, 0, 1] = 1.0
    go = r.standard_normal(x.shape)
    init = np.array([[1.0, 0.1]])
    ax, ac, ai, out_c = O.backward_autograd(x, c, [1.0], [0.9], go, ema_init=init, state_clamp=1 - 1e-6)
    gx, gc, gi = O.backward(x, c, [1.0], [0.9], go, ema_init=init, out_saved=out_c)
    np.testing.assert_allclose(gx, ax, atol=1e-14)
    np.testing.assert_allclose(gc, ac, atol=1e-13)
    np.testing.assert_allclose(gi, ai, atol=1e-14)
    assert gi[0, 0] == 0
    assert O.backward_autograd(x, c, [1.0], [0.9], go, ema_init=init)[2][0, 0] > 0.05


def test_backward_chunked_with_carry_equals_monolithic():
    x, c, g, init, go, gs = _bwd_case(2, 48, 2, 4, 8, True, 15)
    kw = dict(lam_shift=0.05)
    gx, gc, gi = O.backward(x, c, [1.0, 0.8], [0.9, 0.97], go, g=g, ema_init=init, grad_state=gs, **kw)
    # forward carries, then the backward runs chunk by chunk from the end,
    # each chunk's grad_init becoming the previous chunk's grad_state.
    bounds = [(0, 17), (17, 30), (30, 48)]
    inits = [init]
    for t0, t1 in bounds[:-1]:
        inits.append(O.forward(x[:, t0:t1], c, [1.0, 0.8], [0.9, 0.97], g=g[:, t0:t1],
                               ema_init=inits[-1], **kw)[1])
    gxs, gcs, carry = [], np.zeros_like(gc), gs
    for (t0, t1), ini in reversed(list(zip(bounds, inits))):
        a, b, carry = O.backward(x[:, t0:t1], c, [1.0, 0.8], [0.9, 0.97], go[:, t0:t1], g=g[:, t0:t1],
                                 ema_init=ini, grad_state=carry, **kw)
        gxs.insert(0, a)
        gcs += b
    np.testing.assert_allclose(np.concatenate(gxs, axis=1), gx, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(gcs, gc, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(carry, gi, rtol=1e-12, atol=1e-15)


# ---------------------------------------------------------------- reference form
def test_reference_form_agrees_with_oracle():
    B, S, H, hd, K = 2, 200, 4, 8, 8
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(B, S, H * hd, generator=gen)
    x[0, 5, 3] = float("nan")
    x[1, 9, 0] = 0.0
    c = torch.randn(B, H, K, hd, generator=gen) / torch.arange(1, K + 1).view(1, 1, K, 1)
    damp = torch.tensor([0.9 ** h for h in range(H)])
    lam = torch.tensor([0.9995, 0.997, 0.995, 0.95])
    out_rf, fin_rf = RF.forward(x, c, damp, lam)
    out_o, fin_o = O.forward(x.numpy(), c.numpy(), damp.numpy(), lam.numpy())
    # The reference form maps a NaN input to u = 0 (sdpc_kernel.py:1725), so
    # z there is tanh(delta*p(0)) instead of 0: compare the other lanes ...
    mask = np.ones(out_o.shape, bool)
    mask[0, 5:, 3] = False
    assert O.rel_err(out_rf.numpy()[mask], out_o[mask]) < 2e-6
    assert not np.allclose(out_rf.numpy()[0, 5:, 3], out_o[0, 5:, 3])
    # ... and every lane under the oracle's "zero_u" policy.
    out_u, fin_u = O.forward(x.numpy(), c.numpy(), damp.numpy(), lam.numpy(), nan_policy="zero_u")
    assert O.rel_err(out_rf.numpy(), out_u) < 2e-6
    assert O.rel_err(fin_rf.numpy(), fin_u) < 2e-6


def test_reference_form_backward_agrees_with_oracle():
    B, S, H, hd, K = 2, 150, 4, 8, 8
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(B, S, H * hd, generator=gen)
    x[0, 5, 3] = float("nan")
    x[1, 9, 0] = 0.0
    c = torch.randn(B, H, K, hd, generator=gen) / torch.arange(1, K + 1).view(1, 1, K, 1)
    c[1, 2, 0, :] = 12.0                     # head 2 of batch 1 saturates: the mask binds
    damp = torch.tensor([0.9 ** h for h in range(H)])
    lam = torch.tensor([0.9995, 0.997, 0.8, 0.95])
    go = torch.randn(B, S, H * hd, generator=gen)
    out_rf, _ = RF.forward(x, c, damp, lam, ema_init=None)
    gx_rf, gc_rf = RF.backward(x, c, damp, lam, out_rf, go)
    assert (out_rf.abs() >= 1 - 1e-6).any()
    gx, gc, _ = O.backward(x.numpy(), c.numpy(), damp.numpy(), lam.numpy(), go.double().numpy(),
                           nan_policy="zero_u", out_saved=out_rf.numpy())
    assert O.rel_err(gx_rf.numpy(), gx) < 2e-5
    assert O.rel_err(gc_rf.numpy(), gc) < 2e-5


# ---------------------------------------------------------------- mutation checks
def test_pins_catch_a_dropped_coefficient(monkeypatch):
    """The reference's megakernel Clenshaw fallback drops c4..c7
    (sdpc_kernel.py:2070-2077); an oracle with that bug must fail the chebval pin."""
    orig = O.clenshaw
    monkeypatch.setattr(O, "clenshaw", lambda c, u: orig(np.asarray(c)[..., :4], u))
    with pytest.raises(AssertionError):
        test_clenshaw_matches_numpy_chebval(8)


def test_pins_catch_a_wrong_sign_in_the_ema(monkeypatch):
    orig = O.forward

    def bad_forward(*a, **kw):
        lam = np.asarray(a[3], dtype=np.float64)
        return orig(a[0], a[1], a[2], -lam, *a[4:], **kw)

    monkeypatch.setattr(O, "forward", bad_forward)
    with pytest.raises(AssertionError):
        test_ema_matches_scipy_lfilter_with_initial_state()


def test_pins_catch_a_missing_spectral_scale(monkeypatch):
    orig = O.ttt_grad

    def bad(*a, **kw):
        G, out, fin = orig(*a, **kw)
        K = G.shape[2]
        return G * (np.arange(1, K + 1) ** 2).reshape(1, 1, K, 1), out, fin   # forgets 1/(k+1)^2

    monkeypatch.setattr(O, "ttt_grad", bad)
    with pytest.raises(AssertionError):
        test_ttt_gradient_matches_central_finite_differences()
