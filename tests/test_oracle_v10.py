"""Pins of the full-path oracle (oracle/v10_full.py) against library
routines, closed forms and brute force (CPU only)."""
import math

import numpy as np
import pytest
import scipy.signal
import torch
from numpy.polynomial import chebyshev as npcheb

from oracle import v10_full as V

rng = np.random.default_rng(4321)


def test_bf16_round_matches_torch():
    x = rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-40, 38, 20000).astype(np.float32)
    x[:6] = [0.0, -0.0, np.inf, -np.inf, 3.3895314e38, 1e-45]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = V.bf16_round(x)
    np.testing.assert_array_equal(got, want.astype(np.float64))
    assert np.isnan(V.bf16_round(np.array([np.nan], np.float32)))[0]


def test_lut_is_chebyshev_at_its_grid():
    lut = V.chebyshev_lut()
    grid = torch.linspace(0.0, 1.0, 256).numpy().astype(np.float64)
    for k in range(8):
        np.testing.assert_allclose(lut[k], np.cos(k * np.arccos(grid)), atol=2e-6)


@pytest.mark.parametrize("K", [1, 3, 8])
def test_lut_series_interpolates_the_chebyshev_series(K):
    lut = V.chebyshev_lut()
    c = rng.standard_normal((40, K))
    # at the grid points (both signs, odd terms flip): the series itself
    i = rng.integers(0, 256, 40)
    a = i / 255.0
    for sgn in (1.0, -1.0):
        got = V.lut_series(c, a, np.full(40, sgn), lut)
        want = np.array([npcheb.chebval(sgn * a[j], c[j]) for j in range(40)])
        np.testing.assert_allclose(got, want, atol=2e-5 * K)
    # between grid points: linear interpolation error <= h^2/8 max|p''|
    a = rng.uniform(0, 1, 40)
    got = V.lut_series(c, a, np.ones(40), lut)
    want = np.array([npcheb.chebval(a[j], c[j]) for j in range(40)])
    bound = (1 / 255) ** 2 / 8 * np.abs(c).sum(axis=1) * (K - 1) ** 4 + 2e-5 * K
    assert np.all(np.abs(got - want) <= bound)


def test_clenshaw4_uses_only_the_first_four_coefficients():
    c = rng.standard_normal((30, 8))
    u = rng.uniform(-1, 1, 30)
    got = V.clenshaw4_series(c, u)
    want = np.array([npcheb.chebval(u[j], c[j, :4]) for j in range(30)])
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(V.clenshaw4_series(c[:, :2], u),
                               [npcheb.chebval(u[j], c[j, :2]) for j in range(30)], atol=1e-13)


def test_softsign_special_values():
    xb = np.array([np.nan, 0.0, -0.0, 1.0, -3.0, np.inf, -np.inf])
    u, absu, sign, nan = V.v10_softsign(xb)
    assert nan.tolist() == [True] + [False] * 6
    assert u[0] > 0 and u[0] == u[1] == u[2] and u[0] < 1.2e-7          # NaN and +-0 -> +1e-7 side
    np.testing.assert_allclose(u[3:], [0.5, -0.75, 1.0, -1.0], rtol=1e-12)


def _chunk_inputs(B=2, L=40, H=2, hd=4, K=8):
    x = V.bf16_round(rng.standard_normal((B, L, H * hd)).astype(np.float32))
    c = rng.standard_normal((B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, K, 1)
    m = rng.standard_normal((B, H, K, hd)) * 0.01
    return x, c, m


KW = dict(ema_momentum=0.9, base_lr=0.005, beta1=0.9, beta2=0.99, wd=0.01)


def test_chunk_ema_restarts_from_zero_and_matches_lfilter():
    x, c, m = _chunk_inputs()
    s, _, _, z = V.v10_chunk(x, c, m, **KW)
    for b in range(2):
        for d in range(8):
            y = scipy.signal.lfilter([0.1], [1, -0.9], z[b, :, d])
            np.testing.assert_allclose(s[b, :, d], y, rtol=1e-12, atol=1e-15)
    assert np.all(np.abs(z) <= math.tanh(4.0) + 1e-15)


def test_chunk_tanh_clamps_at_four_and_nan_gives_zero():
    x, c, m = _chunk_inputs(B=1, L=6, H=1, hd=4, K=2)
    c[0, 0, 0, :] = [50.0, -50.0, 0.2, 0.0]
    c[0, 0, 1, :] = 0.0
    x[0, 3, 2] = np.nan
    _, _, _, z = V.v10_chunk(x, c, m, **KW)
    gamma = 0.98
    np.testing.assert_allclose(z[0, :, 0], math.tanh(4.0), rtol=1e-14)
    np.testing.assert_allclose(z[0, :, 1], -math.tanh(4.0), rtol=1e-14)
    np.testing.assert_allclose(z[0, [0, 1, 2, 4, 5], 2], math.tanh(0.2 * gamma), rtol=1e-13)
    assert z[0, 3, 2] == 0.0


def test_proxy_gradient_brute_force():
    B, L, D, K = 1, 9, 3, 8
    u = rng.uniform(-1, 1, (B, L, D))
    s = rng.uniform(-1, 1, (B, L, D))
    got = V.proxy_grad(u, s, K)
    for d in range(D):
        for k in range(K):
            acc = 0.0
            for t in range(L - 1):
                e = u[0, t + 1, d] - s[0, t, d]
                acc += e / (1 + math.exp(-3 * abs(e))) * math.cos(k * math.acos(u[0, t, d]))
            assert got[0, d, k] == pytest.approx(acc, rel=1e-10, abs=1e-12)
    # s that predicts u one step ahead gives no gradient
    s2 = np.zeros_like(s)
    s2[:, :-1] = u[:, 1:]
    assert np.all(V.proxy_grad(u, s2, K) == 0)


def test_lion_closed_forms():
    B, H, K, hd = 2, 4, 3, 1
    c = np.ones((B, H, K, hd))
    m = np.zeros((B, H, K, hd))
    gc = np.zeros((B, H, K, hd))
    gc[0, :, 0] = 5.0            # g = +1 over L = 6 tokens
    gc[0, :, 1] = -5.0
    gc[1, 0, 2] = 1e-30
    cn, mn = V.lion_update(c, m, gc, 6, base_lr=0.005, beta1=0.9, beta2=0.99, wd=0.01)
    lam = np.array([0.9995, 0.9995, 0.997, 0.997])
    lr = 0.005 * (1 + 0.25 * (np.arange(4) - 2) / 4)
    decay = lam - lr * 0.01
    np.testing.assert_allclose(cn[0, :, 0, 0], decay + lr, rtol=1e-14)                 # sign +1, ss_0 = 1
    np.testing.assert_allclose(cn[0, :, 1, 0], decay - lr / 2 ** 1.5, rtol=1e-14)      # sign -1, ss_1
    np.testing.assert_allclose(cn[0, :, 2, 0], decay, rtol=1e-14)                      # g = 0: sign 0
    np.testing.assert_allclose(mn[0, :, 0, 0], 0.01, rtol=1e-12)                       # (1 - b2) g
    assert cn[1, 0, 2, 0] == pytest.approx(decay[0] + lr[0] / 3 ** 1.5, rel=1e-14)
    # gate scales lr (and so the decay); dynamic lambda moves the forget factor
    gate = np.array([0.5, 2.0])
    dyn = np.array([1.0, -50.0])
    cg, _ = V.lion_update(c, m, gc, 6, base_lr=0.005, beta1=0.9, beta2=0.99, wd=0.01, gate=gate, dyn=dyn)
    lam_d = np.minimum(lam + 0.008 * 0.5, 0.9999)
    np.testing.assert_allclose(cg[0, :, 0, 0], lam_d - 0.5 * lr * 0.01 + 0.5 * lr, rtol=1e-14)
    np.testing.assert_allclose(cg[1, :, 1, 0], 0.9 - 2 * lr * 0.01, rtol=1e-14)      # clamped at 0.9
    # momentum drives the sign: m > 0 overrides a small negative g
    m2 = np.full((B, H, K, hd), 1.0)
    cm, mm = V.lion_update(c, m2, -gc * 1e-3, 6, base_lr=0.005, beta1=0.9, beta2=0.99, wd=0.01)
    np.testing.assert_allclose(cm[0, :, 0, 0], decay + lr, rtol=1e-14)


def test_lion_one_token_chunk_poisons_momentum_like_the_reference():
    # len - 1 = 0: g = 0 * inf = NaN, so sign = 0 and momentum becomes NaN.
    c = np.ones((1, 1, 2, 1))
    cn, mn = V.lion_update(c, np.zeros_like(c), np.zeros_like(c), 1, base_lr=0.005, beta1=0.9, beta2=0.99,
                           wd=0.01)
    assert np.all(np.isnan(mn)) and np.all(np.isfinite(cn))


def test_full_path_chains_coefficients_over_chunks():
    B, S, H, hd, K = 2, 70, 2, 4, 8
    x = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    c = rng.standard_normal((B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, K, 1)
    m = np.zeros_like(c)
    out, cn, mn = V.v10_full(x, c, m, n_heads=H, chunk_size=32)
    xb = V.bf16_round(x)
    cc, mm = c, m
    outs = []
    for t0 in (0, 32, 64):
        s, cc, mm, _ = V.v10_chunk(xb[:, t0:t0 + 32], cc, mm, **KW)
        outs.append(V.bf16_round(s.astype(np.float32)))
    np.testing.assert_array_equal(out, np.concatenate(outs, axis=1))
    np.testing.assert_array_equal(cn, cc)
    # the EMA restarts at every chunk: out at a chunk's first token is (1 - mu) z
    _, _, _, z = V.v10_chunk(xb[:, 32:64], V.v10_chunk(xb[:, :32], c, m, **KW)[1],
                             V.v10_chunk(xb[:, :32], c, m, **KW)[2], **KW)
    np.testing.assert_allclose(out[:, 32], V.bf16_round((0.1 * z[:, 0]).astype(np.float32)))
    # one chunk when S <= chunk_size
    o1, c1, _ = V.v10_full(x[:, :20], c, m, n_heads=H, chunk_size=32)
    s1, c1b, _, _ = V.v10_chunk(xb[:, :20], c, m, **KW)
    np.testing.assert_array_equal(c1, c1b)


def test_full_path_backward_reduces_to_the_pinned_fast_path_backward():
    # With zb = the exact tanh of the exact series (no LUT, no bf16, no +-4
    # clamp binding) each chunk's backward is the fast-path backward of
    # oracle/cheby_ema.py (pinned by autograd and finite differences) with
    # damping gamma_h, lambda mu on every head, no state gradient.
    from oracle import cheby_ema as O
    B, S, H, hd, K, chunk = 2, 70, 2, 4, 8, 32
    x = rng.standard_normal((B, S, H * hd))
    hist = rng.standard_normal((3, B, H, K, hd)) / np.arange(1, K + 1).reshape(1, 1, 1, K, 1) * 0.5
    go = rng.standard_normal((B, S, H * hd))
    gamma = 0.98 - 0.06 * np.arange(H) / H
    mu = 0.9
    outs, zs = [], []
    for ch in range(3):
        t0, t1 = ch * chunk, min((ch + 1) * chunk, S)
        o, _, parts = O.forward(x[:, t0:t1], hist[ch], gamma, np.full(H, mu), return_parts=True)
        outs.append(o)
        zs.append(parts["z"])
    out, z = np.concatenate(outs, axis=1), np.concatenate(zs, axis=1)
    gx, gc = V.v10_backward(x, out, z, hist, go, n_heads=H, ema_momentum=mu, chunk=chunk)
    for ch in range(3):
        t0, t1 = ch * chunk, min((ch + 1) * chunk, S)
        wx, wc, _ = O.backward(x[:, t0:t1], hist[ch], gamma, np.full(H, mu), go[:, t0:t1])
        np.testing.assert_allclose(gx[:, t0:t1], wx, rtol=1e-9, atol=1e-13)
        if ch == 0:
            np.testing.assert_allclose(gc, wc, rtol=1e-9, atol=1e-13)


def test_full_path_backward_nan_gives_nan_grad_x():
    B, S, H, hd, K = 1, 10, 1, 4, 4
    x = rng.standard_normal((B, S, H * hd))
    x[0, 3, 1] = np.nan
    hist = rng.standard_normal((1, B, H, K, hd))
    gx, gc = V.v10_backward(x, np.zeros_like(x), np.zeros_like(x), hist, np.ones_like(x), n_heads=H,
                            ema_momentum=0.9, chunk=256)
    assert np.isnan(gx[0, 3, 1]) and np.isfinite(np.delete(gx.reshape(-1), 3 * 4 + 1)).all()
    assert np.isfinite(gc).all()


# The fused Clenshaw + EMA kernel (_fused_clenshaw_ema_kernel,
# sdpc_kernel.py:988-1209), restated by V.fused_clenshaw_ema.

def test_clenshaw8_is_the_chebyshev_series_of_all_eight_terms():
    u = rng.uniform(-1, 1, 30)
    for K in (5, 6, 8):
        c = rng.standard_normal((30, K))
        got = V.clenshaw8_series(c, u)
        want = np.array([npcheb.chebval(u[j], c[j]) for j in range(30)])
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("K,use_lut", [(3, False), (4, False), (6, False), (8, False), (8, True), (2, True)])
def test_fused_clenshaw_ema_series_tanh_and_scan(K, use_lut):
    B, S, H, hd = 2, 300, 2, 4
    D = H * hd
    x = rng.standard_normal((B, S, D)).astype(np.float32)
    c = rng.standard_normal((B, H, K, hd)) / 2
    xn, ty, out, fin = V.fused_clenshaw_ema(x, c, n_heads=H, ema_momentum=0.93, use_lut=use_lut)
    u = np.sign(x) * (1.0 - 1.0 / (1.0 + np.maximum(np.abs(x.astype(np.float64)), np.float32(1e-7))))
    np.testing.assert_allclose(xn, u, rtol=1e-15)
    cl = c.transpose(0, 1, 3, 2).reshape(B, 1, D, K)
    if use_lut:
        lut = V.chebyshev_lut()
        p = V.lut_series(cl, np.abs(u), np.sign(u), lut)
        # the LUT series is within its interpolation bound of the exact series
        exact = np.stack([[npcheb.chebval(u[b, :, d], cl[b, 0, d]) for d in range(D)] for b in range(B)], 0)
        assert np.abs(p - exact.transpose(0, 2, 1)).max() < 1e-3
    else:
        terms = cl if K > 4 else cl[..., :4]
        p = np.stack([[npcheb.chebval(u[b, :, d], terms[b, 0, d]) for d in range(D)] for b in range(B)], 0)
        p = p.transpose(0, 2, 1)
    gamma = np.repeat(0.98 - 0.06 * np.arange(H) / H, hd)
    np.testing.assert_allclose(ty, np.tanh(np.clip(gamma * p, -4, 4)), atol=1e-12)
    # zero initial state: every clamp is the identity and the EMA is lfilter's
    ema = scipy.signal.lfilter([0.07], [1.0, -0.93], ty, axis=1)
    np.testing.assert_allclose(out, ema, atol=1e-12)
    np.testing.assert_allclose(fin, ema[:, -1], atol=1e-12)


def test_fused_clenshaw_ema_clamps_the_carry_at_tile_boundaries():
    B, S, H, hd = 1, 200, 1, 3
    x = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    c = rng.standard_normal((B, H, 4, hd)) / 4
    mu = 0.9999
    init = np.array([[5.0, -3.0, 0.5]])
    _, ty, out, fin = V.fused_clenshaw_ema(x, c, n_heads=H, ema_momentum=mu, ema_init=init, block_s=64)
    assert np.all(np.abs(out) <= 1.0)
    # inside the first tile the state runs from the unclamped init: out is
    # the clipped EMA of lfilter with that initial condition
    first = scipy.signal.lfilter([1 - mu], [1.0, -mu], ty[:, :64], axis=1, zi=mu * init[:, None, :])[0]
    np.testing.assert_allclose(out[:, :64], np.clip(first, -1, 1), atol=1e-12)
    # from the second tile on, the carry is the clipped state
    second = scipy.signal.lfilter([1 - mu], [1.0, -mu], ty[:, 64:128], axis=1,
                                  zi=mu * np.clip(first[:, -1:, :], -1, 1))[0]
    np.testing.assert_allclose(out[:, 64:128], np.clip(second, -1, 1), atol=1e-12)
    # a tile as long as the sequence never clamps the carry: only the output
    _, _, out_1, _ = V.fused_clenshaw_ema(x, c, n_heads=H, ema_momentum=mu, ema_init=init, block_s=256)
    whole = scipy.signal.lfilter([1 - mu], [1.0, -mu], ty, axis=1, zi=mu * init[:, None, :])[0]
    np.testing.assert_allclose(out_1, np.clip(whole, -1, 1), atol=1e-12)
    assert np.abs(out_1 - out).max() > 1e-3      # lane 0 starts at 5: the carry clamp binds
    # |init| <= 1: the tile size does not matter
    init2 = np.array([[0.9, -1.0, 0.2]])
    a = V.fused_clenshaw_ema(x, c, n_heads=H, ema_momentum=mu, ema_init=init2, block_s=32)
    b = V.fused_clenshaw_ema(x, c, n_heads=H, ema_momentum=mu, ema_init=init2, block_s=512)
    np.testing.assert_allclose(a[2], b[2], atol=1e-13)
    np.testing.assert_allclose(fin, out[:, -1], atol=0)


def test_fused_clenshaw_ema_special_values_and_empty_sequence():
    # token t of every lane holds special value t
    vals = np.array([np.nan, 0.0, np.inf, -np.inf, -0.0, 3e38, 1e-30, -2.0], np.float32)
    x = np.repeat(vals.reshape(1, 8, 1), 8, axis=2)
    c = np.ones((1, 1, 8, 8)) * 0.1
    xn, ty, out, fin = V.fused_clenshaw_ema(x, c, n_heads=1)
    assert np.all(np.isfinite(out)) and np.all(np.isfinite(xn)) and np.all(np.isfinite(ty))
    tiny = 1.0 - 1.0 / (1.0 + np.float64(np.float32(1e-7)))
    # NaN reads as 0 (x_norm = +tiny) and gives tanh_y = 0; +-Inf give +-1
    assert xn[0, 0, 0] == pytest.approx(tiny, rel=1e-12) and ty[0, 0, 0] == 0.0
    assert xn[0, 1, 0] == pytest.approx(tiny, rel=1e-12) and xn[0, 4, 0] == pytest.approx(tiny, rel=1e-12)
    assert xn[0, 2, 0] == 1.0 and xn[0, 3, 0] == -1.0 and xn[0, 6, 0] == pytest.approx(tiny, rel=1e-12)
    init = rng.standard_normal((1, 8)) * 3
    _, _, out0, fin0 = V.fused_clenshaw_ema(np.zeros((1, 0, 8), np.float32), c, n_heads=1, ema_init=init)
    assert out0.shape == (1, 0, 8)
    np.testing.assert_array_equal(fin0, init)            # unclamped, as the kernel's untouched carry


def test_fused_clenshaw_ema_matches_the_full_path_output_on_one_chunk():
    # precision_tests.py P1: on one chunk with a zero state, the full path's
    # output before Lion is this kernel's on bf16 x, up to the bf16 rounding
    B, S, H, hd, K = 2, 256, 8, 8, 4
    x = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    c = rng.standard_normal((B, H, K, hd))
    full, _, _ = V.v10_full(x, c, np.zeros_like(c), n_heads=H, chunk_size=512)
    _, _, out, _ = V.fused_clenshaw_ema(V.bf16_round(x), c, n_heads=H, ema_momentum=0.9)
    np.testing.assert_array_equal(full, V.bf16_round(out.astype(np.float32)))
