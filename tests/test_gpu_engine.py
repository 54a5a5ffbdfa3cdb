"""The engine's Cheby-RKV call sites on the GPU (orthossm_amd/engine.py):
each route matches the CPU oracle fed with the engine's host steps restated
in float64 (input norm, coefficient init, complexity gate, mu schedule;
sdpc_engine.py:163-225, 239-333), each route gives exactly what a direct call
of the drop-in with the engine's arguments gives (mu passed as a float), the
device-resident mu equals the float one bit for bit, a forward makes no host
synchronisation, the EMA carry continues one scan across calls, and
activation checkpointing leaves the gradients unchanged."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close_fp32, compare_v10
from oracle import cheby_ema as O
from oracle import v10_full as V

from orthossm_amd import apply_cheby_rkv_v10
from orthossm_amd import engine as E
from orthossm_amd.ops import cheby_ema_forward, head_momentum, v10_chunked_ttt
from orthossm_amd.sdpc_kernel import v10_damping

pytestmark = pytest.mark.gpu

D, H, K = 128, 4, 4


def make(dev, seed=0, **kw):
    torch.manual_seed(seed)
    m = E.ChebyContextPath(D, n_cheby_heads=H, max_degree=K, **kw).to(dev)
    # non-zero coefficient head so the coefficients depend on the input
    torch.nn.init.normal_(m.coeff_init_proj[-1].weight, std=0.5)
    return m


def direct(m, x, state, mu, tier):
    """What the reference engine passes to apply_cheby_rkv_v10 for this call."""
    xn = m.input_norm(x)
    xm = xn.mean(dim=1)
    if state is None:
        c = m.coeff_init_proj(xm).view(x.shape[0], H, K, D // H) * m.coeff_spectral_scale
        mom = torch.zeros_like(c)
    else:
        c, mom = state
    gate = m.complexity_gate(xm)
    thr = E.FAST_PATH_THRESHOLD if tier == "fast" else 0
    return apply_cheby_rkv_v10(xn, c, mom, n_heads=H, base_lr=0.005, ema_momentum=mu, gate_global=gate,
                               dynamic_lambda=gate, use_lut=True, seq_threshold=thr)


def host_steps_f64(m, x, tokens_before):
    """The engine's steps before its apply_cheby_rkv_v10 call, in float64 on
    the CPU from the module's weights (sdpc_engine.py:163-209): RMSNorm with
    eps = fp32 machine epsilon, mean over tokens, coefficients
    coeff_init_proj(mean) * 0.1/(k+1), gate sigmoid(MLP(mean)), and mu =
    0.7 + 0.5 (ema_base - 0.7)(1 + cos(pi p)), p = min(tokens/1e8, 1) after
    adding this call's tokens.  Returns (x_normed, coeffs, gate [B], mu)."""
    W = {k: v.detach().cpu().double() for k, v in m.state_dict().items()}
    xd = x.detach().cpu().double()
    B, S, _ = xd.shape
    eps = torch.finfo(torch.float32).eps
    xn = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * W["input_norm.weight"]
    xm = xn.mean(dim=1)

    def mlp(prefix, v):
        hid = F.silu(v @ W[f"{prefix}.0.weight"].T + W[f"{prefix}.0.bias"])
        return hid @ W[f"{prefix}.2.weight"].T + W[f"{prefix}.2.bias"]

    k = torch.arange(K, dtype=torch.float64)
    c = mlp("coeff_init_proj", xm).view(B, H, K, D // H) * (0.1 / (k + 1.0)).view(1, 1, K, 1)
    gate = torch.sigmoid(mlp("complexity_gate.net", xm)).reshape(B)
    p = min((tokens_before + S) / 1e8, 1.0)
    mu = 0.7 + 0.5 * (float(W["ema_base"]) - 0.7) * (1.0 + math.cos(math.pi * p))
    return xn, c, gate, mu


@pytest.mark.parametrize("S,tier,tokens_before", [(200, "fast", 0), (300, "fast", 37_000_000),
                                                  (600, "hybrid", 0), (1100, "full", 80_000_000)])
def test_routes_match_oracle(dev, S, tier, tokens_before):
    m = make(dev, seed=S)
    with torch.no_grad():
        m.input_norm.weight.uniform_(0.5, 1.5, generator=torch.Generator(device=dev).manual_seed(S))
        m.total_tokens_seen.fill_(tokens_before)
    x = torch.randn(2, S, D, generator=torch.Generator().manual_seed(S + 1)) * 1.7
    with torch.no_grad():
        r = m(x.to(dev))
    torch.cuda.synchronize()
    assert r.route == tier
    xn, c, gate, mu = host_steps_f64(m, x, tokens_before)
    assert abs(float(r.ema_momentum) - mu) <= 1e-7
    assert_close_fp32(r.x_normed.cpu(), xn.numpy(), what="x_normed")
    assert_close_fp32(r.gate.reshape(-1).cpu(), gate.numpy(), what="gate")
    if tier == "fast":
        # the fixed-coefficient path: V10 damping 0.98 - 0.06 h/H, mu on every
        # head, NaN as u = 0 (sdpc_kernel.py:1708-1744)
        damping = 0.98 - 0.06 * np.arange(H) / H
        want, _ = O.forward(xn.numpy(), c.numpy(), damping, np.full(H, mu), nan_policy="zero_u")
        assert_close_fp32(r.out.cpu(), want)
        assert_close_fp32(r.state[0].cpu(), c.numpy(), what="coeffs")
        assert torch.count_nonzero(r.state[1]) == 0
    else:
        # the full path with the gate as gate_global and dynamic_lambda
        want = V.v10_full(xn.float().numpy(), c.numpy(), np.zeros(c.shape), n_heads=H, base_lr=0.005,
                          ema_momentum=mu, gate_global=gate.numpy(), dynamic_lambda=gate.numpy(), use_lut=True,
                          chunk_size=256)
        compare_v10(r.out, r.state[0], r.state[1], want)


@pytest.mark.parametrize("S,tier", [(200, "fast"), (600, "hybrid"), (1100, "full")])
def test_routes_match_direct_drop_in_call(dev, S, tier):
    m = make(dev)
    x = torch.randn(2, S, D, generator=torch.Generator().manual_seed(S)).to(dev)
    with torch.no_grad():
        r = m(x)
        assert r.route == tier
        mu = float(r.ema_momentum)                  # the float the reference would pass
        out, c, mom = direct(m, x, None, mu, tier)
    assert torch.equal(r.out, out)
    assert torch.equal(r.state[0], c) and torch.equal(r.state[1], mom)
    if tier != "fast":
        assert not torch.equal(c, r.state[0] * 0)   # Lion moved the coefficients


def test_device_momentum_equals_float_momentum(dev):
    x = torch.randn(2, 700, D, generator=torch.Generator().manual_seed(1)).to(dev)
    c = (torch.randn(2, H, 8, D // H) * 0.3).to(dev)
    mom = (torch.randn(2, H, 8, D // H) * 0.01).to(dev)
    mu_t = torch.tensor(0.8123, device=dev)
    a = v10_chunked_ttt(x, c, mom, n_heads=H, ema_momentum=mu_t)
    b = v10_chunked_ttt(x, c, mom, n_heads=H, ema_momentum=float(mu_t))
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    lam_t = head_momentum(mu_t, H, dev)
    assert torch.equal(lam_t, torch.full((H,), float(mu_t), device=dev))
    f1 = apply_cheby_rkv_v10(x[:, :300], c, mom, n_heads=H, ema_momentum=mu_t)[0]
    f2 = apply_cheby_rkv_v10(x[:, :300], c, mom, n_heads=H, ema_momentum=float(mu_t))[0]
    assert torch.equal(f1, f2)


def test_forward_makes_no_host_sync(dev):
    m = make(dev)
    xs = [torch.randn(1, S, D, device=dev) for S in (100, 500, 1100)]
    with torch.no_grad():
        for x in xs:                     # first calls upload the kernels' constant tables
            m(x)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        probe_raised = False
        try:
            torch.ones(1, device=dev).item()
        except RuntimeError:
            probe_raised = True
        if not probe_raised:
            pytest.skip("this torch build does not report synchronising calls")
        with torch.no_grad():
            for x in xs:
                r = m(x)
        # the reference reads mu back with .item() here (sdpc_engine.py:209)
        with pytest.raises(RuntimeError):
            r.ema_momentum.item()
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()


def test_ema_carry_continues_one_scan(dev):
    m = make(dev, carry_ema=True)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(2, 250, D, generator=gen).to(dev)
    c = (torch.randn(2, H, K, D // H, generator=gen) * 0.3).to(dev)
    state = E.ChebyState(c, torch.zeros_like(c), None)
    with torch.no_grad():
        r1 = m(x[:, :100], state)
        r2 = m(x[:, 100:], r1.state)
        assert r1.route == r2.route == "fast" and r2.state.ema.shape == (2, D)
        assert torch.equal(r1.ema_momentum, r2.ema_momentum)   # 100 vs 250 tokens: mu is 0.9 in fp32
        xn = m.input_norm(x)
        lam = head_momentum(r1.ema_momentum, H, dev)
        whole, fin = cheby_ema_forward(xn, c, v10_damping(H, dev), lam, out_dtype=torch.float32,
                                       nan_policy="zero_u", return_state=True)
    got = torch.cat([r1.out, r2.out], dim=1)
    torch.testing.assert_close(got, whole, rtol=0, atol=2e-6)
    torch.testing.assert_close(r2.state.ema, fin, rtol=0, atol=2e-6)
    # without the carry the second call restarts from zero, as the reference does
    m0 = make(dev)
    with torch.no_grad():
        r0 = m0(x[:, 100:], (c, torch.zeros_like(c)))
    assert not torch.allclose(r0.out, r2.out)
    # a full-path call ends the carry (its EMA restarts at every chunk)
    with torch.no_grad():
        r3 = m(torch.randn(2, 1100, D, device=dev), r2.state)
    assert r3.state.ema is None


@pytest.mark.parametrize("S", [150, 1100])
def test_checkpointing_keeps_gradients(dev, S):
    grads = []
    for ckpt in (False, True):
        m = make(dev, gradient_ckpt=ckpt).train()
        x = torch.randn(2, S, D, generator=torch.Generator().manual_seed(7)).to(dev).requires_grad_(True)
        go = torch.randn(2, S, D, generator=torch.Generator().manual_seed(8)).to(dev)
        r = m(x)
        (r.out * go).sum().backward()
        torch.cuda.synchronize()
        grads.append((x.grad.clone(), m.input_norm.weight.grad.clone(),
                      None if S > 256 else m.coeff_init_proj[-1].weight.grad.clone()))
    for a, b in zip(*grads):
        if a is None:
            continue
        assert torch.isfinite(a).all() and a.abs().max() > 0
        assert torch.equal(a, b)
