"""Parity with series coefficients far outside the benchmark's
c_k ~ N(0, 1/(k+1)^2): c_k ~ N(0, sigma^2) for every k with sigma = 1, 3
and 10, S >= 4096, for the forward, the TTT gradient, the backward and the
drop-in's fixed-coefficient path, against the float64 oracle at the spec's
tolerances (1e-5 for fp32 outputs, 1e-3 for gradients).

Such coefficients are what any caller may pass (the engine's coefficient
projection is an unbounded learned map).  Their monomial form cancels in
fp32, so a lane-block whose scaled monomial coefficients exceed the kernels'
bound (kMonoBound, 256 in exp2 units) evaluates the Chebyshev form by
Clenshaw instead; the mixed cases put lane-blocks of both forms in one
launch.  An fp32 emulation of the forward on the CPU (u, the coefficient
conversion and the series in fp32, the rest exact) puts the monomial form at
0.99 of the output tolerance for sigma = 10 and at 2.1 for sigma = 30,
against 0.34 and 0.90 for Clenshaw."""
import numpy as np
import pytest
import torch

from helpers import assert_close_fp32, assert_close_grad, inputs, oracle_backward, oracle_forward, oracle_ttt, to_dev
from oracle import cheby_ema as O
from orthossm_amd import cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt
from orthossm_amd import sdpc_kernel as K10

pytestmark = pytest.mark.gpu


def wide_inputs(B, S, H, hd, K, sigma, seed, dynamic=False, mixed=False, dtype=torch.float32):
    """BASELINE-style inputs with c_k ~ N(0, sigma^2) for every k; with
    `mixed`, batch row 0 keeps the benchmark's N(0, 1/(k+1)^2)."""
    inp = inputs(B, S, H, hd, K, seed=seed, dynamic=dynamic, dtype=dtype)
    gen = torch.Generator().manual_seed(seed + 7)
    c = torch.randn(B, H, K, hd, generator=gen) * sigma
    if mixed:
        c[0] = inp["coeffs"][0]
    inp["coeffs"] = c
    return inp


def fp32_lambda(inp, lam_shift=0.004, lam_min=0.9, lam_max=0.9999):
    """The oracle's inputs with the kernel's fp32 lambda: with dynamic lambda
    the kernel forms clamp(fma(lam_shift, g, lam_h)) in fp32, which differs
    from the float64 value by up to ~6e-8; at lambda ~ 0.9995 that changes
    (1 - lambda) by ~1e-4 relative per token and moves the output by up to
    ~3e-6 when |s - z| ~ 1 (wide coefficients drive |z| towards 1).  To check
    the series, tanh and scan to the fp32 tolerance, the oracle is given
    g' = (lambda_fp32 - lambda_h) / lam_shift, which reproduces the kernel's
    per-token lambda exactly, and the fp32 clamp bounds."""
    if inp.get("g") is None:
        return inp, {}
    g = inp["g"].double().numpy()
    lam_h = inp["lam"].numpy().astype(np.float64).reshape(1, 1, -1)
    shift = float(np.float32(lam_shift))
    lo, hi = float(np.float32(lam_min)), float(np.float32(lam_max))
    lam32 = np.clip((lam_h + shift * g).astype(np.float32).astype(np.float64), lo, hi)
    out = dict(inp)
    out["g"] = torch.from_numpy((lam32 - lam_h) / shift)
    return out, {"lam_shift": shift, "lam_min": lo, "lam_max": hi}


@pytest.mark.parametrize("sigma", [1.0, 3.0, 10.0])
@pytest.mark.parametrize("dynamic", [False, True])
def test_forward_wide_coefficients(dev, sigma, dynamic):
    inp = wide_inputs(2, 4096, 8, 64, 8, sigma, seed=300, dynamic=dynamic)
    d = to_dev(inp, dev)
    init = torch.linspace(-0.9, 0.9, 2 * 512, dtype=torch.float32).view(2, 512)
    out, fin = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], g=d.get("g"),
                                 ema_init=init.to(dev), return_state=True)
    ref_in, kw = fp32_lambda(inp)
    want_out, want_fin = oracle_forward(ref_in, ema_init=init.numpy(), **kw)
    assert_close_fp32(out.cpu().numpy(), want_out)
    assert_close_fp32(fin.cpu().numpy(), want_fin, what="ema_final")


@pytest.mark.parametrize("K", [3, 5, 8])
def test_forward_mixed_forms_in_one_launch(dev, K):
    """Row 0 at the benchmark's distribution (monomial form), row 1 at
    sigma = 10 (Chebyshev form); also the one-lane geometry (hd = 62) and
    the 128-token tile (short sequence)."""
    for hd, S in ((64, 6000), (62, 4100), (64, 700)):
        inp = wide_inputs(2, S, 8, hd, K, 10.0, seed=310 + K, mixed=True)
        d = to_dev(inp, dev)
        out = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
        assert_close_fp32(out.cpu().numpy(), oracle_forward(inp)[0], what=f"out hd={hd} S={S}")


def test_forward_bf16_wide(dev):
    inp = wide_inputs(2, 4096, 8, 64, 8, 3.0, seed=320, dtype=torch.bfloat16)
    d = to_dev(inp, dev)
    out = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], out_dtype=torch.bfloat16)
    want = oracle_forward(inp)[0]
    assert np.max(np.abs(out.float().cpu().numpy() - want)) <= 2e-2


@pytest.mark.parametrize("sigma,mixed", [(1.0, False), (3.0, False), (10.0, True)])
@pytest.mark.parametrize("target", ["x", "softsign"])
def test_ttt_wide_coefficients(dev, sigma, mixed, target):
    inp = wide_inputs(2, 4096, 8, 64, 8, sigma, seed=330, mixed=mixed)
    d = to_dev(inp, dev)
    out, grad = cheby_ema_ttt(d["x"], d["coeffs"], d["damping"], d["lam"], target=target)
    G, want_out, _ = oracle_ttt(inp, target=target)
    assert_close_fp32(out.cpu().numpy(), want_out)
    assert_close_grad(grad.cpu().numpy(), G, what="ttt grad")


def test_ttt_wide_dynamic_bf16(dev):
    inp = wide_inputs(2, 4096, 8, 64, 8, 3.0, seed=335, dynamic=True, dtype=torch.bfloat16)
    d = to_dev(inp, dev)
    out, grad = cheby_ema_ttt(d["x"], d["coeffs"], d["damping"], d["lam"], g=d["g"], out_dtype=torch.bfloat16)
    ref_in, kw = fp32_lambda(inp)
    G, want_out, _ = oracle_ttt(ref_in, **kw)
    assert np.max(np.abs(out.float().cpu().numpy() - want_out)) <= 2e-2
    assert_close_grad(grad.cpu().numpy(), G, what="ttt grad")


@pytest.mark.parametrize("sigma,mixed,dynamic", [(1.0, False, False), (3.0, False, True), (10.0, True, False)])
def test_backward_wide_coefficients(dev, sigma, mixed, dynamic):
    B, S, H, hd = 2, 4096, 8, 64
    inp = wide_inputs(B, S, H, hd, 8, sigma, seed=340, mixed=mixed, dynamic=dynamic)
    r = np.random.default_rng(341)
    go = r.standard_normal((B, S, H * hd)).astype(np.float32)
    gs = r.standard_normal((B, H * hd)).astype(np.float32)
    d = to_dev(inp, dev)
    out = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], g=d.get("g"))
    gx, gc, gi = cheby_ema_backward(d["x"], d["coeffs"], d["damping"], d["lam"], out,
                                    torch.as_tensor(go, device=dev), g=d.get("g"),
                                    grad_state=torch.as_tensor(gs, device=dev), need_init=True)
    torch.cuda.synchronize()
    ref_in, kw = fp32_lambda(inp)
    want = oracle_backward(ref_in, go, grad_state=gs, out_saved=out.cpu().numpy(), **kw)
    assert_close_grad(gx.cpu(), want[0], what="grad_x")
    assert_close_grad(gc.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(gi.cpu(), want[2], what="grad_init")


@pytest.mark.parametrize("sigma", [1.0, 3.0])
def test_dropin_fast_path_wide_coefficients(dev, sigma):
    """apply_cheby_rkv_v10 below seq_threshold (the fixed-coefficient path,
    sdpc_kernel.py:1708-1744) with wide coefficients: the output and, through
    autograd, dL/dx and dL/dc against the oracle."""
    b, s, d_, nh, deg = 2, 4096, 256, 4, 8
    hd = d_ // nh
    gen = torch.Generator().manual_seed(350)
    x = torch.randn(b, s, d_, generator=gen)
    coeffs = torch.randn(b, nh, deg, hd, generator=gen) * sigma
    go = torch.randn(b, s, d_, generator=gen)
    xg = x.to(dev).requires_grad_(True)
    cg = coeffs.to(dev).requires_grad_(True)
    out, cn, _ = K10.apply_cheby_rkv_v10(xg, cg, torch.zeros(b, nh, deg, hd, device=dev), n_heads=nh,
                                         ema_momentum=0.95, seq_threshold=s + 1)
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    damp = K10.v10_damping(nh).numpy()
    lam = np.full(nh, 0.95, dtype=np.float32)
    xd, cd = x.double().numpy(), coeffs.double().numpy()
    want = O.forward(xd, cd, damp, lam, nan_policy="zero_u")[0]
    assert_close_fp32(out.detach().cpu().numpy(), want)
    gx, gc, _ = O.backward(xd, cd, damp, lam, go.double().numpy(), nan_policy="zero_u",
                           out_saved=out.detach().cpu().numpy())
    assert_close_grad(xg.grad.cpu().numpy(), gx, what="dL/dx")
    assert_close_grad(cg.grad.cpu().numpy(), gc, what="dL/dc")
