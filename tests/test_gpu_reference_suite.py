"""The path-level checks of the reference's own suites, run against this
drop-in.  From test_v10.py: T2 (shapes), T3 (fast path below
seq_threshold leaves the coefficients alone), T4 and T5 (the full path above it updates them),
T6 (Lion keeps two state tensors), T7 (LUT and 4-term Clenshaw series
agree, cosine > 0.99), T8 (gradients through the op finite and non-zero),
T9 (B=4 finite), T13 and T14 (degree 4 and 8 run; timings printed), with
the coefficients drawn by init_chebyshev_coefficients as there
(test_v10.py:63-241, 330-385).  Its model-level checks (T1, T10-T12,
T15-T17: imports, the layer bus, the full model, the local refiner) are
outside this path.  From precision_tests.py: P1 (a one-chunk call equals
the plain series + EMA), P2 (bf16-rounded coefficients move the output by
<= 1.5%), P4 (one-chunk gradients finite) and P5 (<= 3 ms per forward).
From gradient_checker.py: its three levels on its own case.
Where it is cheap the outputs are also compared with the CPU oracle
(oracle/v10_full.py)."""
import time

import numpy as np
import pytest
import torch

from helpers import compare_v10
from oracle import v10_full as V
from orthossm_amd import sdpc_kernel as K10

pytestmark = pytest.mark.gpu

B, S, D, NH = 2, 512, 64, 8
HD = D // NH
DEG = 4   # the reference's V10 default


def _coef(dev, b=B, deg=DEG, seed=0):
    torch.manual_seed(seed)
    return K10.init_chebyshev_coefficients(b, NH, deg, HD, dev)


def test_t2_forward_shapes(dev):
    x = torch.randn(B, S, D, generator=torch.Generator().manual_seed(2)).to(dev)
    coef = _coef(dev)
    mom = torch.zeros_like(coef)
    out, cn, mn = K10.apply_cheby_rkv_v10(x, coef, mom, n_heads=NH, ema_momentum=0.9)
    assert out.shape == x.shape and cn.shape == coef.shape and mn.shape == mom.shape


def test_t3_fast_path_keeps_coefficients(dev):
    x = torch.randn(2, 128, D, generator=torch.Generator().manual_seed(3)).to(dev)
    coef = _coef(dev, seed=3)
    mom = torch.zeros_like(coef)
    out, cn, mn = K10.apply_cheby_rkv_v10(x, coef, mom, n_heads=NH, ema_momentum=0.9, seq_threshold=384)
    torch.cuda.synchronize()
    assert out.shape == x.shape
    assert torch.allclose(cn, coef, atol=1e-6)


@pytest.mark.parametrize("seq", [512, 1024])
def test_t4_t5_full_path_updates_coefficients(dev, seq):
    x = torch.randn(2, seq, D, generator=torch.Generator().manual_seed(seq)).to(dev)
    coef = _coef(dev, seed=seq)
    mom = torch.zeros_like(coef)
    out, cn, mn = K10.apply_cheby_rkv_v10(x, coef, mom, n_heads=NH, ema_momentum=0.9, seq_threshold=384)
    torch.cuda.synchronize()
    assert out.shape == x.shape
    assert not torch.allclose(cn, coef, atol=1e-6)
    # and the same values as the CPU restatement
    compare_v10(out, cn, mn, V.v10_full(x.cpu().numpy(), coef.double().cpu().numpy(),
                                        mom.double().cpu().numpy(), n_heads=NH, ema_momentum=0.9))


def test_t6_lion_state_is_two_tensors(dev):
    x = torch.randn(2, 600, D, generator=torch.Generator().manual_seed(6)).to(dev)
    coef = _coef(dev, seed=6)
    res = K10.apply_cheby_rkv_v10(x, coef, torch.zeros_like(coef), n_heads=NH, seq_threshold=0)
    assert len(res) == 3                      # out, coefficients, momentum: no second moment
    state = res[1].numel() + res[2].numel()
    assert (1 - state / (3 * coef.numel())) * 100 > 30


def test_t7_lut_and_clenshaw_agree(dev):
    x = torch.randn(2, 512, D, generator=torch.Generator().manual_seed(7)).to(dev)
    coef = _coef(dev, seed=7)
    outs = []
    for lut in (True, False):
        out, cn, mn = K10.apply_cheby_rkv_v10(x, coef.clone(), torch.zeros_like(coef), n_heads=NH, ema_momentum=0.9,
                                              use_lut=lut, seq_threshold=0)
        torch.cuda.synchronize()
        compare_v10(out, cn, mn, V.v10_full(x.cpu().numpy(), coef.double().cpu().numpy(),
                                            np.zeros(coef.shape), n_heads=NH, ema_momentum=0.9, use_lut=lut))
        outs.append(out)
    cos = torch.nn.functional.cosine_similarity(outs[0].reshape(1, -1), outs[1].reshape(1, -1)).item()
    print(f"T7 cosine {cos:.5f}", flush=True)
    assert cos > 0.99


def test_t8_gradients_finite_and_nonzero(dev):
    x = torch.randn(2, 512, D, generator=torch.Generator().manual_seed(8)).to(dev).requires_grad_(True)
    coef = _coef(dev, seed=8)
    out, _, _ = K10.apply_cheby_rkv_v10(x, coef, torch.zeros_like(coef), n_heads=NH, ema_momentum=0.9,
                                        seq_threshold=0)
    out.sum().backward()
    torch.cuda.synchronize()
    assert x.grad is not None and torch.isfinite(x.grad).all() and x.grad.abs().max() > 0


def test_t9_multi_batch_finite(dev):
    x = torch.randn(4, 512, D, generator=torch.Generator().manual_seed(9)).to(dev)
    coef = _coef(dev, b=4, seed=9)
    out, _, _ = K10.apply_cheby_rkv_v10(x, coef, torch.zeros_like(coef), n_heads=NH, ema_momentum=0.9,
                                        seq_threshold=0)
    assert torch.isfinite(out).all()


def test_t13_t14_degree_four_and_eight_timed(dev):
    x = torch.randn(2, 1024, D, generator=torch.Generator().manual_seed(13)).to(dev)
    for deg in (4, 8):
        coef = _coef(dev, deg=deg, seed=deg)
        mom = torch.zeros_like(coef)
        for _ in range(3):
            K10.apply_cheby_rkv_v10(x, coef.clone(), mom.clone(), n_heads=NH, ema_momentum=0.9, seq_threshold=0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(20):
            out, _, _ = K10.apply_cheby_rkv_v10(x, coef.clone(), mom.clone(), n_heads=NH, ema_momentum=0.9,
                                                seq_threshold=0)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / 20 * 1e3
        print(f"degree {deg}: {ms:.3f} ms per call (B=2 S=1024 D=64, host included)", flush=True)
        assert torch.isfinite(out).all()


# The path-level checks of the reference's precision_tests.py (P1, P2, P4,
# P5; precision_tests.py:29-199).  P3 tests the local refiner (outside this
# path).

def test_p1_single_chunk_equals_the_plain_series_and_ema(dev):
    """One chunk (S=256 < chunk_size=512): out is the LUT series + EMA with
    the starting coefficients (the reference compares its megakernel with
    its pure Clenshaw+EMA kernel: cosine >= 0.99, mean error <= 1% of the
    mean magnitude), and Lion has updated the coefficients."""
    b, s, nh, deg = 2, 256, 8, 4
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(b, s, D, generator=gen).to(dev)
    c0 = torch.randn(b, nh, deg, D // nh, generator=gen).to(dev)
    m0 = torch.zeros_like(c0)
    out, cn, _ = K10.apply_cheby_rkv_v10(x, c0.clone(), m0.clone(), n_heads=nh, use_lut=True, seq_threshold=0,
                                         chunk_size=512)
    torch.cuda.synchronize()
    # plain series + EMA, no Lion: the oracle's chunk with a zero learning rate
    want, _, _ = V.v10_full(x.cpu().numpy(), c0.double().cpu().numpy(), np.zeros(c0.shape), n_heads=nh,
                            base_lr=0.0, chunk_size=512)
    o = out.float().cpu().flatten()
    w = torch.from_numpy(want).float().flatten()
    cos = torch.nn.functional.cosine_similarity(o, w, dim=0).item()
    norm_err = (o - w).abs().mean().item() / (w.abs().mean().item() + 1e-9)
    print(f"P1 cosine {cos:.6f}, normalised error {norm_err:.2e}", flush=True)
    assert cos >= 0.99 and norm_err <= 0.01
    assert not torch.allclose(cn.float(), c0.float(), atol=1e-6)


def test_p2_bf16_rounded_coefficients(dev):
    b, nh, deg = 2, 8, 4
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(b, 256, D, generator=gen).to(dev)
    c = torch.randn(b, nh, deg, D // nh, generator=gen).to(dev)
    m = torch.zeros_like(c)
    out_f, *_ = K10.apply_cheby_rkv_v10(x, c.clone(), m.clone(), n_heads=nh, seq_threshold=0)
    out_b, *_ = K10.apply_cheby_rkv_v10(x, c.to(torch.bfloat16).float(), m.clone(), n_heads=nh, seq_threshold=0)
    rel = (out_f - out_b).abs().max().item() / (out_f.abs().max().item() + 1e-9)
    print(f"P2 relative error {rel:.2e}", flush=True)
    assert rel <= 0.015


def test_p4_single_chunk_gradients_finite(dev):
    b, nh, deg = 2, 8, 4
    gen = torch.Generator().manual_seed(14)
    xg = torch.randn(b, 256, D, generator=gen).to(dev).requires_grad_(True)
    cg = torch.randn(b, nh, deg, D // nh, generator=gen).to(dev).requires_grad_(True)
    out, _, _ = K10.apply_cheby_rkv_v10(xg, cg, torch.zeros(b, nh, deg, D // nh, device=dev), n_heads=nh,
                                        seq_threshold=0, chunk_size=512)
    out.sum().backward()
    torch.cuda.synchronize()
    assert xg.grad is not None and torch.isfinite(xg.grad).all()
    assert cg.grad is not None and torch.isfinite(cg.grad).all()


def test_p5_latency_within_the_reference_bound(dev):
    x = torch.randn(2, 1024, 128, generator=torch.Generator().manual_seed(15)).to(dev)
    c = torch.randn(2, 8, 4, 16, generator=torch.Generator().manual_seed(16)).to(dev)
    m = torch.zeros_like(c)
    for _ in range(5):
        K10.apply_cheby_rkv_v10(x, c.clone(), m.clone(), n_heads=8, seq_threshold=0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        K10.apply_cheby_rkv_v10(x, c.clone(), m.clone(), n_heads=8, seq_threshold=0)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / 20 * 1e3
    print(f"P5 {ms:.3f} ms per forward (B=2 S=1024 D=128, host included)", flush=True)
    assert ms <= 3.0


def test_gradient_checker_three_levels(dev):
    """The reference's gradient checker (gradient_checker.py:284-330, 154-228)
    on its own case, B=1 S=16 D=16 NH=2 deg=4, coefficients N(0,1)*0.05, one
    upstream gradient, through apply_cheby_rkv_core (S < seq_threshold: the
    fast path).  L1: the forward matches the reference path (here the
    float64 oracle, fp32 tolerance); L2: dL/dx and dL/dc from autograd
    through the drop-in match the reference's analytic gradients (1e-3);
    L3: the reference's analytic gradient matches central differences with
    the checker's epsilons (median over them) with cosine > 0.9999 and
    relative error < 0.005, as it requires (in float64 here)."""
    from oracle import cheby_ema as O
    from orthossm_amd.sdpc_kernel import v10_damping

    torch.manual_seed(42)
    b, s, d, nh, deg = 1, 16, 16, 2, 4
    hd = d // nh
    x = torch.randn(b, s, d)
    coeffs = torch.randn(b, nh, deg, hd) * 0.05
    grad_out = torch.randn(b, s, d)
    xg = x.to(dev).requires_grad_(True)
    cg = coeffs.to(dev).requires_grad_(True)
    out, *_ = K10.apply_cheby_rkv_core(xg, cg, torch.zeros(b, nh, deg, hd, device=dev), n_heads=nh, ema_momentum=0.9)
    out.backward(grad_out.to(dev))
    torch.cuda.synchronize()

    damp = v10_damping(nh).numpy()
    lam = np.full(nh, 0.9, dtype=np.float32)
    xd, cd, god = x.double().numpy(), coeffs.double().numpy(), grad_out.double().numpy()
    fwd = lambda xx, cc: O.forward(xx, cc, damp, lam, nan_policy="zero_u")[0]      # noqa: E731
    want = fwd(xd, cd)
    # L1
    assert np.max(np.abs(out.detach().cpu().numpy() - want)) <= 1e-5 * np.max(np.abs(want)) + 1e-6
    # L2
    gx, gc, _ = O.backward(xd, cd, damp, lam, god, nan_policy="zero_u", out_saved=want)
    for got, w, what in ((xg.grad, gx, "dL/dx"), (cg.grad, gc, "dL/dc")):
        g = got.cpu().double().numpy()
        assert np.max(np.abs(g - w)) <= 1e-3 * np.max(np.abs(w)), what
    # L3 (dL/dx; up to 64 elements, the checker's max_fd_elements)
    xf = xd.reshape(-1)
    fd = []
    for eps in (0.03, 0.05, 0.08, 0.12, 0.2):
        col = []
        for i in range(min(xf.size, 64)):
            h = eps * max(abs(xf[i]), 1.0) * 1e-3
            xp, xm = xf.copy(), xf.copy()
            xp[i] += h
            xm[i] -= h
            col.append(((fwd(xp.reshape(xd.shape), cd) - fwd(xm.reshape(xd.shape), cd)) * god).sum() / (2 * h))
        fd.append(col)
    fd = np.median(np.array(fd), axis=0)
    an = gx.reshape(-1)[:fd.size]
    cos = float(an @ fd / (np.linalg.norm(an) * np.linalg.norm(fd)))
    rel = float(np.linalg.norm(an - fd) / (np.linalg.norm(an) + 1e-8))
    print(f"L3 cosine {cos:.8f}, relative error {rel:.2e}", flush=True)
    assert cos > 0.9999 and rel < 0.005
