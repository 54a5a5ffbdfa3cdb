"""GPU parity of the fixed-coefficient LUT/Clenshaw forward
(osm_cheby_ema_lut_fwd through the C ABI), which replaces the reference's
_fused_clenshaw_ema_kernel (sdpc_kernel.py:988-1209), against the float64
restatement oracle/v10_full.py:fused_clenshaw_ema; and the kernel object's
launch syntax as precision_tests.py:61-73 uses it."""
import math

import numpy as np
import pytest
import torch

from oracle import v10_full as V
from orthossm_amd import apply_cheby_rkv_v10
from orthossm_amd.ops import cheby_ema_lut_forward
from orthossm_amd.sdpc_kernel import LUT_TABLE_SIZE, _fused_clenshaw_ema_kernel, get_chebyshev_lut

pytestmark = pytest.mark.gpu


def case(B, S, H, hd, K, seed, x_scale=1.0, init_scale=None):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, H * hd, generator=gen) * x_scale
    c = torch.randn(B, H, K, hd, generator=gen) / torch.arange(1, K + 1).view(1, 1, K, 1)
    init = None if init_scale is None else torch.randn(B, H * hd, generator=gen) * init_scale
    return x, c, init


def f32(v):
    """A momentum as the kernel receives it (a float32 argument, as Triton
    passes a Python float to _fused_clenshaw_ema_kernel)."""
    return float(np.float32(v))


def rel(got, want):
    got = got.detach().double().cpu().numpy()
    return np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)


@pytest.mark.parametrize("B,S,H,hd,K,use_lut,block_s,mu,init_scale,xdt", [
    (2, 300, 4, 16, 8, True, 128, 0.9, None, torch.float32),       # one partial block past 256
    (2, 1000, 4, 16, 4, True, 128, 0.9, 0.5, torch.float32),       # four blocks, ema_init
    (1, 777, 8, 20, 3, False, 64, 0.97, 0.8, torch.float32),       # hd off 8-lane groups, 4-term Clenshaw
    (2, 512, 2, 32, 6, False, 32, 0.95, None, torch.float32),      # 8-term Clenshaw above four terms
    (2, 700, 4, 16, 8, True, 16, 0.999, 0.3, torch.float32),       # 16-token tiles: 16-lane workgroups
    (3, 257, 2, 8, 5, True, 256, 0.9, None, torch.bfloat16),       # bf16 x, a 1-token last block
    (1, 5, 1, 8, 8, True, 128, 0.9, 0.1, torch.float32),           # S < one run group
    (8, 300, 8, 128, 8, True, 128, 0.9, None, torch.float32),      # >= 512 16-lane workgroups
])
def test_lut_forward_matches_oracle(dev, B, S, H, hd, K, use_lut, block_s, mu, init_scale, xdt):
    x, c, init = case(B, S, H, hd, K, seed=S + K + hd, init_scale=init_scale)
    xd = x.to(xdt)
    out, xn, ty, fin = cheby_ema_lut_forward(xd.to(dev), c.to(dev), n_heads=H, ema_momentum=mu,
                                             ema_init=None if init is None else init.to(dev), use_lut=use_lut,
                                             clamp_tile=block_s)
    torch.cuda.synchronize()
    wxn, wty, wout, wfin = V.fused_clenshaw_ema(xd.float().numpy(), c.double().numpy(), n_heads=H,
                                                ema_momentum=f32(mu), ema_init=None if init is None else init.numpy(),
                                                use_lut=use_lut, block_s=block_s)
    assert rel(xn, wxn) <= 1e-6
    assert rel(ty, wty) <= 1e-5
    assert rel(out, wout) <= 1e-5
    assert rel(fin, wfin) <= 1e-5


@pytest.mark.parametrize("block_s", [32, 128, 256, 512])
def test_carry_clamp_binds_at_tile_boundaries(dev, block_s):
    # mu near 1 and |ema_init| up to 5: the carried state is clamped at every
    # tile boundary, which moves every later output
    B, S, H, hd, K = 2, 1100, 2, 16, 8
    x, c, init = case(B, S, H, hd, K, seed=block_s, init_scale=3.0)
    mu = 0.9995
    out, xn, ty, fin = cheby_ema_lut_forward(x.to(dev), c.to(dev), n_heads=H, ema_momentum=mu,
                                             ema_init=init.to(dev), clamp_tile=block_s)
    torch.cuda.synchronize()
    _, _, wout, wfin = V.fused_clenshaw_ema(x.numpy(), c.double().numpy(), n_heads=H, ema_momentum=f32(mu),
                                            ema_init=init.numpy(), block_s=block_s)
    _, _, free, _ = V.fused_clenshaw_ema(x.numpy(), c.double().numpy(), n_heads=H, ema_momentum=f32(mu),
                                         ema_init=init.numpy(), block_s=4096)
    assert np.abs(wout - free).max() > 1e-2          # the case exercises the clamp
    assert rel(out, wout) <= 1e-5
    assert rel(fin, wfin) <= 1e-5


def test_special_values_empty_and_optional_outputs(dev):
    B, S, H, hd, K = 2, 600, 4, 16, 8
    x, c, init = case(B, S, H, hd, K, seed=5, init_scale=0.5)
    vals = [float("nan"), 0.0, float("inf"), -float("inf"), -0.0, 3e38, 1e-30, -3e38]
    for i, v in enumerate(vals):
        x[:, 37 * i + 1, ::3] = v
    out, xn, ty, fin = cheby_ema_lut_forward(x.to(dev), c.to(dev), n_heads=H, ema_init=init.to(dev))
    torch.cuda.synchronize()
    wxn, wty, wout, wfin = V.fused_clenshaw_ema(x.numpy(), c.double().numpy(), n_heads=H, ema_momentum=f32(0.9),
                                                ema_init=init.numpy())
    assert torch.isfinite(out).all() and torch.isfinite(xn).all() and torch.isfinite(ty).all()
    assert rel(xn, wxn) <= 1e-6 and rel(ty, wty) <= 1e-5 and rel(out, wout) <= 1e-5 and rel(fin, wfin) <= 1e-5
    # without x_norm / tanh_y buffers the same out and final state
    out2, xn2, ty2, fin2 = cheby_ema_lut_forward(x.to(dev), c.to(dev), n_heads=H, ema_init=init.to(dev),
                                                 want_x_norm=False, want_tanh_y=False)
    assert xn2 is None and ty2 is None
    assert torch.equal(out2, out) and torch.equal(fin2, fin)
    # S = 0: the state passes through unclamped; B = 0: nothing to do
    init5 = init.to(dev) * 10
    o0, _, _, f0 = cheby_ema_lut_forward(torch.zeros(B, 0, H * hd, device=dev), c.to(dev), n_heads=H,
                                         ema_init=init5)
    torch.cuda.synchronize()
    assert o0.shape == (B, 0, H * hd) and torch.equal(f0, init5)
    cheby_ema_lut_forward(torch.zeros(0, 10, H * hd, device=dev), c[:0].to(dev), n_heads=H)


def test_reference_launch_syntax_matches_precision_tests_p1(dev):
    # precision_tests.py:32-89 as written: the full path on one chunk against
    # the fused kernel launched with Triton's grid syntax
    torch.manual_seed(42)
    B, S, D, nH, deg = 2, 256, 64, 8, 4
    x = torch.randn(B, S, D, device=dev)
    coeffs0 = torch.randn(B, nH, deg, D // nH, device=dev)
    mom0 = torch.zeros(B, nH, deg, D // nH, device=dev)
    out_mega, coeffs_mega, _ = apply_cheby_rkv_v10(x, coeffs0.clone(), mom0.clone(), n_heads=nH, use_lut=True,
                                                   seq_threshold=0, chunk_size=512)
    x_bf16 = x.contiguous().to(torch.bfloat16)
    coeff_c = coeffs0.contiguous()
    lut_c = get_chebyshev_lut(dev).contiguous()
    x_norm_ref = torch.empty(B, S, D, device=dev, dtype=torch.float32)
    tanh_y_ref = torch.empty(B, S, D, device=dev, dtype=torch.float32)
    out_ref = torch.empty(B, S, D, device=dev, dtype=torch.float32)
    ema_init = torch.zeros(B, D, device=dev, dtype=torch.float32)
    ema_final = torch.empty(B, D, device=dev, dtype=torch.float32)
    BLOCK_HD = min(32, 1 << (D // nH - 1).bit_length())
    n_hd_blocks = math.ceil((D // nH) / BLOCK_HD)
    grid_f = (B * nH * n_hd_blocks,)
    _fused_clenshaw_ema_kernel[grid_f](
        x_bf16, coeff_c, lut_c,
        x_norm_ref, tanh_y_ref, out_ref,
        ema_init, ema_final,
        S, D, D // nH, nH, deg, LUT_TABLE_SIZE, 0.9,
        x_bf16.stride(0), x_bf16.stride(1), x_bf16.stride(2),
        coeff_c.stride(0), coeff_c.stride(1), coeff_c.stride(2), coeff_c.stride(3),
        lut_c.stride(0), lut_c.stride(1),
        x_norm_ref.stride(0), x_norm_ref.stride(1), x_norm_ref.stride(2),
        tanh_y_ref.stride(0), tanh_y_ref.stride(1), tanh_y_ref.stride(2),
        out_ref.stride(0), out_ref.stride(1), out_ref.stride(2),
        ema_init.stride(0), ema_init.stride(1),
        BLOCK_HD=BLOCK_HD, BLOCK_S=128, USE_LUT=True,
    )
    torch.cuda.synchronize()
    # P1's own checks
    cos = torch.nn.functional.cosine_similarity(out_mega.flatten(), out_ref.flatten(), dim=0).item()
    norm_err = (out_mega - out_ref).abs().mean().item() / (out_ref.abs().mean().item() + 1e-9)
    assert cos >= 0.99 and norm_err <= 0.01
    assert not torch.allclose(coeffs_mega, coeffs0, atol=1e-6)
    # and the stronger check: the full path's output is this output rounded to bf16
    assert (out_mega != out_ref.to(torch.bfloat16).float()).float().mean().item() <= 1e-3
    wxn, wty, wout, wfin = V.fused_clenshaw_ema(x_bf16.float().cpu().numpy(), coeffs0.double().cpu().numpy(),
                                                n_heads=nH, ema_momentum=f32(0.9))
    assert rel(out_ref, wout) <= 1e-5 and rel(x_norm_ref, wxn) <= 1e-6 and rel(tanh_y_ref, wty) <= 1e-5
    assert rel(ema_final, wfin) <= 1e-5


def test_launcher_writes_strided_outputs_and_checks_its_arguments(dev):
    B, S, D, nH, deg = 2, 300, 32, 4, 8
    x = torch.randn(B, S, D, device=dev)
    c = torch.randn(B, nH, deg, D // nH, device=dev) / 3
    lut = get_chebyshev_lut(dev)
    # x_norm laid out [B, D, S] (lane stride S): written through a copy
    xn = torch.empty(B, D, S, device=dev).transpose(1, 2)
    ty = torch.empty(B, S, D, device=dev)
    out = torch.empty(B, S, D, device=dev)
    init = torch.randn(B, D, device=dev) * 0.3
    fin = torch.empty(B, D, device=dev)

    def args(**over):
        a = [x, c, lut, xn, ty, out, init, fin, S, D, D // nH, nH, deg, LUT_TABLE_SIZE, 0.95,
             *x.stride(), *c.stride(), *lut.stride(), *xn.stride(), *ty.stride(), *out.stride(), *init.stride()]
        kw = dict(BLOCK_HD=8, BLOCK_S=64, USE_LUT=True)
        kw.update(over)
        return a, kw

    grid = (B * nH * 1,)
    a, kw = args()
    _fused_clenshaw_ema_kernel[grid](*a, **kw)
    torch.cuda.synchronize()
    wxn, wty, wout, wfin = V.fused_clenshaw_ema(x.cpu().numpy(), c.double().cpu().numpy(), n_heads=nH,
                                                ema_momentum=f32(0.95), ema_init=init.cpu().numpy(), block_s=64)
    assert rel(xn, wxn) <= 1e-6 and rel(ty, wty) <= 1e-5 and rel(out, wout) <= 1e-5 and rel(fin, wfin) <= 1e-5
    # a grid given as a function of the launch arguments, as Triton allows
    _fused_clenshaw_ema_kernel[lambda meta: (B * meta["n_heads"],)](*a, **kw)
    with pytest.raises(ValueError):
        _fused_clenshaw_ema_kernel[(B * nH * 2,)](*a, **kw)        # not the kernel's grid
    with pytest.raises(TypeError):
        _fused_clenshaw_ema_kernel[grid](*a)                        # BLOCK_HD etc. missing
    bad = list(a)
    bad[16] = 1                                                     # stride_xs not x's
    with pytest.raises(NotImplementedError):
        _fused_clenshaw_ema_kernel[grid](*bad, **kw)
