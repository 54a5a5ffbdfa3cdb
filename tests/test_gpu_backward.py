"""GPU parity of the fused backward (osm_cheby_ema_bwd through the C ABI)
against the float64 backward oracle (itself pinned by torch autograd and
finite differences), plus the autograd wrapper and the drop-in op's
gradients."""
import numpy as np
import pytest
import torch

from helpers import assert_close_fp32, assert_close_grad, inputs, oracle_backward, oracle_forward, to_dev
from oracle import cheby_ema as O
from orthossm_amd import apply_cheby_rkv_v10, cheby_ema, cheby_ema_backward, cheby_ema_forward
from orthossm_amd.synthetic import CONFIGS, make_config_inputs

pytestmark = pytest.mark.gpu


def fwd_bwd(inp, dev, go, gs=None, init=None, nan_policy="zero_z", clamp=True, out_dtype=None):
    """GPU forward (for the saved output) then GPU backward."""
    d = to_dev(inp, dev)
    ini = None if init is None else torch.as_tensor(init, dtype=torch.float32, device=dev)
    out = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], g=d.get("g"), ema_init=ini,
                            nan_policy=nan_policy, clamp=clamp, out_dtype=out_dtype)
    god = torch.as_tensor(go, dtype=torch.float32).to(device=dev, dtype=out.dtype)
    gsd = None if gs is None else torch.as_tensor(gs, dtype=torch.float32, device=dev)
    gx, gc, gi = cheby_ema_backward(d["x"], d["coeffs"], d["damping"], d["lam"], out if clamp else None, god,
                                    g=d.get("g"), grad_state=gsd, nan_policy=nan_policy, clamp=clamp,
                                    need_init=True)
    torch.cuda.synchronize()
    return out, gx, gc, gi


def grads_case(B, S, H, hd, K, seed, dynamic=False):
    inp = inputs(B, S, H, hd, K, seed=seed, dynamic=dynamic)
    r = np.random.default_rng(seed + 1)
    go = r.standard_normal((B, S, H * hd)).astype(np.float32)
    gs = r.standard_normal((B, H * hd)).astype(np.float32)
    init = r.uniform(-0.5, 0.5, size=(B, H * hd)).astype(np.float32)
    return inp, go, gs, init


def check(inp, out, gx, gc, gi, go, gs, init, **kw):
    want = oracle_backward(inp, go, grad_state=gs, ema_init=init, out_saved=out.float().cpu().numpy(), **kw)
    assert_close_grad(gx.float().cpu(), want[0], what="grad_x")
    assert_close_grad(gc.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(gi.cpu(), want[2], what="grad_init")


@pytest.mark.parametrize("B,S,H,hd,K,dyn", [
    (1, 1, 8, 64, 8, False),         # one token
    (2, 191, 8, 64, 8, False),       # one partial (192-token) tile
    (1, 193, 8, 64, 8, False),       # full tile + 1 token
    (3, 1000, 4, 32, 5, False),      # hd < 64, K padded to 8
    (1, 300, 3, 20, 8, False),       # D = 60: partial lane-block
    (2, 777, 2, 12, 3, False),       # D = 24, K <= 4 kernel
    (1, 64 * 128 + 77, 2, 32, 8, False),    # crosses a look-back checkpoint
    (2, 3 * 64 * 128 + 5, 1, 64, 8, True),  # several checkpoints, dynamic lambda
    (3, 5000, 6, 64, 8, True),       # lane-block count not a multiple of 8
    (2, 4096, 8, 64, 8, False),
])
def test_backward_shapes(dev, B, S, H, hd, K, dyn):
    inp, go, gs, init = grads_case(B, S, H, hd, K, seed=B * 100 + S, dynamic=dyn)
    out, gx, gc, gi = fwd_bwd(inp, dev, go, gs, init)
    check(inp, out, gx, gc, gi, go, gs, init)


def test_backward_without_state_gradient(dev):
    inp, go, _, _ = grads_case(2, 2000, 8, 64, 8, seed=5)
    out, gx, gc, gi = fwd_bwd(inp, dev, go)
    check(inp, out, gx, gc, gi, go, None, None)


@pytest.mark.parametrize("nan_policy", ["zero_z", "zero_u"])
def test_backward_special_values(dev, nan_policy):
    inp, go, gs, init = grads_case(1, 600, 2, 32, 8, seed=3)
    x = inp["x"]
    specials = [0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-42, 3e38, -3e38, 1e30, 1e-7, 5e-8,
                -2e-7]
    for i, v in enumerate(specials):
        x[0, 10 * i + 5, (7 * i) % 64] = v
    x[0, 400:420, :] = float("nan")          # a run of NaN rows
    out, gx, gc, gi = fwd_bwd(inp, dev, go, gs, init, nan_policy=nan_policy)
    check(inp, out, gx, gc, gi, go, gs, init, nan_policy=nan_policy)
    gxc = gx.cpu()
    assert torch.all(gxc[0, 400:420] == 0)
    assert gxc[0, 5, 0] == 0 and gxc[0, 45, 28] == 0      # x = 0, x = NaN


def test_backward_clamp_mask(dev):
    # Lanes 0..31 saturate (z = 1 in fp32 from a large c0, ema_init = 1):
    # every output there is within rounding of 1, the mask zeroes their
    # adjoint and the gradient of ema_init.
    inp, go, gs, _ = grads_case(1, 700, 2, 32, 8, seed=9)
    inp["coeffs"][0, 0, 0, :] = 40.0
    init = np.zeros((1, 64), np.float32)
    init[0, :32] = 1.0
    out, gx, gc, gi = fwd_bwd(inp, dev, go, gs, init)
    assert torch.all(out[0, :, :32] >= O.MASK_BOUND)
    check(inp, out, gx, gc, gi, go, gs, init)
    assert torch.all(gi.cpu()[0, :32] == 0) and torch.all(gi.cpu()[0, 32:] != 0)


def test_backward_without_clamp(dev):
    inp, go, gs, init = grads_case(2, 900, 4, 16, 8, seed=4)
    out, gx, gc, gi = fwd_bwd(inp, dev, go, gs, init, clamp=False)
    want = oracle_backward(inp, go, grad_state=gs, ema_init=init, clamp_out=False)
    assert_close_grad(gx.cpu(), want[0], what="grad_x")
    assert_close_grad(gc.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(gi.cpu(), want[2], what="grad_init")


def test_backward_bf16(dev):
    inp, go, gs, init = grads_case(2, 3000, 8, 64, 8, seed=8)
    inp["x"] = inp["x"].to(torch.bfloat16)
    out, gx, gc, gi = fwd_bwd(inp, dev, go, gs, init, out_dtype=torch.bfloat16)
    assert gx.dtype == torch.bfloat16
    # dL/dout is rounded to bf16 (the dtype of out) before the backward.
    go_b = torch.as_tensor(go).to(torch.bfloat16).float().numpy()
    want = oracle_backward(inp, go_b, grad_state=gs, ema_init=init, out_saved=out.float().cpu().numpy())
    assert_close_grad(gx.float().cpu(), want[0], rtol=1e-2, what="grad_x")   # bf16 storage of grad_x
    assert_close_grad(gc.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(gi.cpu(), want[2], what="grad_init")


def test_backward_chunked_carry_matches_monolithic(dev):
    # Forward in chunks with the EMA carry, then the backward chunk by chunk
    # from the end, each chunk's grad_init feeding the previous one's grad_state.
    inp, go, gs, init = grads_case(2, 3000, 4, 64, 8, seed=12, dynamic=True)
    d = to_dev(inp, dev)
    god = torch.as_tensor(go, device=dev)
    st = torch.as_tensor(init, device=dev)
    bounds = [(0, 1000), (1000, 2100), (2100, 3000)]
    outs, inits = [], []
    for t0, t1 in bounds:
        inits.append(st)
        o, st = cheby_ema_forward(d["x"][:, t0:t1], d["coeffs"], d["damping"], d["lam"], g=d["g"][:, t0:t1],
                                  ema_init=st, return_state=True)
        outs.append(o)
    carry = torch.as_tensor(gs, device=dev)
    gxs, gcs = [], torch.zeros_like(d["coeffs"])
    for (t0, t1), o, ini in reversed(list(zip(bounds, outs, inits))):
        gx, gc, carry = cheby_ema_backward(d["x"][:, t0:t1], d["coeffs"], d["damping"], d["lam"], o,
                                           god[:, t0:t1], g=d["g"][:, t0:t1], grad_state=carry, need_init=True)
        gxs.insert(0, gx)
        gcs += gc
    torch.cuda.synchronize()
    out = torch.cat(outs, dim=1)
    want = oracle_backward(inp, go, grad_state=gs, ema_init=init, out_saved=out.cpu().numpy())
    assert_close_grad(torch.cat(gxs, dim=1).cpu(), want[0], what="grad_x")
    assert_close_grad(gcs.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(carry.cpu(), want[2], what="grad_init")


def test_backward_is_deterministic(dev):
    inp, go, gs, init = grads_case(2, 5000, 8, 64, 8, seed=6)
    a = fwd_bwd(inp, dev, go, gs, init)
    b = fwd_bwd(inp, dev, go, gs, init)
    for u, v in zip(a[1:], b[1:]):
        assert torch.equal(u, v)


def test_backward_headline_linearity(dev):
    # BASELINE configs[1] at full size: the backward is linear in
    # (dL/dout, dL/d ema_final), so bwd(g1) + bwd(g2) = bwd(g1 + g2).
    cfg = CONFIGS["headline"]
    inp = make_config_inputs(cfg)
    d = to_dev(inp, dev)
    out = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
    gen = torch.Generator(device=dev).manual_seed(1)
    g1 = torch.randn(out.shape, device=dev, generator=gen)
    g2 = torch.randn(out.shape, device=dev, generator=gen)
    r = [cheby_ema_backward(d["x"], d["coeffs"], d["damping"], d["lam"], out, g) for g in (g1, g2, g1 + g2)]
    torch.cuda.synchronize()
    for i, what in enumerate(("grad_x", "grad_coeffs")):
        s = (r[0][i].double() + r[1][i].double()).cpu().numpy()
        assert_close_grad(r[2][i].cpu(), s, rtol=1e-4, what=what)


def test_autograd_function(dev):
    inp, go, gs, init = grads_case(2, 1500, 4, 32, 8, seed=21, dynamic=True)
    d = to_dev(inp, dev)
    x = d["x"].clone().requires_grad_(True)
    c = d["coeffs"].clone().requires_grad_(True)
    ini = torch.as_tensor(init, device=dev).requires_grad_(True)
    out, fin = cheby_ema(x, c, d["damping"], d["lam"], g=d["g"], ema_init=ini, return_state=True)
    loss = (out * torch.as_tensor(go, device=dev)).sum() + (fin * torch.as_tensor(gs, device=dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    want = oracle_backward(inp, go, grad_state=gs, ema_init=init, out_saved=out.detach().cpu().numpy())
    assert_close_grad(x.grad.cpu(), want[0], what="grad_x")
    assert_close_grad(c.grad.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(ini.grad.cpu(), want[2], what="grad_init")


def test_dropin_fast_path_gradients(dev):
    # apply_cheby_rkv_v10 below seq_threshold: the reference differentiates
    # its fast path with autograd; the oracle restates that gradient (damping
    # 0.98 - 0.06 h/H, scalar momentum on every head, NaN as u = 0).
    B, S, H, hd, K = 2, 300, 4, 16, 4
    gen = torch.Generator().manual_seed(31)
    x = torch.randn(B, S, H * hd, generator=gen)
    x[1, 17, 5] = float("nan")
    c = torch.randn(B, H, K, hd, generator=gen) / torch.arange(1, K + 1).view(1, 1, K, 1)
    go = torch.randn(B, S, H * hd, generator=gen)
    xd = x.to(dev).requires_grad_(True)
    cd = c.to(dev).requires_grad_(True)
    out, c_out, m_out = apply_cheby_rkv_v10(xd, cd, None, n_heads=H, ema_momentum=0.9)
    (out * go.to(dev)).sum().backward()
    torch.cuda.synchronize()
    want = O.backward(x.double().numpy(), c.numpy(), O.v10_damping(H), np.full(H, 0.9), go.double().numpy(),
                      nan_policy="zero_u", out_saved=out.detach().cpu().numpy())
    assert_close_grad(xd.grad.cpu(), want[0], what="grad_x")
    assert_close_grad(cd.grad.cpu(), want[1], what="grad_coeffs")
    assert xd.grad[1, 17, 5].item() == 0.0
