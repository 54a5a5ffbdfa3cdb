"""Seeded random configurations of the forward, the TTT gradient, the
backward and the full path (online TTT with Lion) against the CPU oracle: head counts and sizes (any hd, D not
a multiple of 64), sequence lengths from 1 token, 1..16 Chebyshev terms
(1..8 for the TTT), random per-head lambda and damping, dynamic lambda, fp32
and bf16 input and output, an initial EMA state, strided (non-contiguous)
x, both NaN policies, the output clamp on and off, and a few special values
(NaN, +-Inf, huge, subnormal) planted in x; for the full path also chunk
sizes, the LUT and Clenshaw series, the complexity gate, dynamic lambda and
the Lion hyperparameters; the full path's gradients; and the engine's
call sites.  Each case is drawn from its own seed, so a failure names a
reproducible configuration."""
import numpy as np
import pytest
import torch

from helpers import assert_close_fp32, assert_close_grad, compare_v10, oracle_backward, oracle_forward, oracle_ttt
from oracle import v10_full as V
from orthossm_amd import cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt
from orthossm_amd.ops import v10_chunked_ttt
from orthossm_amd.synthetic import make_inputs

pytestmark = pytest.mark.gpu

HD_CHOICES = (1, 2, 3, 4, 5, 7, 8, 12, 16, 20, 24, 31, 32, 33, 48, 63, 64, 65, 80, 96, 128)
SPECIALS = (float("nan"), float("inf"), float("-inf"), 3e38, -1e30, 1e-42, -0.0)
N_CASES = 40


def draw(seed, op):
    """One configuration: a dict of shape, flags and CPU inputs."""
    r = np.random.default_rng(1000 * {"fwd": 1, "ttt": 2, "bwd": 3}[op] + seed)
    H = int(r.integers(1, 9))
    hd = int(r.choice(HD_CHOICES))
    B = int(r.integers(1, 4))
    D = H * hd
    s_max = max(1, min(4000, int(3e6 // (B * D))))
    S = int(np.exp(r.uniform(0.0, np.log(s_max)))) if r.random() > 0.1 else int(r.integers(1, 4))
    K = int(r.integers(1, 9 if op == "ttt" else 17))
    dyn = bool(r.random() < 0.3)
    x_bf16 = bool(r.random() < 0.3)
    out_bf16 = bool(r.random() < 0.3) and op != "bwd"
    inp = make_inputs(B, S, D, H, K, seed=seed, dynamic=dyn, dtype=torch.bfloat16 if x_bf16 else torch.float32)
    inp["lam"] = torch.tensor(r.uniform(0.5, 0.9995, size=H), dtype=torch.float32)
    inp["damping"] = torch.tensor(r.uniform(0.3, 1.2, size=H), dtype=torch.float32)
    specials = bool(r.random() < 0.25)
    if specials:
        x = inp["x"]
        for v in SPECIALS:
            x[int(r.integers(0, B)), int(r.integers(0, S)), int(r.integers(0, D))] = v
    cfg = {
        "B": B, "S": S, "H": H, "hd": hd, "K": K, "dyn": dyn, "x_bf16": x_bf16, "out_bf16": out_bf16,
        "init": r.uniform(-0.9, 0.9, size=(B, D)).astype(np.float32) if r.random() < 0.5 else None,
        "strided": bool(r.random() < 0.25),
        "clamp": bool(r.random() < 0.8) or op == "ttt",   # the TTT loss always clamps (as its oracle)
        "nan_policy": "zero_u" if r.random() < 0.3 else "zero_z",
        "target": "softsign" if r.random() < 0.3 else "x",
        "specials": specials,
    }
    return cfg, inp, r


def device_x(x_cpu, dev, strided, r):
    """x on the device, as a view into wider rows when ``strided``."""
    if not strided:
        return x_cpu.to(dev)
    B, S, D = x_cpu.shape
    off = int(r.integers(1, 4))
    wide = torch.zeros(B, S, D + off + 2, dtype=x_cpu.dtype)
    wide[:, :, off:off + D] = x_cpu
    return wide.to(dev)[:, :, off:off + D]


def common(cfg, inp, dev, r):
    x = device_x(inp["x"], dev, cfg["strided"], r)
    g = None if inp["g"] is None else inp["g"].to(dev)
    init = None if cfg["init"] is None else torch.from_numpy(cfg["init"]).to(dev)
    return x, inp["coeffs"].to(dev), inp["damping"].to(dev), inp["lam"].to(dev), g, init


def check_out(out, want, cfg, what="out"):
    atol = 1e-6 if cfg["K"] <= 8 else 4e-6
    if out.dtype == torch.bfloat16:
        got = out.float().cpu().numpy().astype(np.float64)
        both = np.isnan(got) & np.isnan(want)
        assert not (np.isnan(got) ^ np.isnan(want)).any(), f"{what}: NaN pattern differs"
        err = np.abs(np.where(both, 0, got) - np.where(both, 0, want))
        assert err.max(initial=0.0) <= 2e-2 and np.all(err <= 2.0 ** -8 * np.abs(np.where(both, 0, want)) + atol), \
            f"{what}: bf16 error {err.max(initial=0.0):.3e}"
    else:
        assert_close_fp32(out.cpu(), want, atol=atol, what=what)


def describe(cfg):
    return ", ".join(f"{k}={v}" for k, v in cfg.items() if k != "init") + f", init={cfg['init'] is not None}"


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_forward(dev, seed):
    cfg, inp, r = draw(seed, "fwd")
    print(describe(cfg), flush=True)
    x, c, damp, lam, g, init = common(cfg, inp, dev, r)
    out, fin = cheby_ema_forward(x, c, damp, lam, g=g, ema_init=init, clamp=cfg["clamp"],
                                 nan_policy=cfg["nan_policy"], return_state=True,
                                 out_dtype=torch.bfloat16 if cfg["out_bf16"] else torch.float32)
    torch.cuda.synchronize()
    want, wfin = oracle_forward(inp, ema_init=cfg["init"], clamp_out=cfg["clamp"], nan_policy=cfg["nan_policy"])
    check_out(out, want, cfg)
    check_out(fin, wfin, cfg, what="ema_final")


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_ttt(dev, seed):
    cfg, inp, r = draw(seed, "ttt")
    print(describe(cfg), flush=True)
    x, c, damp, lam, g, init = common(cfg, inp, dev, r)
    out, grad, fin = cheby_ema_ttt(x, c, damp, lam, g=g, ema_init=init, clamp=cfg["clamp"],
                                   nan_policy=cfg["nan_policy"], target=cfg["target"], return_state=True,
                                   out_dtype=torch.bfloat16 if cfg["out_bf16"] else torch.float32)
    torch.cuda.synchronize()
    G, want, wfin = oracle_ttt(inp, ema_init=cfg["init"], target=cfg["target"], nan_policy=cfg["nan_policy"])
    check_out(out, want, cfg)
    check_out(fin, wfin, cfg, what="ema_final")
    # A special value in x is also a target of the loss: the gradient of its
    # lane is then NaN or Inf (or, for 3e38, past the fp32 range in the sums);
    # those lanes are compared by finiteness only, the others by value.
    B, S, D = inp["x"].shape
    xf = inp["x"].float()
    lane_ok = (torch.isfinite(xf) & (xf.abs() < 1e6)).all(dim=1).numpy()           # [B, D]
    ok = np.broadcast_to(lane_ok.reshape(B, cfg["H"], 1, cfg["hd"]), G.shape)
    g = grad.cpu().numpy()
    assert np.isfinite(g[ok]).all() and (~np.isfinite(G[ok])).sum() == 0
    assert ok.any() or not lane_ok.any()
    assert_close_grad(np.where(ok, g, 0.0), np.where(ok, G, 0.0), what="grad")
    assert (np.isfinite(g) | ~ok).all()


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_backward(dev, seed):
    cfg, inp, r = draw(seed, "bwd")
    print(describe(cfg), flush=True)
    x, c, damp, lam, g, init = common(cfg, inp, dev, r)
    B, S, D = inp["x"].shape
    go = r.standard_normal((B, S, D)).astype(np.float32)
    gs = r.standard_normal((B, D)).astype(np.float32) if r.random() < 0.5 else None
    out = cheby_ema_forward(x, c, damp, lam, g=g, ema_init=init, clamp=cfg["clamp"], nan_policy=cfg["nan_policy"])
    gx, gc, gi = cheby_ema_backward(x, c, damp, lam, out if cfg["clamp"] else None,
                                    torch.from_numpy(go).to(device=dev, dtype=out.dtype), g=g,
                                    grad_state=None if gs is None else torch.from_numpy(gs).to(dev),
                                    clamp=cfg["clamp"], nan_policy=cfg["nan_policy"], need_init=True)
    torch.cuda.synchronize()
    want = oracle_backward(inp, go.astype(np.float64) if out.dtype == torch.float32 else
                           torch.from_numpy(go).to(out.dtype).double().numpy(),
                           grad_state=gs, ema_init=cfg["init"], clamp_out=cfg["clamp"], nan_policy=cfg["nan_policy"],
                           out_saved=out.float().cpu().numpy() if cfg["clamp"] else None)
    # grad_x is stored in x's dtype: bf16 storage rounds it to 2^-8 relative
    assert_close_grad(gx.float().cpu(), want[0], rtol=1e-2 if cfg["x_bf16"] else 1e-3, what="grad_x")
    assert_close_grad(gc.cpu(), want[1], what="grad_coeffs")
    assert_close_grad(gi.cpu(), want[2], what="grad_init")


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_full_path(dev, seed):
    r = np.random.default_rng(4000 + seed)
    H = int(r.choice((1, 2, 4, 8)))
    hd = int(r.choice((4, 8, 12, 16, 20, 32, 48, 64, 128)))
    B = int(r.integers(1, 4))
    K = int(r.integers(1, 9))
    chunk = int(r.choice((64, 100, 128, 256, 300, 512)))
    S = int(r.integers(1, 1500)) if r.random() > 0.1 else int(r.integers(1, 4))
    use_lut = bool(r.random() < 0.7)
    kw = dict(n_heads=H, chunk_size=chunk, use_lut=use_lut, base_lr=float(r.uniform(0.001, 0.02)),
              ema_momentum=float(r.uniform(0.7, 0.99)), beta1=float(r.uniform(0.8, 0.95)),
              beta2=float(r.uniform(0.9, 0.999)))
    wd = float(r.uniform(0.0, 0.05))
    gate = torch.tensor(r.uniform(0.2, 2.5, size=B), dtype=torch.float32) if r.random() < 0.4 else None
    dyn = torch.tensor(r.uniform(0.05, 0.95, size=B), dtype=torch.float32) if r.random() < 0.4 else None
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, H * hd, generator=gen)
    c = torch.randn(B, H, K, hd, generator=gen) / torch.arange(1, K + 1).view(1, 1, K, 1)
    m = torch.randn(B, H, K, hd, generator=gen) * float(r.choice((0.0, 0.01, 0.1)))
    x_in = x.to(torch.bfloat16) if r.random() < 0.3 else x
    print(f"B={B} S={S} H={H} hd={hd} K={K} chunk={chunk} lut={use_lut} gate={gate is not None} "
          f"dyn={dyn is not None} x={x_in.dtype} {kw}", flush=True)
    out, cn, mn = v10_chunked_ttt(x_in.to(dev), c.to(dev), m.to(dev), weight_decay=wd,
                                  gate_global=None if gate is None else gate.to(dev),
                                  dynamic_lambda=None if dyn is None else dyn.to(dev), **kw)
    torch.cuda.synchronize()
    want = V.v10_full(x_in.float().numpy(), c.double().numpy(), m.double().numpy(), wd=wd,
                      gate_global=None if gate is None else gate.numpy(),
                      dynamic_lambda=None if dyn is None else dyn.numpy(), **kw)
    compare_v10(out, cn, mn, want)


@pytest.mark.parametrize("seed", range(16))
def test_random_full_path_gradients(dev, seed):
    """dL/dx (and dL/dc for one-chunk sequences, the only case where the
    chunk loop lets it flow) of the differentiable drop-in against the
    oracle's backward of the full path on the GPU forward's saved tensors."""
    from orthossm_amd import apply_cheby_rkv_v10

    r = np.random.default_rng(5000 + seed)
    H = int(r.choice((1, 2, 4, 8)))
    hd = int(r.choice((4, 8, 16, 24, 32, 64)))
    B = int(r.integers(1, 4))
    K = int(r.integers(1, 9))
    chunk = int(r.choice((64, 100, 256, 512)))
    S = int(r.integers(2, 1200))
    print(f"B={B} S={S} H={H} hd={hd} K={K} chunk={chunk}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, H * hd, generator=gen)
    c = torch.randn(B, H, K, hd, generator=gen) / torch.arange(1, K + 1).view(1, 1, K, 1)
    m = torch.randn(B, H, K, hd, generator=gen) * 0.01
    go = torch.randn(B, S, H * hd, generator=gen)
    xd = x.to(dev).requires_grad_(True)
    cd = c.to(dev).requires_grad_(True)
    out, _, _ = apply_cheby_rkv_v10(xd, cd, m.to(dev), n_heads=H, chunk_size=chunk, seq_threshold=0)
    (out * go.to(dev)).sum().backward()
    torch.cuda.synchronize()
    _, _, _, z, hist = v10_chunked_ttt(x.to(dev), c.to(dev), m.to(dev), n_heads=H, chunk_size=chunk,
                                       save_for_backward=True)
    wx, wc = V.v10_backward(x.numpy(), out.detach().cpu().numpy(), z.float().cpu().numpy(), hist.cpu().numpy(),
                            go.numpy(), n_heads=H, ema_momentum=0.9, chunk=chunk)
    assert_close_grad(xd.grad.cpu(), wx, what="grad_x")
    if S <= chunk:
        assert_close_grad(cd.grad.cpu(), wc, what="grad_coeffs")
    else:
        assert cd.grad is None


def _engine_host_steps_f64(m, x, tokens_before, state):
    """The engine's steps before its call into the op, in float64 on the CPU
    from the module's weights (sdpc_engine.py:163-209): RMSNorm (eps = fp32
    machine epsilon), token mean, coefficients coeff_init_proj(mean) *
    0.1/(k+1) (or the given state), gate sigmoid(MLP(mean)), mu from the
    token count after this call.  Returns (x_normed, coeffs, momentum, gate,
    mu)."""
    import math

    import torch.nn.functional as F
    W = {k: v.detach().cpu().double() for k, v in m.state_dict().items()}
    xd = x.detach().cpu().double()
    b, s, d = xd.shape
    h, k_terms, hd = m.n_cheby_heads, m.max_degree, m.head_dim
    xn = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps) * W["input_norm.weight"]
    xm = xn.mean(dim=1)

    def mlp(prefix, v):
        hid = F.silu(v @ W[f"{prefix}.0.weight"].T + W[f"{prefix}.0.bias"])
        return hid @ W[f"{prefix}.2.weight"].T + W[f"{prefix}.2.bias"]

    if state is None:
        kk = torch.arange(k_terms, dtype=torch.float64)
        c = mlp("coeff_init_proj", xm).view(b, h, k_terms, hd) * (0.1 / (kk + 1.0)).view(1, 1, k_terms, 1)
        mom = torch.zeros_like(c)
    else:
        c, mom = state[0].cpu().double(), state[1].cpu().double()
    gate = torch.sigmoid(mlp("complexity_gate.net", xm)).reshape(b)
    p = min((tokens_before + s) / 1e8, 1.0)
    mu = 0.7 + 0.5 * (float(W["ema_base"]) - 0.7) * (1.0 + math.cos(math.pi * p))
    return xn, c, mom, gate, mu


@pytest.mark.parametrize("seed", range(12))
def test_random_engine_routes(dev, seed):
    """The engine's call sites with random widths, heads, degrees, chunk
    sizes, lengths (all three routes), token counts and incoming state,
    against the oracle fed with the engine's host steps."""
    from oracle import cheby_ema as O
    from orthossm_amd import engine as E

    r = np.random.default_rng(6000 + seed)
    d = int(r.choice((64, 128, 256)))
    h = int(r.choice([v for v in (2, 4, 8) if d % v == 0]))
    k_terms = int(r.choice((4, 8)))
    chunk = int(r.choice((128, 256)))
    s = int(r.integers(16, 1500))
    b = int(r.integers(1, 4))
    tokens_before = int(r.integers(0, 100_000_000))
    torch.manual_seed(seed)
    m = E.ChebyContextPath(d, n_cheby_heads=h, max_degree=k_terms, chunk_size=chunk).to(dev)
    torch.nn.init.normal_(m.coeff_init_proj[-1].weight, std=0.5)
    with torch.no_grad():
        m.input_norm.weight.uniform_(0.5, 1.5, generator=torch.Generator(device=dev).manual_seed(seed))
        m.total_tokens_seen.fill_(tokens_before)
    state = None
    if r.random() < 0.4:
        g = torch.Generator().manual_seed(seed + 1)
        state = ((torch.randn(b, h, k_terms, d // h, generator=g) * 0.1).to(dev),
                 (torch.randn(b, h, k_terms, d // h, generator=g) * 0.01).to(dev))
    x = torch.randn(b, s, d, generator=torch.Generator().manual_seed(seed + 2)) * 1.5
    print(f"d={d} h={h} K={k_terms} chunk={chunk} B={b} S={s} tokens_before={tokens_before} "
          f"state={state is not None}", flush=True)
    with torch.no_grad():
        res = m(x.to(dev), state)
    torch.cuda.synchronize()
    assert res.route == E.route(s)
    xn, c, mom, gate, mu = _engine_host_steps_f64(m, x, tokens_before, state)
    assert abs(float(res.ema_momentum) - mu) <= 1e-7
    assert_close_fp32(res.x_normed.cpu(), xn.numpy(), what="x_normed")
    if res.route == "fast":
        damping = 0.98 - 0.06 * np.arange(h) / h
        want, _ = O.forward(xn.numpy(), c.numpy(), damping, np.full(h, mu), nan_policy="zero_u")
        assert_close_fp32(res.out.cpu(), want)
        assert_close_fp32(res.state[0].cpu(), c.numpy(), what="coeffs")
    else:
        want = V.v10_full(xn.float().numpy(), c.numpy(), mom.numpy(), n_heads=h, base_lr=0.005, ema_momentum=mu,
                          gate_global=gate.numpy(), dynamic_lambda=gate.numpy(), use_lut=True, chunk_size=chunk)
        compare_v10(res.out, res.state[0], res.state[1], want)
