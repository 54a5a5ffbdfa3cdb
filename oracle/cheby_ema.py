"""float64 CPU restatement of the Cheby-RKV forward and its TTT gradient.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package.

Operator (indices b<B, t<S, h<H, j<hd, lane d = h*hd + j, D = H*hd)::

    u[b,t,d] = x / (1 + |x|)                         softsign
    p[b,t,d] = sum_{k<K} c[b,h,k,j] T_k(u)           Clenshaw
    z[b,t,d] = tanh(delta_h * p)                     damping + tanh
    s[b,t,d] = lam[b,t,h] s[b,t-1,d] + (1-lam) z     EMA, s[b,-1,d] = ema_init
    out      = clamp(s, -1, 1)

Reference lines each piece restates (paths relative to the reference root):

* softsign            sdpc_kernel.py:1722-1725 (PyTorch path) and
                      sdpc_kernel.py:2020-2027 (Triton path).  The spec form
                      x/(1+|x|) is used; +-Inf maps to +-1.
* NaN policy          sdpc_kernel.py:2086: a NaN input gives z = 0
                      (nan_policy "zero_z"); or, as the PyTorch fast path
                      sdpc_kernel.py:1725, u = 0 (nan_policy "zero_u").
* Clenshaw            sdpc_kernel.py:1139-1156 (b_k = c_k + 2u b_{k+1} - b_{k+2},
                      p = c_0 + u b_1 - b_2), equal to the basis+einsum form of
                      sdpc_kernel.py:1728-1731, 1751-1776.
* damping, tanh       sdpc_kernel.py:1734-1739 (damping is a parameter here).
* EMA + carry         sdpc_kernel.py:422-433, 440-539 (affine combine, carry
                      in/out [B,D]); per-head lambda as in
                      chimera_experiment/chimera_v2_ssm.py:86-101.
* output clamp        sdpc_kernel.py:2104-2106 (applied to the output; the
                      carried state is the unclamped recurrence).
* dynamic lambda      clamp form of sdpc_kernel.py:2188-2194, applied per
                      token and head: lam = clamp(lam_h + shift*g, lo, hi).
* TTT gradient        loss = mean((out[:, t] - y[:, t+1])^2) over t < S-1 with
                      y = x (or softsign(x)); G_k = dL/dc_k / (k+1)^2
                      (README.md:96-97).  Adjoint chain as in
                      sdpc_kernel.py:681-777 (reverse EMA) and 784-915
                      (dL/dy through tanh, Chebyshev basis).
* backward            dL/dx, dL/dc, dL/d ema_init of (out, ema_final): the
                      fast path's autograd (sdpc_kernel.py:1708-1744) with the
                      EMA's masked reverse scan (1677-1701, 682-777).

Pinning (tests/test_oracle.py): Clenshaw against numpy.polynomial.chebyshev
and cos(k*theta); softsign/tanh special values; the EMA against
scipy.signal.lfilter and closed forms; dynamic lambda against a brute-force
loop; the TTT adjoint gradient and the backward against torch autograd and
central finite differences (the backward's clamp mask against autograd of a
state-clamped forward); the whole forward against the reference-form
restatement in ``oracle/reference_form.py``.
"""
from __future__ import annotations

import numpy as np

# Per-head EMA decay and damping of the BASELINE spec (README.md:90-94 lists
# the lambdas; damping 0.9**h is the spec's choice).
BASELINE_LAMBDA = (0.9995, 0.9995, 0.997, 0.997, 0.995, 0.995, 0.95, 0.95)


def baseline_lambda(H: int) -> np.ndarray:
    lam = list(BASELINE_LAMBDA[:H]) + [BASELINE_LAMBDA[-1]] * max(0, H - len(BASELINE_LAMBDA))
    return np.asarray(lam, dtype=np.float64)


def baseline_damping(H: int) -> np.ndarray:
    return 0.9 ** np.arange(H, dtype=np.float64)


def v10_damping(H: int) -> np.ndarray:
    """Damping hard-coded in the reference kernels: 0.98 - 0.06*h/H
    (sdpc_kernel.py:1734-1736, 2080)."""
    return 0.98 - 0.06 * np.arange(H, dtype=np.float64) / H


def softsign(x: np.ndarray) -> np.ndarray:
    """u = x/(1+|x|) in float64; +-Inf -> +-1; NaN stays NaN (the caller
    applies the NaN policy on z).  sdpc_kernel.py:1722-1725."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        u = x / (1.0 + np.abs(x))
    return np.where(np.isinf(x), np.sign(x), u)


def clenshaw(c: np.ndarray, u: np.ndarray) -> np.ndarray:
    """p = sum_k c[..., k] T_k(u) by the Clenshaw recurrence
    (sdpc_kernel.py:1139-1156).  ``c`` has the coefficient axis last and
    broadcasts against ``u``."""
    c = np.asarray(c, dtype=np.float64)
    u = np.asarray(u, dtype=np.float64)
    K = c.shape[-1]
    b1 = np.zeros(np.broadcast_shapes(c.shape[:-1], u.shape))
    b2 = np.zeros_like(b1)
    for k in range(K - 1, 0, -1):
        b1, b2 = c[..., k] + 2.0 * u * b1 - b2, b1
    return c[..., 0] + u * b1 - b2


def chebyshev_basis(u: np.ndarray, K: int) -> np.ndarray:
    """T_0..T_{K-1} at u, stacked on a new last axis (sdpc_kernel.py:1751-1776)."""
    u = np.asarray(u, dtype=np.float64)
    T = [np.ones_like(u)]
    if K > 1:
        T.append(u)
    for _ in range(2, K):
        T.append(2.0 * u * T[-1] - T[-2])
    return np.stack(T[:K], axis=-1)


def lane_coeffs(coeffs: np.ndarray) -> np.ndarray:
    """[B,H,K,hd] -> [B,D,K] with lane d = h*hd + j."""
    c = np.asarray(coeffs, dtype=np.float64)
    B, H, K, hd = c.shape
    return c.transpose(0, 1, 3, 2).reshape(B, H * hd, K)


def lambda_field(lam, B, S, H, g=None, lam_shift=0.004, lam_min=0.9, lam_max=0.9999):
    """Per-token, per-head decay [B,S,H].  Static: lam_h broadcast.  Dynamic:
    clamp(lam_h + lam_shift*g[b,t,h], lam_min, lam_max) (clamp form of
    sdpc_kernel.py:2188-2194).  ``g`` may be [S,H] or [B,S,H]."""
    lam = np.asarray(lam, dtype=np.float64).reshape(1, 1, H)
    if g is None:
        return np.broadcast_to(lam, (B, S, H))
    g = np.asarray(g, dtype=np.float64)
    g = np.broadcast_to(g, (B, S, H))
    # The kernel evaluates lam_h + shift*g in fp32 arithmetic on fp32 inputs;
    # the oracle keeps float64, which differs by < 1e-7 relative.
    return np.clip(lam + lam_shift * g, lam_min, lam_max)


def forward(x, coeffs, damping, lam, *, g=None, lam_shift=0.004, lam_min=0.9,
            lam_max=0.9999, ema_init=None, clamp_out=True, return_parts=False, nan_policy="zero_z"):
    """Cheby-RKV forward in float64.

    x [B,S,D]; coeffs [B,H,K,hd]; damping [H]; lam [H]; g optional [S,H] or
    [B,S,H]; ema_init optional [B,D] (or [B,H,hd]).
    Returns (out [B,S,D], ema_final [B,D]) and, with return_parts, a dict of
    the intermediates u, z, s (unclamped) and lam_t [B,S,H].
    """
    x = np.asarray(x, dtype=np.float64)
    B, S, D = x.shape
    Bc, H, K, hd = np.shape(coeffs)
    assert Bc == B and H * hd == D, "coeffs shape does not match x"
    u = softsign(x)
    nan = np.isnan(x)
    uc = np.where(nan, 0.0, u)
    cl = lane_coeffs(coeffs)                                   # [B,D,K]
    p = clenshaw(cl[:, None, :, :], uc)                        # [B,S,D]
    delta = np.repeat(np.asarray(damping, dtype=np.float64), hd)  # [D]
    z = np.tanh(delta * p)
    if nan_policy == "zero_z":
        z = np.where(nan, 0.0, z)                              # sdpc_kernel.py:2086
    else:
        assert nan_policy == "zero_u"                          # sdpc_kernel.py:1725
    lam_t = lambda_field(lam, B, S, H, g, lam_shift, lam_min, lam_max)
    lam_d = np.repeat(lam_t, hd, axis=2)                       # [B,S,D]
    s = np.empty_like(z)
    state = np.zeros((B, D)) if ema_init is None else np.asarray(ema_init, np.float64).reshape(B, D).copy()
    for t in range(S):
        lt = lam_d[:, t, :]
        state = lt * state + (1.0 - lt) * z[:, t, :]
        s[:, t, :] = state
    out = np.clip(s, -1.0, 1.0) if clamp_out else s
    if return_parts:
        return out, state, {"u": u, "z": z, "s": s, "lam_t": lam_t}
    return out, state


def forward_chunked(x, coeffs, damping, lam, chunk, **kw):
    """Chunked streaming with EMA carry: each chunk starts from the previous
    chunk's ema_final.  Must equal ``forward`` on the whole sequence."""
    x = np.asarray(x, dtype=np.float64)
    g = kw.pop("g", None)
    ema = kw.pop("ema_init", None)
    outs = []
    for t0 in range(0, x.shape[1], chunk):
        gc = None
        if g is not None:
            gg = np.asarray(g)
            gc = gg[t0:t0 + chunk] if gg.ndim == 2 else gg[:, t0:t0 + chunk]
        o, ema = forward(x[:, t0:t0 + chunk], coeffs, damping, lam, g=gc, ema_init=ema, **kw)
        outs.append(o)
    return np.concatenate(outs, axis=1), ema


def ttt_grad(x, coeffs, damping, lam, *, g=None, lam_shift=0.004, lam_min=0.9,
             lam_max=0.9999, ema_init=None, target="x", nan_policy="zero_z"):
    """TTT coefficient gradient by the closed-form adjoint, float64.

    loss = mean over (b, t<S-1, d) of (clamp(s[b,t,d]) - y[b,t+1,d])^2 with
    y = x (target 'x') or y = softsign(x) (target 'softsign').
    Returns (G [B,H,K,hd] = dloss/dc_k / (k+1)^2, out, ema_final).

    Adjoint (sdpc_kernel.py:681-777, 784-915, with per-token lambda):
        gL[t]  = 2/N (out[t] - y[t+1]) * [|s[t]| <= 1]   (t < S-1), 0 at S-1
        a[t]   = gL[t] + lam[t+1] a[t+1]
        dp[t]  = (1 - lam[t]) a[t] (1 - z[t]^2) delta_h
        dc_k   = sum_t dp[t] T_k(u[t])      (u = 0 where x is NaN; dp = 0 there
                                              under nan_policy "zero_z")
    """
    x = np.asarray(x, dtype=np.float64)
    B, S, D = x.shape
    _, H, K, hd = np.shape(coeffs)
    out, ema_final, parts = forward(x, coeffs, damping, lam, g=g, lam_shift=lam_shift,
                                    lam_min=lam_min, lam_max=lam_max, ema_init=ema_init,
                                    return_parts=True, nan_policy=nan_policy)
    s, z, lam_t = parts["s"], parts["z"], parts["lam_t"]
    nan = np.isnan(x)
    u = np.where(nan, 0.0, parts["u"])
    if S < 2:
        return np.zeros((B, H, K, hd)), out, ema_final
    y = x if target == "x" else np.where(nan, np.nan, parts["u"])
    N = B * (S - 1) * D
    gL = np.zeros_like(s)
    gL[:, :-1, :] = (2.0 / N) * (out[:, :-1, :] - y[:, 1:, :]) * (np.abs(s[:, :-1, :]) <= 1.0)
    lam_d = np.repeat(lam_t, hd, axis=2)
    a = np.empty_like(s)
    acc = np.zeros((B, D))
    for t in range(S - 1, -1, -1):
        nxt = lam_d[:, t + 1, :] if t + 1 < S else 0.0
        acc = gL[:, t, :] + nxt * acc
        a[:, t, :] = acc
    delta = np.repeat(np.asarray(damping, dtype=np.float64), hd)
    dp = (1.0 - lam_d) * a * (1.0 - z * z) * delta
    if nan_policy == "zero_z":
        dp = np.where(nan, 0.0, dp)
    Tk = chebyshev_basis(u, K)                                 # [B,S,D,K]
    dc = np.einsum("bsd,bsdk->bdk", dp, Tk)                    # [B,D,K]
    G = dc.reshape(B, H, hd, K).transpose(0, 1, 3, 2)
    G = G / (np.arange(1, K + 1, dtype=np.float64) ** 2).reshape(1, 1, K, 1)
    return G, out, ema_final


SOFTSIGN_GRAD_MIN = float(np.float32(1e-7))
# The reference compares |out| with 1 - 1e-6 on fp32 tensors, so the bound
# is that value rounded to fp32.
MASK_BOUND = float(np.float32(1.0 - 1e-6))


def backward(x, coeffs, damping, lam, grad_out, *, g=None, lam_shift=0.004, lam_min=0.9,
             lam_max=0.9999, ema_init=None, grad_state=None, clamp_out=True, nan_policy="zero_z",
             out_saved=None):
    """Gradients of (out, ema_final) w.r.t. x, coeffs and ema_init, float64,
    given dL/dout = grad_out [B,S,D] and optionally dL/d ema_final =
    grad_state [B,D]; lambda (static or dynamic) and damping are constants.
    Returns (grad_x [B,S,D], grad_coeffs [B,H,K,hd], grad_init [B,D]).

    Restates the reference's gradient of the fast path (sdpc_kernel.py:
    1708-1744 differentiated by autograd, with the EMA's own backward
    _EMAFastPathFn.backward 1677-1701 and its reverse scan 682-777)::

        a[t]  = m[t] (dL/dout[t] + lam[t+1] a[t+1]),   a[S] = dL/d ema_final, lam[S] = 1
        m[t]  = [|out[t]| < 1 - 1e-6 (fp32)]   (out = the saved forward output; m = 1 without the clamp)
        dp[t] = (1 - lam[t]) a[t] delta (1 - z[t]^2)
        dL/dc_k       = sum_t dp[t] T_k(u[t])
        dL/dx[t]      = dp[t] p'(u[t]) / (1 + |x[t]|)^2,  p'(u) = sum_k k c_k U_{k-1}(u)
        dL/d ema_init = lam[0] a[0]

    The mask gates the carried adjoint as well as dL/dout[t] (the reference
    scan's affine step is a = m*mu, b = m*g, sdpc_kernel.py:696-702).
    dL/dx is 0 where |x| < 1e-7 (fp32) and at NaN: the reference clamps |x|
    at 1e-7 before the softsign (sdpc_kernel.py:1723) and masks NaN with
    torch.where (1725), so autograd passes no gradient there.  Under
    nan_policy 'zero_z' a NaN token's z is the constant 0 and adds nothing to
    dL/dc; under 'zero_u' it adds dp T_k(0).  The reference's full-path
    backward runs the same adjoint with the static momentum even when the
    forward used dynamic lambda (sdpc_kernel.py:2443); here lam[t] is the one
    the forward used."""
    x = np.asarray(x, dtype=np.float64)
    B, S, D = x.shape
    _, H, K, hd = np.shape(coeffs)
    out, fin, parts = forward(x, coeffs, damping, lam, g=g, lam_shift=lam_shift, lam_min=lam_min,
                              lam_max=lam_max, ema_init=ema_init, clamp_out=clamp_out, return_parts=True,
                              nan_policy=nan_policy)
    z, lam_t = parts["z"], parts["lam_t"]
    if out_saved is not None:
        out = np.asarray(out_saved, dtype=np.float64)
    nan = np.isnan(x)
    u = np.where(nan, 0.0, parts["u"])
    go = np.asarray(grad_out, dtype=np.float64)
    m = (np.abs(out) < MASK_BOUND) if clamp_out else np.ones(out.shape, bool)
    lam_d = np.repeat(lam_t, hd, axis=2)
    a = np.empty_like(z)
    acc = np.zeros((B, D)) if grad_state is None else np.asarray(grad_state, np.float64).reshape(B, D).copy()
    for t in range(S - 1, -1, -1):
        lam_next = lam_d[:, t + 1, :] if t + 1 < S else 1.0
        acc = np.where(m[:, t, :], go[:, t, :] + lam_next * acc, 0.0)
        a[:, t, :] = acc
    delta = np.repeat(np.asarray(damping, dtype=np.float64), hd)
    dp = (1.0 - lam_d) * a * delta * (1.0 - z * z)
    if nan_policy == "zero_z":
        dp = np.where(nan, 0.0, dp)
    Tk = chebyshev_basis(u, K)                                  # [B,S,D,K]
    gc = np.einsum("bsd,bsdk->bdk", dp, Tk).reshape(B, H, hd, K).transpose(0, 1, 3, 2)
    # p'(u) from U_{k-1}: U_0 = 1, U_1 = 2u, U_k = 2u U_{k-1} - U_{k-2}
    cl = lane_coeffs(coeffs)                                    # [B,D,K]
    U = [np.ones_like(u), 2.0 * u]
    for _ in range(2, K):
        U.append(2.0 * u * U[-1] - U[-2])
    dpdu = np.zeros_like(u)
    for k in range(1, K):
        dpdu += k * cl[:, None, :, k] * U[k - 1]
    with np.errstate(invalid="ignore"):
        dudx = 1.0 / (1.0 + np.abs(x)) ** 2
    live = ~nan & (np.abs(x) >= SOFTSIGN_GRAD_MIN)
    gx = np.where(live, dp * dpdu * dudx, 0.0)
    gi = lam_d[:, 0, :] * a[:, 0, :]
    return gx, gc, gi


def _forward_torch(x, coeffs, damping, lam, g, lam_shift, lam_min, lam_max, ema_init,
                   nan_policy="zero_z", state_clamp=None):
    """The forward as a float64 torch graph (small shapes: the EMA is a
    loop).  The softsign is written as the reference writes it
    (sdpc_kernel.py:1722-1725).  With ``state_clamp`` = c the recurrence's
    state is clamped to [-c, c] at every step and is the output."""
    import torch

    B, S, D = x.shape
    _, H, K, hd = coeffs.shape
    nan = torch.isnan(x)
    u = x.sign() * (1.0 - 1.0 / (1.0 + x.abs().clamp(min=1e-7)))
    u = torch.where(nan, torch.zeros_like(u), u)
    cl = coeffs.permute(0, 1, 3, 2).reshape(B, 1, D, K)
    T = [torch.ones_like(u), u]
    for _ in range(2, K):
        T.append(2.0 * u * T[-1] - T[-2])
    basis = torch.stack(T[:K], dim=-1)
    p = (basis * cl).sum(-1)
    delta = torch.as_tensor(np.repeat(np.asarray(damping, np.float64), hd))
    z = torch.tanh(delta * p)
    if nan_policy == "zero_z":
        z = torch.where(nan, torch.zeros_like(z), z)
    lam_t = torch.as_tensor(np.ascontiguousarray(lambda_field(lam, B, S, H, g, lam_shift, lam_min, lam_max)))
    lam_d = lam_t.repeat_interleave(hd, dim=2)
    state = torch.zeros(B, D, dtype=torch.float64) if ema_init is None else ema_init
    outs = []
    for t in range(S):
        state = lam_d[:, t] * state + (1.0 - lam_d[:, t]) * z[:, t]
        if state_clamp is not None:
            state = torch.clamp(state, -state_clamp, state_clamp)
        outs.append(state)
    s = torch.stack(outs, dim=1)
    out = s if state_clamp is not None else torch.clamp(s, -1.0, 1.0)
    return out, state, u


def backward_autograd(x, coeffs, damping, lam, grad_out, *, g=None, lam_shift=0.004, lam_min=0.9,
                      lam_max=0.9999, ema_init=None, grad_state=None, nan_policy="zero_z",
                      state_clamp=None):
    """Same gradients by torch float64 autograd of ``_forward_torch``
    (small shapes).  Returns (grad_x, grad_coeffs, grad_init, out)."""
    import torch

    xt = torch.as_tensor(np.asarray(x, dtype=np.float64)).clone().requires_grad_(True)
    B, S, D = xt.shape
    c = torch.as_tensor(np.asarray(coeffs, dtype=np.float64)).clone().requires_grad_(True)
    init = torch.zeros(B, D, dtype=torch.float64) if ema_init is None else \
        torch.as_tensor(np.asarray(ema_init, np.float64).reshape(B, D))
    init = init.clone().requires_grad_(True)
    out, fin, _ = _forward_torch(xt, c, damping, lam, g, lam_shift, lam_min, lam_max, init,
                                 nan_policy, state_clamp)
    loss = (out * torch.as_tensor(np.asarray(grad_out, np.float64))).sum()
    if grad_state is not None:
        loss = loss + (fin * torch.as_tensor(np.asarray(grad_state, np.float64).reshape(B, D))).sum()
    loss.backward()
    return xt.grad.numpy(), c.grad.numpy(), init.grad.numpy(), out.detach().numpy()


def ttt_grad_autograd(x, coeffs, damping, lam, *, g=None, lam_shift=0.004, lam_min=0.9,
                      lam_max=0.9999, ema_init=None, target="x"):
    """Same gradient by torch float64 autograd on the explicit forward graph
    (small shapes only: the EMA is a Python loop over t)."""
    import torch

    xt = torch.as_tensor(np.asarray(x, dtype=np.float64))
    B, S, D = xt.shape
    _, H, K, hd = np.shape(coeffs)
    c = torch.as_tensor(np.asarray(coeffs, dtype=np.float64)).clone().requires_grad_(True)
    nan = torch.isnan(xt)
    u = torch.where(torch.isinf(xt), torch.sign(xt), xt / (1.0 + xt.abs()))
    u = torch.where(nan, torch.zeros_like(u), u)
    cl = c.permute(0, 1, 3, 2).reshape(B, 1, D, K)
    T = [torch.ones_like(u), u]
    for _ in range(2, K):
        T.append(2.0 * u * T[-1] - T[-2])
    basis = torch.stack(T[:K], dim=-1)
    p = (basis * cl).sum(-1)
    delta = torch.as_tensor(np.repeat(np.asarray(damping, np.float64), hd))
    z = torch.tanh(delta * p)
    z = torch.where(nan, torch.zeros_like(z), z)
    lam_t = torch.as_tensor(np.ascontiguousarray(lambda_field(lam, B, S, H, g, lam_shift, lam_min, lam_max)))
    lam_d = lam_t.repeat_interleave(hd, dim=2)
    state = torch.zeros(B, D, dtype=torch.float64) if ema_init is None else \
        torch.as_tensor(np.asarray(ema_init, np.float64).reshape(B, D))
    outs = []
    for t in range(S):
        state = lam_d[:, t] * state + (1.0 - lam_d[:, t]) * z[:, t]
        outs.append(state)
    s = torch.stack(outs, dim=1)
    out = torch.clamp(s, -1.0, 1.0)
    y = xt if target == "x" else torch.where(nan, xt, u)
    loss = torch.nn.functional.mse_loss(out[:, :-1], y[:, 1:])
    loss.backward()
    G = c.grad.numpy() / (np.arange(1, K + 1, dtype=np.float64) ** 2).reshape(1, 1, K, 1)
    return G, out.detach().numpy(), state.detach().numpy()


def rel_err(a, b):
    """max|a-b| / max|b| over finite entries (0 when b is all zero and a == b)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.max(np.abs(b)) if b.size else 0.0
    num = np.max(np.abs(a - b)) if a.size else 0.0
    return num / den if den > 0 else num
