"""CPU restatement of the reference's full ``apply_cheby_rkv_v10`` path:
chunked online TTT with an inline Lion update.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` (and bench's CPU baseline),
never by the product package.

Per chunk of ``chunk_size`` tokens (sdpc_kernel.py:2574-2606; one chunk when
S <= chunk_size, 2563-2572), ``FusedChebyRKVv10.forward`` (2353-2433) runs
``_ortho_megakernel`` (1890-2287) with the chunk's coefficients and Lion
momentum and returns the updated ones, which the next chunk uses:

* x is rounded to bf16 (2385); u = sign(x) (1 - 1/(1 + max(|x|, 1e-7))) with
  a NaN read as 0 and sign(0) = +1 (2020-2027), so NaN and 0 give u = +1.19e-7;
* the series is a 256-point half-range LUT with linear interpolation and odd
  parity (2030-2069, table 63-81), or with use_lut=False the four-term
  Clenshaw fallback that ignores c4..c7 (2070-2077);
* y *= 0.98 - 0.06 h/H; z = tanh(clamp(y, -4, 4)) in exp form; NaN x gives
  z = 0 (2080-2086);
* EMA with the scalar ``ema_momentum`` from a zero state at every chunk
  (2398, 2097-2124; the per-128-token clamp of the carried state never binds
  because |z| <= tanh(4) < 1);
* proxy gradient over the chunk's pairs (t, t+1): err = u[t+1] - s[t],
  gv = err / (1 + exp(-3|err|)), gc_k = sum_t gv T_k(u[t]) with T_k of the
  exact u (2126-2170);
* Lion (2179-2287, constants 1416-1437): g = gc / (len - 1);
  interp = b1 m + (1-b1) g; m' = b2 m + (1-b2) g;
  c' = decay c + lr ss_k sign(interp), ss_k = (k+1)^-1.5,
  lr = base_lr (1 + 0.25 (h - H/2)/H) (x gate[b]),
  decay = lam_h - lr wd, lam_h = MULTI_SCALE_LAMBDA[h] (0.995 past 8 heads),
  with dynamic_lambda[b]: lam_h <- clamp(lam_h + 0.008 (dl - 0.5), 0.9, 0.9999);
* the returned output is the fp32 EMA rounded to bf16 (2422, 2433).

Arithmetic is float64 except for the two bf16 roundings the reference
applies (x on entry, the output), and the LUT itself, which holds the
reference's float32 table values (``chebyshev_lut``).
"""
from __future__ import annotations

import numpy as np

MULTI_SCALE_LAMBDA = (0.9995, 0.9995, 0.997, 0.997, 0.995, 0.995, 0.97, 0.95)
LUT_SIZE = 256
MAX_DEGREE = 8


def bf16_round(a) -> np.ndarray:
    """Round float32 values to bf16 (round to nearest even; NaN stays NaN),
    returned as float64."""
    f = np.asarray(a, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(np.isnan(f), np.nan, out)


def chebyshev_lut(table_size: int = LUT_SIZE, max_degree: int = MAX_DEGREE) -> np.ndarray:
    """T_k at torch.linspace(0, 1, table_size) in float32 by the Chebyshev
    recurrence, as the reference builds its table (sdpc_kernel.py:63-81);
    [max_degree, table_size] float32."""
    import torch

    x = torch.linspace(0.0, 1.0, table_size)
    T = torch.zeros(max_degree, table_size)
    T[0] = 1.0
    if max_degree > 1:
        T[1] = x
    for k in range(2, max_degree):
        T[k] = 2.0 * x * T[k - 1] - T[k - 2]
    return T.numpy()


def v10_softsign(xb):
    """u, |u|, sign and the NaN mask of the megakernel's softsign
    (sdpc_kernel.py:2020-2027) on bf16-rounded x."""
    xb = np.asarray(xb, dtype=np.float64)
    nan = np.isnan(xb)
    xs = np.where(nan, 0.0, xb)
    ax = np.maximum(np.abs(xs), np.float64(np.float32(1e-7)))
    with np.errstate(over="ignore"):
        absu = 1.0 - 1.0 / (1.0 + ax)
    sign = np.where(xs >= 0.0, 1.0, -1.0)
    return sign * absu, absu, sign, nan


def lut_series(c, absu, sign, lut):
    """sum_k c_k T_k(u) by LUT interpolation (sdpc_kernel.py:2030-2069).
    c: [..., K] broadcasting against absu/sign with the coefficient axis last."""
    n = lut.shape[1]
    fidx = absu * (n - 1)
    idx0 = np.clip(np.floor(fidx).astype(np.int64), 0, None)
    idx0 = np.where(idx0 >= n - 1, n - 2, idx0)
    frac = np.clip(fidx - idx0, 0.0, 1.0)
    K = c.shape[-1]
    y = np.zeros(np.broadcast_shapes(c.shape[:-1], absu.shape))
    lut64 = lut.astype(np.float64)
    for k in range(min(K, lut.shape[0])):
        ta = lut64[k][idx0]
        tb = lut64[k][idx0 + 1]
        term = c[..., k] * (ta + frac * (tb - ta))
        y = y + (term * sign if k % 2 else term)
    return y


def clenshaw4_series(c, u):
    """The megakernel's Clenshaw fallback (sdpc_kernel.py:2070-2077): only
    c0..c3 enter, whatever K is."""
    K = c.shape[-1]
    ck = [c[..., k] if k < K else 0.0 for k in range(4)]
    u3 = ck[3]
    u2 = 2.0 * u * u3 + ck[2]
    u1 = 2.0 * u * u2 - u3 + ck[1]
    return u * u1 - u2 + ck[0]


def lion_constants(H: int, K: int):
    """(lambda [H], spectral scale [K], lr scale [H]) as sdpc_kernel.py:1423-1437."""
    n_active = min(H, len(MULTI_SCALE_LAMBDA))
    lam = np.array(list(MULTI_SCALE_LAMBDA[:n_active]) + [0.995] * max(0, H - n_active))
    ss = 1.0 / (np.arange(K, dtype=np.float64) + 1.0) ** 1.5
    lr_scale = 1.0 + 0.25 * (np.arange(H, dtype=np.float64) - H / 2.0) / max(H, 1)
    return lam, ss, lr_scale


def v10_chunk(xb, c, m, *, ema_momentum, base_lr, beta1, beta2, wd, gate=None, dyn=None, use_lut=True,
              lut=None):
    """One FusedChebyRKVv10 forward on a chunk.  xb: bf16-rounded x
    [B,L,D] (float64); c, m: [B,H,K,hd].  Returns (s [B,L,D] float64 EMA
    output before the bf16 rounding, c_new, m_new, z)."""
    B, L, D = xb.shape
    _, H, K, hd = c.shape
    Kk = min(K, MAX_DEGREE)
    u, absu, sign, nan = v10_softsign(xb)
    cl = c.transpose(0, 1, 3, 2).reshape(B, 1, D, K)[..., :Kk]        # [B,1,D,Kk]
    if use_lut:
        y = lut_series(cl, absu, sign, lut if lut is not None else chebyshev_lut())
    else:
        y = clenshaw4_series(cl, u)
    gamma = np.repeat(0.98 - 0.06 * np.arange(H) / H, hd)
    yc = np.clip(y * gamma, -4.0, 4.0)
    e2 = np.exp(2.0 * yc)
    z = np.where(nan, 0.0, (e2 - 1.0) / (e2 + 1.0))
    mu = float(ema_momentum)
    s = np.empty_like(z)
    state = np.zeros((B, D))
    for t in range(L):
        state = mu * state + (1.0 - mu) * z[:, t]
        s[:, t] = state
    s = np.clip(s, -1.0, 1.0)
    gc = proxy_grad(u, s, Kk)                                                # [B,D,Kk]
    gc = gc.reshape(B, H, hd, Kk).transpose(0, 1, 3, 2)                       # [B,H,Kk,hd]
    c_new, m_new = lion_update(c, m, gc, L, base_lr=base_lr, beta1=beta1, beta2=beta2, wd=wd, gate=gate,
                               dyn=dyn)
    return s, c_new, m_new, z


def proxy_grad(u, s, K):
    """gc[b,d,k] = sum over pairs (t, t+1) of the chunk of gv T_k(u[t]),
    gv = err / (1 + exp(-3|err|)), err = u[t+1] - s[t] (sdpc_kernel.py:2126-2170)."""
    err = np.zeros_like(s)
    err[:, :-1] = u[:, 1:] - s[:, :-1]
    gv = err / (1.0 + np.exp(-3.0 * np.abs(err)))
    T = [np.ones_like(u), u]
    for _ in range(2, K):
        T.append(2.0 * u * T[-1] - T[-2])
    return np.stack([np.sum(gv * T[k], axis=1) for k in range(K)], axis=-1)


def lion_update(c, m, gc, L, *, base_lr, beta1, beta2, wd, gate=None, dyn=None):
    """Lion step of the megakernel (sdpc_kernel.py:2179-2287) for the first
    gc.shape[2] coefficients; gc [B,H,Kk,hd] is the chunk's summed proxy
    gradient over L tokens.  Returns (c_new, m_new) [B,H,K,hd]."""
    B, H, Kk, hd = gc.shape
    lam, ss, lr_scale = lion_constants(H, Kk)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv_s = 1.0 / np.float64(L - 1) if L > 1 else np.inf
        g = gc * inv_s
    lr = base_lr * lr_scale[None, :] * np.ones((B, 1))                       # [B,H]
    eff = np.broadcast_to(lam[None, :], (B, H)).copy()
    if dyn is not None:
        eff = np.clip(lam[None, :] + 0.008 * (np.asarray(dyn, np.float64).reshape(B, 1) - 0.5), 0.90, 0.9999)
    if gate is not None:
        lr = lr * np.asarray(gate, np.float64).reshape(B, 1)
    decay = (eff - lr * wd)[:, :, None, None]
    cK = np.asarray(c, np.float64)[:, :, :Kk]
    mK = np.asarray(m, np.float64)[:, :, :Kk]
    with np.errstate(invalid="ignore"):
        interp = beta1 * mK + (1.0 - beta1) * g
        m_new_k = beta2 * mK + (1.0 - beta2) * g
    sgn = np.where(interp > 0, 1.0, np.where(interp < 0, -1.0, 0.0))
    c_new_k = decay * cK + lr[:, :, None, None] * ss[None, None, :, None] * sgn
    c_new = np.asarray(c, np.float64).copy()
    m_new = np.asarray(m, np.float64).copy()
    c_new[:, :, :Kk] = c_new_k
    m_new[:, :, :Kk] = m_new_k
    return c_new, m_new


def v10_full(x, coeffs, momentum, *, n_heads=4, base_lr=0.005, ema_momentum=0.9, beta1=0.9, beta2=0.99,
             wd=0.01, chunk_size=256, gate_global=None, dynamic_lambda=None, use_lut=True, lut=None):
    """The full path of apply_cheby_rkv_v10 (S >= seq_threshold).  Returns
    (out [B,S,D] bf16 values as float64, coeffs, momentum) after the last
    chunk.  Coefficients of later chunks come from the Lion update of
    earlier ones (sdpc_kernel.py:2574-2606)."""
    x = np.asarray(x, dtype=np.float32)
    B, S, D = x.shape
    c = np.asarray(coeffs, dtype=np.float64)
    m = np.asarray(momentum, dtype=np.float64)
    assert c.shape[1] == n_heads
    xb = bf16_round(x)
    outs = []
    for t0 in range(0, S, chunk_size):
        s, c, m, _ = v10_chunk(xb[:, t0:t0 + chunk_size], c, m, ema_momentum=ema_momentum, base_lr=base_lr,
                               beta1=beta1, beta2=beta2, wd=wd, gate=gate_global, dyn=dynamic_lambda,
                               use_lut=use_lut, lut=lut)
        outs.append(bf16_round(s.astype(np.float32)))
    return np.concatenate(outs, axis=1), c, m


def clenshaw8_series(c, u):
    """The fused Clenshaw + EMA kernel's Clenshaw above four coefficients
    (sdpc_kernel.py:1148-1156): all of c0..c7 enter (zeros past K),
    b_k = 2u b_{k+1} - b_{k+2} + c_k, y = u b_1 - b_2 + c_0."""
    K = c.shape[-1]
    ck = [c[..., k] if k < K else 0.0 for k in range(8)]
    b1, b2 = ck[7], 0.0
    for k in range(6, 0, -1):
        b1, b2 = 2.0 * u * b1 - b2 + ck[k], b1
    return u * b1 - b2 + ck[0]


def fused_clenshaw_ema(x, coeffs, *, n_heads, ema_momentum=0.9, ema_init=None, use_lut=True, lut=None,
                       block_s=128):
    """The reference's _fused_clenshaw_ema_kernel (sdpc_kernel.py:988-1209)
    in float64: x as given (no bf16 rounding; callers pass bf16 x when they
    want it), the megakernel's softsign (1079-1085), the LUT series
    (1101-1141) or Clenshaw over c0..c3 for K <= 4 and c0..c7 above
    (1142-1156), damping 0.98 - 0.06 h/H and the clamped exp-form tanh with
    NaN x -> 0 (1158-1165), then per tile of ``block_s`` tokens the EMA from
    the carried state, out = clamp(s, -1, 1), and the carry into the next
    tile = out at the tile's last token (1176-1200); the final state is the
    last carry (1206-1209; ema_init itself when S = 0).

    x [B,S,D], coeffs [B,H,K,hd] (K <= 8), ema_init [B,D] or None;
    ema_momentum is used as given (the kernel receives it as a float32
    argument, so parity checks pass that value).  Returns (x_norm, tanh_y,
    out, final) as float64."""
    x = np.asarray(x, dtype=np.float64)
    B, S, D = x.shape
    c = np.asarray(coeffs, dtype=np.float64)
    H = n_heads
    _, _, K, hd = c.shape
    assert c.shape[1] == H and H * hd == D and 1 <= K <= MAX_DEGREE
    u, absu, sign, nan = v10_softsign(x)
    cl = c.transpose(0, 1, 3, 2).reshape(B, 1, D, K)
    if use_lut:
        y = lut_series(cl, absu, sign, lut if lut is not None else chebyshev_lut())
    elif K <= 4:
        y = clenshaw4_series(cl, u)
    else:
        y = clenshaw8_series(cl, u)
    gamma = np.repeat(0.98 - 0.06 * np.arange(H) / H, hd)
    yc = np.clip(y * gamma, -4.0, 4.0)
    e2 = np.exp(2.0 * yc)
    z = np.where(nan, 0.0, (e2 - 1.0) / (e2 + 1.0))
    mu = float(ema_momentum)
    carry = np.zeros((B, D)) if ema_init is None else np.asarray(ema_init, np.float64).reshape(B, D).copy()
    out = np.empty((B, S, D))
    for t0 in range(0, S, block_s):
        state = carry
        for t in range(t0, min(t0 + block_s, S)):
            state = mu * state + (1.0 - mu) * z[:, t]
            out[:, t] = np.clip(state, -1.0, 1.0)
        carry = out[:, min(t0 + block_s, S) - 1]
    return u, z, out, carry


def v10_backward(x, out, zb, hist, grad_out, *, n_heads, ema_momentum, chunk):
    """The reference's backward of the full path (FusedChebyRKVv10.backward,
    sdpc_kernel.py:2436-2515) applied to every chunk (the chunk loop,
    2583-2603, feeds each chunk its own coefficients; the EMA and its adjoint
    restart at every chunk):

        u      = sign(x) (1 - 1/(1 + max(|x|, 1e-7))), NaN -> 0     (2450-2453, fp32 x)
        a[t]   = m[t] (dL/dout[t] + mu a[t+1]), a = 0 past the chunk, m = [|out| < 1 - 1e-6]
        dL/dy  = (1 - mu) a (1 - zb^2)           zb: the forward's bf16 z   (879-881)
        dL/dc_k = sum_t gamma dL/dy T_k(u)                                  (883-913)
        dL/dx  = dL/dy gamma sum_k k c_k U_{k-1}(u) / (1 + |x|)^2           (923-961, 2505)

    hist: [n_chunks, B, H, K, hd] coefficients each chunk used.  Returns
    (grad_x [B,S,D], grad_coeffs of the first chunk [B,H,K,hd])."""
    x = np.asarray(x, dtype=np.float64)
    B, S, D = x.shape
    n_chunks, _, H, K, hd = np.shape(hist)
    mu = float(ema_momentum)
    nan = np.isnan(x)
    xs = np.where(nan, 0.0, x)
    ax = np.maximum(np.abs(xs), np.float64(np.float32(1e-7)))
    u = np.where(nan, 0.0, np.sign(xs) * (1.0 - 1.0 / (1.0 + ax)))
    bound = float(np.float32(1.0 - 1e-6))
    m = np.abs(np.asarray(out, np.float64)) < bound
    g = np.asarray(grad_out, np.float64)
    zb = np.asarray(zb, np.float64)
    gamma = np.repeat(0.98 - 0.06 * np.arange(H) / H, hd)
    gx = np.zeros_like(x)
    gc0 = None
    for ch in range(n_chunks):
        t0, t1 = ch * chunk, min((ch + 1) * chunk, S)
        adj = np.zeros((B, t1 - t0, D))
        acc = np.zeros((B, D))
        for t in range(t1 - 1, t0 - 1, -1):
            acc = np.where(m[:, t], g[:, t] + mu * acc, 0.0)
            adj[:, t - t0] = acc
        dldy = (1.0 - mu) * adj * (1.0 - zb[:, t0:t1] ** 2)
        uc = u[:, t0:t1]
        T = [np.ones_like(uc), uc]
        for _ in range(2, K):
            T.append(2.0 * uc * T[-1] - T[-2])
        gc = np.stack([np.sum(gamma * dldy * T[k], axis=1) for k in range(K)], axis=-1)   # [B,D,K]
        if ch == 0:
            gc0 = gc.reshape(B, H, hd, K).transpose(0, 1, 3, 2)
        cl = np.asarray(hist[ch], np.float64).transpose(0, 1, 3, 2).reshape(B, 1, D, K)
        U = [np.ones_like(uc), 2.0 * uc]
        for _ in range(2, K):
            U.append(2.0 * uc * U[-1] - U[-2])
        dp = np.zeros_like(uc)
        for k in range(1, K):
            dp += k * cl[..., k] * U[k - 1]
        with np.errstate(invalid="ignore"):
            gx[:, t0:t1] = dldy * gamma * dp / (1.0 + np.abs(x[:, t0:t1])) ** 2
    return gx, gc0
