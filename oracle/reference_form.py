"""float32 torch restatement of the reference's own PyTorch formulation.

TEST INFRASTRUCTURE ONLY (tests and the ``cpu_baseline`` leg of bench.py).

This follows how the reference computes the operator on its PyTorch path,
with the BASELINE per-head constants as parameters:

* stable softsign  sign(x) * (1 - 1/(1 + max(|x|, 1e-7))), NaN -> 0
  (sdpc_kernel.py:1722-1725);
* a materialised Chebyshev basis [B,S,H,hd,K] contracted with the
  coefficients by einsum 'bsndk,bndk->bsnd' (sdpc_kernel.py:1728-1731,
  1751-1776);
* per-head damping multiply and torch.tanh (sdpc_kernel.py:1734-1739);
* the per-head-lambda EMA as a sequential loop over t
  (chimera_experiment/chimera_v2_ssm.py:86-101), vectorised over heads by a
  per-lane lambda vector.

It is what ``bench.py`` times on the host cores as the CPU baseline, and an
independent formulation the float64 oracle is cross-checked against.
"""
from __future__ import annotations

import torch


def _z(x: torch.Tensor, coeffs: torch.Tensor, damping: torch.Tensor) -> torch.Tensor:
    """softsign -> Chebyshev basis + einsum -> damping -> tanh, [B,S,D]."""
    B, S, D = x.shape
    _, H, K, hd = coeffs.shape
    ax = x.abs().clamp(min=1e-7)
    u = x.sign() * (1.0 - 1.0 / (1.0 + ax))
    u = torch.where(torch.isnan(x), torch.zeros_like(x), u)
    uh = u.view(B, S, H, hd)
    T = [torch.ones_like(uh), uh]
    for _ in range(2, K):
        T.append(2.0 * uh * T[-1] - T[-2])
    basis = torch.stack(T[:K], dim=-1)                       # [B,S,H,hd,K]
    y = torch.einsum("bsndk,bndk->bsnd", basis, coeffs.permute(0, 1, 3, 2))
    y = y * damping.view(1, 1, H, 1).to(y.dtype)
    return torch.tanh(y).reshape(B, S, D)


def forward(x: torch.Tensor, coeffs: torch.Tensor, damping: torch.Tensor, lam: torch.Tensor,
            ema_init: torch.Tensor | None = None):
    """x [B,S,D] float32; coeffs [B,H,K,hd]; damping [H]; lam [H].
    Returns (out [B,S,D], ema_final [B,D])."""
    B, S, D = x.shape
    hd = coeffs.shape[3]
    z = _z(x, coeffs, damping)
    lam_d = lam.to(z.dtype).repeat_interleave(hd)            # [D]
    one_m = 1.0 - lam_d
    state = torch.zeros(B, D, dtype=z.dtype) if ema_init is None else ema_init.reshape(B, D).to(z.dtype).clone()
    out = torch.empty_like(z)
    for t in range(S):
        state = lam_d * state + one_m * z[:, t]
        out[:, t] = state
    return out.clamp(-1.0, 1.0), state


def backward(x: torch.Tensor, coeffs: torch.Tensor, damping: torch.Tensor, lam: torch.Tensor,
             out: torch.Tensor, grad_out: torch.Tensor):
    """The reference's gradient of the fast path: the EMA adjoint as its
    _EMAFastPathFn.backward computes it (sdpc_kernel.py:1677-1701: mask
    |out| < 1 - 1e-6, adj[t] = m[t] (g[t] + lam adj[t+1]), dL/dz = (1-lam) adj;
    here as a sequential loop over t with a per-lane lambda), then torch
    autograd through softsign, basis, einsum, damping and tanh.
    Returns (grad_x, grad_coeffs)."""
    B, S, D = x.shape
    hd = coeffs.shape[3]
    lam_d = lam.to(grad_out.dtype).repeat_interleave(hd)
    m = (out.abs() < 1.0 - 1e-6).to(grad_out.dtype)
    adj = torch.empty_like(grad_out)
    a = torch.zeros(B, D, dtype=grad_out.dtype)
    for t in range(S - 1, -1, -1):
        a = m[:, t] * (grad_out[:, t] + lam_d * a)
        adj[:, t] = a
    xg = x.detach().clone().requires_grad_(True)
    cg = coeffs.detach().clone().requires_grad_(True)
    with torch.enable_grad():
        z = _z(xg, cg, damping)
        z.backward((1.0 - lam_d) * adj)
    return xg.grad, cg.grad
