"""Drop-in replacement for the reference's public op ``apply_cheby_rkv_v10``.

Reference: sdpc_kernel.py:2522-2606 (public op), alias
``apply_cheby_rkv_core`` at sdpc_kernel.py:2610.

Covered: the fixed-coefficient path the reference takes when
``S < seq_threshold`` (``_fast_path_forward``, sdpc_kernel.py:1708-1744):
stable softsign, Chebyshev evaluation, damping 0.98 - 0.06*h/H, tanh, EMA
with the scalar momentum ``ema_momentum`` on every head, output clamp, and a
NaN input counted as u = 0 as that path does (sdpc_kernel.py:1725); the
coefficients and momentum come back unchanged (cast to fp32, as
sdpc_kernel.py:2549-2552).  The Chebyshev series is evaluated exactly
(the reference's fast path also evaluates it exactly, by basis + einsum).
Gradients flow to x and coeffs through the fused backward, as the
reference's autograd does through that path (its EMA backward
_EMAFastPathFn.backward, sdpc_kernel.py:1677-1701, masks the adjoint with
|out| < 1 - 1e-6).

The full path (``S >= seq_threshold``; sdpc_kernel.py:2559-2606: online TTT
over ``chunk_size``-token chunks, each a ``FusedChebyRKVv10.forward`` with the
inline Lion update, LUT or 4-term Clenshaw series, clamped tanh, EMA restarted
at every chunk, bf16 rounding of x and of the output) runs as one launch of
``v10_chunked_ttt``; with gradients enabled, through ``v10_full_path``,
whose backward is the reference's (FusedChebyRKVv10.backward,
sdpc_kernel.py:2436-2515) on every chunk.
"""
from __future__ import annotations

import torch

from .ops import cheby_ema, cheby_ema_forward, head_momentum, v10_chunked_ttt, v10_full_path


def v10_damping(n_heads: int, device=None) -> torch.Tensor:
    """Per-head damping hard-coded in the reference kernels (sdpc_kernel.py:1734-1736)."""
    h = torch.arange(n_heads, dtype=torch.float32, device=device)
    return 0.98 - 0.06 * h / n_heads


def apply_cheby_rkv_v10(x, coeffs, momentum_buf, n_heads=4, base_lr=0.005, ema_momentum=0.9,
                        lion_beta1=0.9, lion_beta2=0.99, lion_wd=0.01, chunk_size=256, use_bf16=False,
                        gate_global=None, dynamic_lambda=None, use_lut=True, seq_threshold=384,
                        lion_max_norm=14.0):
    """Same signature and return convention as the reference:
    returns (out [B,S,D] fp32, coeffs fp32, momentum_buf fp32 or None).
    ``ema_momentum`` may also be a one-element tensor on the device, read
    there by the kernels (the reference takes a Python float, which its
    engine obtains with a host synchronisation, sdpc_engine.py:209)."""
    B, S, D = x.shape
    if coeffs.dtype != torch.float32:
        coeffs = coeffs.float()
    if momentum_buf is not None and momentum_buf.dtype != torch.float32:
        momentum_buf = momentum_buf.float()
    H = n_heads
    if D % H:
        raise ValueError(f"D={D} is not divisible by n_heads={H}")
    if not (seq_threshold > 0 and S < seq_threshold):
        run = v10_chunked_ttt
        if torch.is_grad_enabled() and (x.requires_grad or coeffs.requires_grad):
            run = v10_full_path
        out, c_new, m_new = run(
            x, coeffs, momentum_buf, n_heads=H, base_lr=base_lr, ema_momentum=ema_momentum, beta1=lion_beta1,
            beta2=lion_beta2, weight_decay=lion_wd, chunk_size=chunk_size, gate_global=gate_global,
            dynamic_lambda=dynamic_lambda, use_lut=use_lut)
        return out, c_new, m_new
    if coeffs.shape[2] > 8:
        # The reference's PyTorch fast path evaluates any number of terms; its
        # kernels (and its engine, max_degree <= 8) stop at eight.
        raise ValueError(f"the fast path supports at most 8 Chebyshev coefficients, got {coeffs.shape[2]}")
    damping = v10_damping(H, x.device)
    lam = head_momentum(ema_momentum, H, x.device)
    if torch.is_grad_enabled() and (x.requires_grad or coeffs.requires_grad):
        out = cheby_ema(x, coeffs, damping, lam, out_dtype=torch.float32, nan_policy="zero_u")
    else:
        out = cheby_ema_forward(x, coeffs, damping, lam, out_dtype=torch.float32, nan_policy="zero_u")
    return out, coeffs, momentum_buf


apply_cheby_rkv_core = apply_cheby_rkv_v10
