"""The Chebyshev-RKV call sites of the reference's engine,
``SpectralDualPathContextEngine`` (sdpc_engine.py:57-351), on the gfx950
kernels.

What the engine does around ``apply_cheby_rkv_v10`` is mirrored here:

* the ``cheby_state`` forms it accepts (sdpc_engine.py:173-192): ``None``
  (input-dependent coefficients from the mean of the normalised input through
  ``coeff_init_proj`` times the spectral scale 0.1/(k+1), zero momentum),
  ``(coeffs, momentum)``, the older ``(coeffs, m1, m2)`` form (m1 is the
  momentum), or a bare coefficient tensor ([B,K,hd] gains a head axis; fewer
  than ``max_degree`` coefficients are zero-padded; zero momentum);
* the complexity gate (``GatedComplexityPredictor``,
  sdpc_kernel.py:1818-1830) fed as both ``gate_global`` and
  ``dynamic_lambda`` (sdpc_engine.py:195-197, 239-249);
* the adaptive EMA momentum, 0.7 + 0.5 (ema_base - 0.7)(1 + cos(pi p)),
  p = clamp(tokens seen / 1e8, 0, 1), counted after adding this call's
  tokens (sdpc_engine.py:199-208).  The reference reads it back to the host
  (``.item()``, sdpc_engine.py:209) to pass a float; here it stays a device
  scalar that the kernels read, so a forward makes no host synchronisation;
* the length routing (sdpc_engine.py:216-225): S < 384 takes the fast path
  (``seq_threshold=384``), 384 <= S < 1024 the hybrid and S >= 1024 the full
  path, both with ``seq_threshold=0`` (sdpc_engine.py:275-285, 300-333); the
  full path optionally under activation checkpointing when training
  (``gradient_ckpt``, sdpc_engine.py:323-333);
* the new state ``(coeffs.detach(), momentum.detach())``
  (sdpc_engine.py:266, 297).

Parameter and buffer names follow the engine's (``input_norm``,
``complexity_gate.net``, ``coeff_init_proj``, ``coeff_spectral_scale``,
``ema_base``, ``total_tokens_seen``), so those entries of an engine
state_dict load here.

Added, with no counterpart in the reference: an EMA-state carry.  The
reference restarts the EMA from zero at every call; with ``carry_ema=True``
the state returned is a ``ChebyState(coeffs, momentum, ema)`` whose ``ema``
[B, D] seeds the next fast-path call, so consecutive short calls continue one
scan.  The full path restarts its EMA at every chunk (as the reference does),
so after a full-path call ``ema`` is None.

Not built (outside the Cheby-RKV path): the local refiner (SLR), landmark
archive, LightBus, SwiGLU fusion, state refresh, recall residual and the
diagnostics.  ``forward`` returns the normalised input and the gate with the
Chebyshev output so an engine can feed those parts.
"""
from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint as torch_checkpoint

from .ops import cheby_ema, cheby_ema_forward, head_momentum
from .sdpc_kernel import GatedComplexityPredictor, apply_cheby_rkv_v10, v10_damping

# Length routing thresholds (sdpc_engine.py:51-53).
FAST_PATH_THRESHOLD = 384
HYBRID_PATH_THRESHOLD = 1024
# Tokens over which the EMA momentum anneals (sdpc_engine.py:205).
PROJECTED_TOKENS = 1e8


class ChebyState(NamedTuple):
    """Recurrent state with the EMA carry: coeffs and momentum [B,H,K,hd]
    fp32, ema [B, D] fp32 or None."""
    coeffs: torch.Tensor
    momentum: torch.Tensor
    ema: torch.Tensor | None


class ChebyPathOutput(NamedTuple):
    out: torch.Tensor              # [B,S,D] fp32 Chebyshev-RKV output
    state: tuple                   # (coeffs, momentum) or ChebyState
    x_normed: torch.Tensor         # input_norm(x), the other paths' input
    gate: torch.Tensor             # [B,1] complexity gate
    ema_momentum: torch.Tensor     # 0-d fp32 device tensor used as mu
    route: str                     # "fast", "hybrid" or "full"


def route(seq_len: int) -> str:
    """The engine's tier for a sequence length (sdpc_engine.py:216-225)."""
    if seq_len < FAST_PATH_THRESHOLD:
        return "fast"
    if seq_len < HYBRID_PATH_THRESHOLD:
        return "hybrid"
    return "full"


def ema_momentum_schedule(tokens_seen: torch.Tensor, ema_base: torch.Tensor) -> torch.Tensor:
    """0.7 + 0.5 (ema_base - 0.7)(1 + cos(pi p)), p = clamp(tokens/1e8, 0, 1),
    in fp32 on the tensors' device (sdpc_engine.py:203-208)."""
    progress = (tokens_seen.float() / PROJECTED_TOKENS).clamp(0.0, 1.0)
    return 0.7 + 0.5 * (ema_base - 0.7) * (1.0 + torch.cos(progress * math.pi))


def parse_cheby_state(cheby_state, max_degree: int):
    """(coeffs, momentum, ema) from the state forms the engine accepts
    (sdpc_engine.py:182-192), plus ChebyState; None for the state means
    the caller initialises the coefficients."""
    if isinstance(cheby_state, ChebyState):
        return cheby_state.coeffs, cheby_state.momentum, cheby_state.ema
    if isinstance(cheby_state, tuple) and len(cheby_state) == 2:
        return cheby_state[0], cheby_state[1], None
    if isinstance(cheby_state, tuple) and len(cheby_state) == 3:
        return cheby_state[0], cheby_state[1], None          # (coeffs, m1, m2): m1 is the momentum
    coeffs = cheby_state
    if coeffs.dim() == 3:
        coeffs = coeffs.unsqueeze(1)
    if coeffs.shape[2] < max_degree:
        coeffs = F.pad(coeffs, (0, 0, 0, max_degree - coeffs.shape[2]))
    return coeffs, torch.zeros_like(coeffs), None


class ChebyContextPath(nn.Module):
    """The Chebyshev-RKV half of the engine: input norm, coefficient init,
    complexity gate, EMA momentum schedule, length routing and the call into
    the fused kernels.  Constructor arguments keep the engine's names."""

    def __init__(self, d_model: int, n_cheby_heads: int = 8, max_degree: int = 4, chunk_size: int = 256,
                 use_bf16: bool = False, use_lut: bool = True, gradient_ckpt: bool = False,
                 carry_ema: bool = False, base_lr: float = 0.005):
        super().__init__()
        if d_model % n_cheby_heads:
            raise ValueError(f"d_model={d_model} is not divisible by n_cheby_heads={n_cheby_heads}")
        self.d_model = d_model
        self.n_cheby_heads = n_cheby_heads
        self.head_dim = d_model // n_cheby_heads
        self.max_degree = max_degree
        self.chunk_size = chunk_size
        self.use_bf16 = use_bf16
        self.use_lut = use_lut
        self.gradient_ckpt = gradient_ckpt
        self.carry_ema = carry_ema
        self.base_lr = base_lr

        self.complexity_gate = GatedComplexityPredictor(d_model)
        self.coeff_init_proj = nn.Sequential(
            nn.Linear(d_model, d_model // 4), nn.SiLU(),
            nn.Linear(d_model // 4, n_cheby_heads * max_degree * self.head_dim))
        nn.init.zeros_(self.coeff_init_proj[-1].weight)     # zero coefficients at start
        nn.init.zeros_(self.coeff_init_proj[-1].bias)
        k = torch.arange(max_degree, dtype=torch.float32)
        self.register_buffer("coeff_spectral_scale", (0.1 / (k + 1.0)).view(1, 1, max_degree, 1))
        self.input_norm = nn.RMSNorm(d_model)
        self.register_buffer("ema_base", torch.tensor(0.9))
        self.register_buffer("total_tokens_seen", torch.tensor(0, dtype=torch.long))

    def _cheby_compute(self, x_normed, coeffs, momentum, ema_momentum, gate, seq_threshold):
        return apply_cheby_rkv_v10(x_normed, coeffs, momentum, n_heads=self.n_cheby_heads, base_lr=self.base_lr,
                                   ema_momentum=ema_momentum, chunk_size=self.chunk_size, use_bf16=self.use_bf16,
                                   gate_global=gate, dynamic_lambda=gate, use_lut=self.use_lut,
                                   seq_threshold=seq_threshold)

    def _fast_with_carry(self, x_normed, coeffs, ema_init, ema_momentum):
        """The fast path (sdpc_kernel.py:1708-1744) continuing the EMA from
        ``ema_init``; returns (out, ema_final)."""
        dev = x_normed.device
        H = self.n_cheby_heads
        coeffs = coeffs.float()
        damping = v10_damping(H, dev)
        lam = head_momentum(ema_momentum, H, dev)
        kw = dict(ema_init=ema_init, out_dtype=torch.float32, return_state=True, nan_policy="zero_u")
        if torch.is_grad_enabled() and (x_normed.requires_grad or coeffs.requires_grad or
                                        (ema_init is not None and ema_init.requires_grad)):
            return cheby_ema(x_normed, coeffs, damping, lam, **kw)
        return cheby_ema_forward(x_normed, coeffs, damping, lam, **kw)

    def forward(self, x: torch.Tensor, cheby_state=None) -> ChebyPathOutput:
        B, S, D = x.shape
        if D != self.d_model:
            raise ValueError(f"x has D={D}, the module d_model={self.d_model}")
        n_h, hd, deg = self.n_cheby_heads, self.head_dim, self.max_degree
        x_normed = self.input_norm(x)
        x_mean = x_normed.mean(dim=1)
        if cheby_state is None:
            coeffs = self.coeff_init_proj(x_mean).view(B, n_h, deg, hd) * self.coeff_spectral_scale
            momentum = torch.zeros(B, n_h, deg, hd, device=x.device)
            ema = None
        else:
            coeffs, momentum, ema = parse_cheby_state(cheby_state, deg)
        gate = self.complexity_gate(x_mean)
        with torch.no_grad():
            self.total_tokens_seen.add_(S)
            mu = ema_momentum_schedule(self.total_tokens_seen, self.ema_base).float()

        tier = route(S)
        if tier == "fast":
            if self.carry_ema:
                out, ema = self._fast_with_carry(x_normed, coeffs, ema, mu)
            else:
                out, coeffs, momentum = self._cheby_compute(x_normed, coeffs, momentum, mu, gate,
                                                            FAST_PATH_THRESHOLD)
        else:
            if tier == "full" and self.gradient_ckpt and self.training:
                out, coeffs, momentum = torch_checkpoint(self._cheby_compute, x_normed, coeffs, momentum, mu, gate,
                                                         0, use_reentrant=False)
            else:
                out, coeffs, momentum = self._cheby_compute(x_normed, coeffs, momentum, mu, gate, 0)
            ema = None
        coeffs = coeffs.float()
        if momentum is not None:
            momentum = momentum.float()
        if self.carry_ema:
            state = ChebyState(coeffs.detach(), None if momentum is None else momentum.detach(),
                               None if ema is None else ema.detach())
        else:
            state = (coeffs.detach(), None if momentum is None else momentum.detach())
        return ChebyPathOutput(out, state, x_normed, gate, mu, tier)
