"""Synthetic workloads of the BASELINE configurations.

One CPU ``torch.Generator`` seeded with ``seed`` draws, in this order:
x ~ N(0,1) [B,S,D]; c[b,h,k,j] = N(0,1)/(k+1) [B,H,K,hd]; and, for the
dynamic-lambda config, g ~ U(-1,1) [B,S,H].  Generation is on the CPU so
every consumer (GPU kernels, oracle, CPU baseline) sees identical values.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

BASELINE_LAMBDA = (0.9995, 0.9995, 0.997, 0.997, 0.995, 0.995, 0.95, 0.95)


@dataclass(frozen=True)
class Config:
    name: str
    B: int
    S: int
    D: int
    H: int
    K: int = 8
    dynamic: bool = False
    dtype: torch.dtype = torch.float32
    ttt: bool = False
    chunk: int = 0  # >0: processed as consecutive chunks with EMA carry
    bwd: bool = False  # the backward pass (dL/dx, dL/dc, dL/d ema_init) instead of the forward
    v10: int = 0       # >0: the reference's full path (online TTT + Lion) with chunks of this many tokens

    @property
    def hd(self) -> int:
        return self.D // self.H


# BASELINE.json configs[0..4]
CONFIGS = {
    "cpu_ref": Config("cpu_ref", B=1, S=2048, D=512, H=8),
    "headline": Config("headline", B=4, S=16384, D=512, H=8),
    "streaming": Config("streaming", B=1, S=262144, D=512, H=8, chunk=16384),
    "dynamic": Config("dynamic", B=8, S=32768, D=1024, H=8, dynamic=True),
    "bf16_ttt": Config("bf16_ttt", B=16, S=65536, D=512, H=8, dtype=torch.bfloat16, ttt=True),
    # the backward of configs[1]
    "backward": Config("backward", B=4, S=16384, D=512, H=8, bwd=True),
    # the reference's full apply_cheby_rkv_v10 path at the configs[1] shape
    "v10_full": Config("v10_full", B=4, S=16384, D=512, H=8, v10=256),
}


def baseline_lambda(H: int) -> torch.Tensor:
    lam = list(BASELINE_LAMBDA[:H]) + [BASELINE_LAMBDA[-1]] * max(0, H - len(BASELINE_LAMBDA))
    return torch.tensor(lam, dtype=torch.float32)


def baseline_damping(H: int) -> torch.Tensor:
    return torch.tensor([0.9 ** h for h in range(H)], dtype=torch.float32)


def make_inputs(B: int, S: int, D: int, H: int, K: int = 8, *, seed: int = 0, dynamic: bool = False,
                dtype: torch.dtype = torch.float32):
    """Returns dict(x, coeffs, damping, lam, g) on the CPU.  x is cast to
    ``dtype`` after drawing in fp32; everything else is fp32."""
    hd = D // H
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, D, generator=gen)
    k = torch.arange(K, dtype=torch.float32).view(1, 1, K, 1)
    c = torch.randn(B, H, K, hd, generator=gen) / (k + 1.0)
    g = torch.rand(B, S, H, generator=gen) * 2.0 - 1.0 if dynamic else None
    return {
        "x": x.to(dtype),
        "coeffs": c,
        "damping": baseline_damping(H),
        "lam": baseline_lambda(H),
        "g": g,
    }


def make_config_inputs(cfg: Config, seed: int = 0):
    return make_inputs(cfg.B, cfg.S, cfg.D, cfg.H, cfg.K, seed=seed, dynamic=cfg.dynamic, dtype=cfg.dtype)
