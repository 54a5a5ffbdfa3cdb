"""MI355X-native (gfx950) Cheby-RKV hot path of OrthoSSM.

Fused softsign -> Clenshaw -> per-head damping -> tanh -> per-head EMA scan,
with dynamic lambda, EMA carry across chunks, bf16 I/O, the fused TTT
coefficient gradient, the backward and the full online-TTT path,
implemented as hand-written HIP kernels behind the C ABI of
``include/osm.h`` (library ``orthossm_amd/_lib/libosm.so``); the engine's
call sites in ``orthossm_amd.engine``.
"""
from .ops import cheby_ema, cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt
from .sdpc_kernel import apply_cheby_rkv_core, apply_cheby_rkv_v10
from .engine import ChebyContextPath, ChebyState

__all__ = ["cheby_ema", "cheby_ema_forward", "cheby_ema_backward", "cheby_ema_ttt", "apply_cheby_rkv_v10",
           "apply_cheby_rkv_core", "ChebyContextPath", "ChebyState"]
