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

The module also carries the other names the reference's callers import from
``sdpc_kernel`` together with the op (sdpc_engine.py:39-43,
chimera_experiment/chimera_v2_ssm.py:54, pretrain_real.py:211,
benchmark_ortho.py:20, model.py:20, benchmark_ruler_pg19.py:30,
precision_tests.py:33, ortho_diagnostics.py:174): the spectral coefficient
initialisation ``init_chebyshev_coefficients``, the complexity gate module
``GatedComplexityPredictor``, the LUT accessor ``get_chebyshev_lut`` with
``LUT_TABLE_SIZE`` and ``MAX_DEGREE``, and ``MULTI_SCALE_LAMBDA``.  The
one kernel object a caller launches directly, ``_fused_clenshaw_ema_kernel``
(precision_tests.py:33, 61-73: ``kernel[grid](pointers, sizes, strides,
BLOCK_HD=..., BLOCK_S=..., USE_LUT=...)``), is a launcher with the same
launch syntax and argument list over ``osm_cheby_ema_lut_fwd``.
"""
from __future__ import annotations

import math
import threading

import torch
import torch.nn as nn

from .ops import (LUT_POINTS, LUT_TERMS, V10_LION_LAMBDA, cheby_ema, cheby_ema_forward, cheby_ema_lut_forward,
                  chebyshev_lut_table, head_momentum, v10_chunked_ttt, v10_full_path)

# Points of the full path's half-table LUT and the number of Chebyshev terms
# it holds (sdpc_kernel.py:58-59).
LUT_TABLE_SIZE: int = LUT_POINTS
MAX_DEGREE: int = LUT_TERMS
# Per-head Lion forget factors of the full path, heads 0..7 (sdpc_kernel.py:1416).
MULTI_SCALE_LAMBDA = list(V10_LION_LAMBDA)
# Most Chebyshev coefficients the fixed-coefficient (fast) path evaluates.
MAX_FAST_TERMS = 32

_lut_lock = threading.Lock()
_lut_by_device: dict = {}


def get_chebyshev_lut(device) -> torch.Tensor:
    """The [MAX_DEGREE, LUT_TABLE_SIZE] fp32 Chebyshev half-table on
    ``device`` (T_k on linspace(0, 1, 256), fp32 recurrence), built once per
    device under a lock (sdpc_kernel.py:84-96).  The full path's kernels read
    the same table."""
    key = torch.device(device)
    hit = _lut_by_device.get(key)
    if hit is None:
        with _lut_lock:
            hit = _lut_by_device.get(key)
            if hit is None:
                hit = chebyshev_lut_table().to(key).contiguous()
                _lut_by_device[key] = hit
    return hit


class GatedComplexityPredictor(nn.Module):
    """Global TTT gate from the mean input: Linear(D, D/4), SiLU,
    Linear(D/4, 1), sigmoid (sdpc_kernel.py:1818-1830).  The module layout
    (``net.0``, ``net.2``) is the reference's, so its state_dict entries load."""

    def __init__(self, d_model: int):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(d_model, d_model // 4), nn.SiLU(), nn.Linear(d_model // 4, 1),
                                 nn.Sigmoid())

    def forward(self, x_mean: torch.Tensor) -> torch.Tensor:
        return self.net(x_mean)


def init_chebyshev_coefficients(batch: int, n_heads: int, degree: int, head_dim: int, device) -> torch.Tensor:
    """Initial coefficients [batch, n_heads, degree, head_dim] fp32
    (sdpc_kernel.py:1833-1867).

    One standard-normal draw of that shape (the same call on the torch
    generator as the reference, so a seeded run draws the same numbers),
    scaled per term by sigma_k = 0.1/(k+1).  With two or more heads, each
    batch row's heads are then decorrelated, treating head h as the row
    vector of its degree*head_dim coefficients:

    * degree*head_dim >= n_heads: the rows are replaced by the orthonormal
      basis that QR (Gram-Schmidt order, head 0 first) gives for them, each
      rescaled to its original norm, so the rows become mutually orthogonal
      and keep their lengths;
    * degree*head_dim < n_heads (more heads than dimensions, so no
      orthogonal set exists): the norm-1 rows are replaced by their polar
      factor U V^T (the nearest matrix with orthonormal columns) times
      sqrt(n_heads / (degree*head_dim)), a Parseval tight frame, and each row
      is rescaled to its original norm.
    """
    k = torch.arange(degree, device=device, dtype=torch.float32)
    sigma = (0.1 / (k + 1.0)).view(1, 1, degree, 1)
    coeffs = torch.randn(batch, n_heads, degree, head_dim, device=device) * sigma
    if n_heads < 2:
        return coeffs
    width = degree * head_dim
    rows = coeffs.view(batch, n_heads, width)
    norms = rows.norm(dim=2, keepdim=True)
    if width >= n_heads:
        q, _ = torch.linalg.qr(rows.transpose(1, 2))        # [batch, width, n_heads]
        out = q.transpose(1, 2) * norms
    else:
        unit = rows / (norms + 1e-8)
        u, _, vh = torch.linalg.svd(unit, full_matrices=False)
        out = (u @ vh) * math.sqrt(n_heads / width) * norms
    return out.reshape(batch, n_heads, degree, head_dim)


def v10_damping(n_heads: int, device=None) -> torch.Tensor:
    """Per-head damping hard-coded in the reference kernels (sdpc_kernel.py:1734-1736)."""
    h = torch.arange(n_heads, dtype=torch.float32, device=device)
    return 0.98 - 0.06 * h / n_heads


# The fast path's per-head damping and lambda tensors, built once per
# (device, heads) and (device, heads, momentum) instead of on every call (a
# call with small inputs otherwise spends most of its host time building
# them).  Entries are never dropped (a cached tensor may still be read by a
# launch on another stream); past _CONST_CACHE_MAX entries new values are
# built per call instead.
_const_lock = threading.Lock()
_const_cache: dict = {}
_CONST_CACHE_MAX = 64


def _fast_constants(n_heads: int, device: torch.device, ema_momentum):
    """(damping [H], lam [H]) fp32 on ``device`` for the fast path; a tensor
    ``ema_momentum`` (on the device, not read back) is expanded per call."""
    dev = torch.device(device)
    dkey = ("damping", dev, n_heads)
    if isinstance(ema_momentum, torch.Tensor):
        lkey = None
    else:
        lkey = ("lam", dev, n_heads, float(ema_momentum))
    with _const_lock:
        damping = _const_cache.get(dkey)
        lam = _const_cache.get(lkey) if lkey is not None else None
    if damping is None:
        damping = v10_damping(n_heads, dev)
    if lam is None:
        lam = head_momentum(ema_momentum, n_heads, dev)
    with _const_lock:
        for key, val in ((dkey, damping), (lkey, lam)):
            if key is not None and len(_const_cache) < _CONST_CACHE_MAX:
                _const_cache.setdefault(key, val)
    return damping, lam


def apply_cheby_rkv_v10(x, coeffs, momentum_buf, n_heads=4, base_lr=0.005, ema_momentum=0.9,
                        lion_beta1=0.9, lion_beta2=0.99, lion_wd=0.01, chunk_size=256, use_bf16=False,
                        gate_global=None, dynamic_lambda=None, use_lut=True, seq_threshold=384,
                        lion_max_norm=14.0):
    """Same signature and return convention as the reference:
    returns (out [B,S,D] fp32, coeffs fp32, momentum_buf fp32 or None).
    ``ema_momentum`` may also be a one-element tensor on the device, read
    there by the kernels (the reference takes a Python float, which its
    engine obtains with a host synchronisation, sdpc_engine.py:209).
    ``lion_max_norm`` and ``use_bf16`` are accepted and have no effect, as
    in the reference: its megakernel takes ``max_norm`` (sdpc_kernel.py:1907,
    passed at 2324) and never reads it, and the full path rounds x to bf16
    whatever ``use_bf16`` says (2385)."""
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
    if coeffs.shape[2] > MAX_FAST_TERMS:
        # The reference's PyTorch fast path evaluates any number of terms
        # (sdpc_kernel.py:1751-1776); its Triton kernels and its engine
        # (max_degree <= 8) stop at eight.  Here the fixed-coefficient kernels
        # take up to 32 (more than 8 by Clenshaw).
        raise ValueError(f"the fast path supports at most {MAX_FAST_TERMS} Chebyshev coefficients, "
                         f"got {coeffs.shape[2]}")
    damping, lam = _fast_constants(H, x.device, ema_momentum)
    if torch.is_grad_enabled() and (x.requires_grad or coeffs.requires_grad):
        out = cheby_ema(x, coeffs, damping, lam, out_dtype=torch.float32, nan_policy="zero_u")
    else:
        out = cheby_ema_forward(x, coeffs, damping, lam, out_dtype=torch.float32, nan_policy="zero_u")
    return out, coeffs, momentum_buf


apply_cheby_rkv_core = apply_cheby_rkv_v10


class _FusedClenshawEmaLauncher:
    """``_fused_clenshaw_ema_kernel[grid](...)`` with the reference's argument
    list (sdpc_kernel.py:988-1005): pointer arguments are tensors, written in
    place (XNorm, TanhY, EMAOut, FinalState) as the Triton kernel writes
    through them.  The launch runs ``osm_cheby_ema_lut_fwd`` on the current
    stream; BLOCK_S is the interval at which the carried state is clamped,
    as the kernel's tile carry does (sdpc_kernel.py:1193-1200), and BLOCK_HD
    only shapes the grid, which must be the reference's
    (B * n_heads * ceil(head_dim / BLOCK_HD),).  Strides must be those of the
    tensors passed (the kernel reads through them; other strides raise)."""

    _ARGS = ("X_ptr", "C_ptr", "LUT_ptr", "XNorm_ptr", "TanhY_ptr", "EMAOut_ptr", "InitState_ptr", "FinalState_ptr",
             "seq_len", "total_dim", "head_dim", "n_heads", "degree", "lut_size", "momentum",
             "stride_xb", "stride_xs", "stride_xd",
             "stride_cb", "stride_ch", "stride_cdeg", "stride_cd",
             "stride_lk", "stride_lt",
             "stride_xnb", "stride_xns", "stride_xnd",
             "stride_tyb", "stride_tys", "stride_tyd",
             "stride_ob", "stride_os", "stride_od",
             "stride_sb", "stride_sd",
             "BLOCK_HD", "BLOCK_S", "USE_LUT")

    def __getitem__(self, grid):
        def launch(*args, **kwargs):
            return self._launch(grid, args, kwargs)
        return launch

    def _launch(self, grid, args, kwargs):
        if len(args) > len(self._ARGS):
            raise TypeError(f"_fused_clenshaw_ema_kernel takes {len(self._ARGS)} arguments, got {len(args)}")
        a = dict(zip(self._ARGS, args))
        for k, v in kwargs.items():
            if k not in self._ARGS:
                raise TypeError(f"_fused_clenshaw_ema_kernel got an unexpected argument {k!r}")
            if k in a:
                raise TypeError(f"_fused_clenshaw_ema_kernel got multiple values for {k!r}")
            a[k] = v
        missing = [k for k in self._ARGS if k not in a]
        if missing:
            raise TypeError(f"_fused_clenshaw_ema_kernel is missing {missing}")
        x, c, lut = a["X_ptr"], a["C_ptr"], a["LUT_ptr"]
        S, D, hd, H, K = (int(a[k]) for k in ("seq_len", "total_dim", "head_dim", "n_heads", "degree"))
        if H * hd != D or x.dim() != 3 or x.shape[1] < S or x.shape[2] != D:
            raise ValueError(f"x {tuple(x.shape)} does not match seq_len={S}, n_heads={H}, head_dim={hd}")
        B = x.shape[0]
        block_hd = int(a["BLOCK_HD"])
        g = tuple(grid(dict(a)) if callable(grid) else grid)
        if g[:1] != (B * H * math.ceil(hd / block_hd),) or any(int(v) != 1 for v in g[1:]):
            raise ValueError(f"grid {g} is not the kernel's (B * n_heads * cdiv(head_dim, BLOCK_HD),)")
        if int(a["lut_size"]) != LUT_TABLE_SIZE:
            raise ValueError(f"lut_size={a['lut_size']}: the table has {LUT_TABLE_SIZE} points")
        if not 1 <= K <= MAX_DEGREE or c.shape[2] < K:
            raise ValueError(f"degree={K} outside [1, {MAX_DEGREE}] or beyond the coefficients' {c.shape[2]}")

        def strides_of(t, names):
            got = tuple(int(a[n]) for n in names)
            if got != tuple(t.stride()):
                raise NotImplementedError(f"{names[0][:-1]}*: strides {got} differ from the tensor's {tuple(t.stride())}")

        strides_of(x, ("stride_xb", "stride_xs", "stride_xd"))
        strides_of(c, ("stride_cb", "stride_ch", "stride_cdeg", "stride_cd"))
        strides_of(lut, ("stride_lk", "stride_lt"))
        rows = {"XNorm_ptr": ("stride_xnb", "stride_xns", "stride_xnd"),
                "TanhY_ptr": ("stride_tyb", "stride_tys", "stride_tyd"),
                "EMAOut_ptr": ("stride_ob", "stride_os", "stride_od")}
        for name, st in rows.items():
            strides_of(a[name], st)
        init, fin = a["InitState_ptr"], a["FinalState_ptr"]
        strides_of(init, ("stride_sb", "stride_sd"))
        strides_of(fin, ("stride_sb", "stride_sd"))

        def dest(t, shape):
            # the kernel writes through the caller's pointer: a lane-stride-1
            # view is written directly, anything else via a copy afterwards
            v = t[:, :shape[1]] if len(shape) == 3 else t
            return v if v.stride(-1) == 1 and v.dtype == torch.float32 else None

        xn, ty, out = a["XNorm_ptr"], a["TanhY_ptr"], a["EMAOut_ptr"]
        shp = (B, S, D)
        d_xn, d_ty, d_out, d_fin = dest(xn, shp), dest(ty, shp), dest(out, shp), dest(fin, (B, D))
        r_out, r_xn, r_ty, r_fin = cheby_ema_lut_forward(
            x[:, :S], c[:, :, :K], n_heads=H, ema_momentum=float(a["momentum"]), ema_init=init[:, :D],
            use_lut=bool(a["USE_LUT"]), lut=lut, clamp_tile=int(a["BLOCK_S"]), out=d_out, x_norm=d_xn,
            tanh_y=d_ty, ema_final=d_fin)
        if d_out is None:
            out[:, :S].copy_(r_out)
        if d_xn is None:
            xn[:, :S].copy_(r_xn)
        if d_ty is None:
            ty[:, :S].copy_(r_ty)
        if d_fin is None:
            fin.copy_(r_fin)


# The reference's fused Clenshaw + EMA kernel object (sdpc_kernel.py:988),
# launched as ``_fused_clenshaw_ema_kernel[grid](...)`` (precision_tests.py:61-73).
_fused_clenshaw_ema_kernel = _FusedClenshawEmaLauncher()
