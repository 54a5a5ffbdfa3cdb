"""Torch-facing operators over the C ABI (HIP kernels on gfx950).

``cheby_ema_forward``  fused forward (static or dynamic lambda, EMA carry).
``cheby_ema_ttt``      fused forward + TTT coefficient gradient.

Both run on the current torch stream of the input's device and never
synchronise the host.  Inputs are not modified.  There is no CPU path: a
tensor that is not on a ROCm device raises.
"""
from __future__ import annotations

import ctypes
import threading
from typing import Sequence

import torch

from . import _native as nat

_ws_lock = threading.Lock()
_ws_cache: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Zero-initialised workspace reused per (device, stream).  Calls on one
    stream are ordered, so they never overlap on a workspace."""
    key = (device.index, stream)
    with _ws_lock:
        ws = _ws_cache.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, 1 << 20)
            size = (size + (1 << 20) - 1) & ~((1 << 20) - 1)
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
            _ws_cache[key] = ws
        return ws


def _as_param(v, H: int, device, name: str) -> torch.Tensor:
    t = v if isinstance(v, torch.Tensor) else torch.as_tensor(v, dtype=torch.float32)
    t = t.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if t.numel() != H:
        raise ValueError(f"{name} must have H={H} entries, got {t.numel()}")
    return t


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return nat.F32
    if dt == torch.bfloat16:
        return nat.BF16
    raise TypeError(f"unsupported dtype {dt}; use float32 or bfloat16")


def _prepare(x, coeffs, damping, lam, g, lam_shift, lam_min, lam_max, ema_init, clamp, out_dtype, out,
             nan_policy="zero_z"):
    if not isinstance(x, torch.Tensor) or x.dim() != 3:
        raise ValueError("x must be a [B,S,D] tensor")
    if x.device.type != "cuda":
        raise RuntimeError("orthossm_amd runs on a ROCm GPU only; x is on " + str(x.device))
    dev = x.device
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    if x.stride(2) != 1 or x.stride(1) % 4 or x.stride(0) % 4 or x.data_ptr() % (4 * x.element_size()):
        x = x.contiguous()
    B, S, D = x.shape
    if coeffs.dim() != 4:
        raise ValueError("coeffs must be [B,H,K,hd]")
    Bc, H, K, hd = coeffs.shape
    if Bc != B or H * hd != D:
        raise ValueError(f"coeffs {tuple(coeffs.shape)} does not match x {tuple(x.shape)}")
    c = coeffs.to(device=dev, dtype=torch.float32)
    if c.stride(3) != 1:
        c = c.contiguous()
    damp = _as_param(damping, H, dev, "damping")
    lamt = _as_param(lam, H, dev, "lam")
    gt = None
    if g is not None:
        gt = g.to(device=dev, dtype=torch.float32)
        if gt.dim() == 2:
            gt = gt.unsqueeze(0).expand(B, S, H)
        if tuple(gt.shape) != (B, S, H):
            raise ValueError(f"g must be [S,H] or [B,S,H], got {tuple(g.shape)}")
    init = None
    if ema_init is not None:
        init = ema_init.to(device=dev, dtype=torch.float32).reshape(B, D).contiguous()
    odt = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((B, S, D), device=dev, dtype=odt)
    elif tuple(out.shape) != (B, S, D) or out.dtype != odt or out.device != dev:
        raise ValueError("out has the wrong shape, dtype or device")
    if out.stride(2) != 1 or out.stride(1) % 4 or out.stride(0) % 4 or out.data_ptr() % (4 * out.element_size()):
        raise ValueError("out must have a contiguous lane dimension and 4-element aligned rows")
    a = nat.ChebyArgs()
    a.abi_version = nat.ABI_VERSION
    if nan_policy not in ("zero_z", "zero_u"):
        raise ValueError("nan_policy must be 'zero_z' or 'zero_u'")
    a.flags = (0 if clamp else nat.FLAG_NO_CLAMP) | (nat.FLAG_NAN_ZERO_U if nan_policy == "zero_u" else 0)
    a.B, a.S, a.H, a.hd, a.K = B, S, H, hd, K
    a.x, a.x_dtype, a.x_stride_b, a.x_stride_s = x.data_ptr(), _dtype_code(x.dtype), x.stride(0), x.stride(1)
    a.out, a.out_dtype = out.data_ptr(), _dtype_code(out.dtype)
    a.out_stride_b, a.out_stride_s = out.stride(0), out.stride(1)
    a.coeffs, a.c_stride_b, a.c_stride_h, a.c_stride_k = c.data_ptr(), c.stride(0), c.stride(1), c.stride(2)
    a.damping, a.lam = damp.data_ptr(), lamt.data_ptr()
    if gt is not None:
        a.g, a.g_stride_b, a.g_stride_s, a.g_stride_h = gt.data_ptr(), gt.stride(0), gt.stride(1), gt.stride(2)
    a.lam_shift, a.lam_min, a.lam_max = float(lam_shift), float(lam_min), float(lam_max)
    a.ema_init = init.data_ptr() if init is not None else None
    keep = (x, c, damp, lamt, gt, init)  # keeps every pointed-to tensor alive across the call
    return a, out, keep


def cheby_ema_forward(x: torch.Tensor, coeffs: torch.Tensor, damping: Sequence[float] | torch.Tensor,
                      lam: Sequence[float] | torch.Tensor, *, g: torch.Tensor | None = None,
                      lam_shift: float = 0.004, lam_min: float = 0.9, lam_max: float = 0.9999,
                      ema_init: torch.Tensor | None = None, clamp: bool = True,
                      out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
                      return_state: bool = False, state_out: torch.Tensor | None = None,
                      nan_policy: str = "zero_z"):
    """Fused softsign -> Clenshaw -> damping -> tanh -> EMA on the GPU.

    x [B,S,D] fp32|bf16, coeffs [B,H,K,hd] fp32, damping/lam [H], g optional
    [S,H] or [B,S,H] (dynamic lambda), ema_init optional [B,D].
    Returns out [B,S,D] (dtype of x unless out_dtype), and ema_final [B,D]
    fp32 when return_state.  ``state_out`` (contiguous [B,D] fp32 on the
    device) receives ema_final instead of a new tensor.  ``nan_policy``: a
    NaN input gives z = 0 ('zero_z', the reference's Triton kernels) or counts
    as u = 0 ('zero_u', the reference's PyTorch fast path).
    """
    lib = nat.load()
    a, out, keep = _prepare(x, coeffs, damping, lam, g, lam_shift, lam_min, lam_max, ema_init, clamp,
                            out_dtype, out, nan_policy)
    dev = out.device
    ema_final = _state_buffer(a, dev, return_state, state_out)
    stream = torch.cuda.current_stream(dev).cuda_stream
    nbytes = lib.osm_workspace_bytes(ctypes.byref(a), 0)
    if nbytes == 0:
        nat.check(_rc_from_error(lib, a, 0))
    ws = _workspace(dev, stream, nbytes)
    nat.check(lib.osm_cheby_ema_fwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                    ctypes.c_void_p(stream)))
    del keep
    return (out, ema_final) if return_state else out


def cheby_ema_ttt(x: torch.Tensor, coeffs: torch.Tensor, damping, lam, *, g: torch.Tensor | None = None,
                  lam_shift: float = 0.004, lam_min: float = 0.9, lam_max: float = 0.9999,
                  ema_init: torch.Tensor | None = None, target: str = "x", clamp: bool = True,
                  out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
                  return_state: bool = False, state_out: torch.Tensor | None = None,
                  grad_out: torch.Tensor | None = None, nan_policy: str = "zero_z"):
    """Fused forward plus the TTT coefficient gradient
    grad[b,h,k,j] = d/dc MSE(out[:, :-1], y[:, 1:]) / (k+1)^2, y = x ('x') or
    softsign(x) ('softsign').  Returns (out, grad) or (out, grad, ema_final).
    ``grad_out`` (contiguous [B,H,K,hd] fp32) and ``state_out`` receive the
    results instead of new tensors."""
    lib = nat.load()
    tgt = {"x": nat.TARGET_X, "softsign": nat.TARGET_SOFTSIGN}.get(target)
    if tgt is None:
        raise ValueError("target must be 'x' or 'softsign'")
    a, out, keep = _prepare(x, coeffs, damping, lam, g, lam_shift, lam_min, lam_max, ema_init, clamp,
                            out_dtype, out, nan_policy)
    dev = out.device
    if grad_out is None:
        grad = torch.empty((a.B, a.H, a.K, a.hd), device=dev, dtype=torch.float32)
    else:
        _check_dest(grad_out, (a.B, a.H, a.K, a.hd), dev, "grad_out")
        grad = grad_out
    ema_final = _state_buffer(a, dev, return_state, state_out)
    stream = torch.cuda.current_stream(dev).cuda_stream
    nbytes = lib.osm_workspace_bytes(ctypes.byref(a), 1)
    if nbytes == 0:
        nat.check(_rc_from_error(lib, a, 1))
    ws = _workspace(dev, stream, nbytes)
    nat.check(lib.osm_cheby_ema_ttt(ctypes.byref(a), ctypes.c_void_p(grad.data_ptr()), tgt,
                                    ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(stream)))
    del keep
    return (out, grad, ema_final) if return_state else (out, grad)


def _check_dest(t: torch.Tensor, shape, dev, name: str) -> None:
    if t.dtype != torch.float32 or tuple(t.shape) != tuple(shape) or t.device != dev or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor of shape {tuple(shape)} on {dev}")


def _state_buffer(a, dev, return_state: bool, state_out: torch.Tensor | None):
    """ema_final destination: state_out if given, a new [B,D] tensor if
    return_state, else none (the kernel then skips the store)."""
    if state_out is not None:
        _check_dest(state_out, (a.B, a.H * a.hd), dev, "state_out")
        buf = state_out
    elif return_state:
        buf = torch.empty((a.B, a.H * a.hd), device=dev, dtype=torch.float32)
    else:
        buf = None
    a.ema_final = buf.data_ptr() if buf is not None else None
    return buf


def _rc_from_error(lib, a, ttt: int) -> int:
    """osm_workspace_bytes returned 0: re-run validation through the entry
    point with no workspace to obtain the status code and message."""
    if ttt:
        return lib.osm_cheby_ema_ttt(ctypes.byref(a), None, 0, None, 0, None)
    return lib.osm_cheby_ema_fwd(ctypes.byref(a), None, 0, None)
