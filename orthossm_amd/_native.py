"""ctypes binding of the C ABI declared in ``include/osm.h``.

The shared library is built in-tree by ``orthossm_amd.build`` into
``orthossm_amd/_lib/libosm.so``.  There is no fallback: if the library is
missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libosm.so")

ABI_VERSION = 2
MAX_K = 32       # forward and backward
MAX_K_TTT = 8    # the TTT gradient
MAX_K_V10 = 8    # the full path's series (coefficients past it pass through)
F32 = 0
BF16 = 1
FLAG_NO_CLAMP = 0x1
FLAG_NAN_ZERO_U = 0x2
FLAG_FULL_JACOBIAN = 0x4
FLAG_TIMING_JITTER = 0x8   # test aid: pseudo-random delays before look-back publishes
FLAG_POLL_LIMIT_ZERO = 0x10   # test aid: a look-back wait gives up at its first unpublished read
TARGET_X = 0
TARGET_SOFTSIGN = 1
OP_FWD = 0
OP_TTT = 1
OP_BWD = 2
V10_USE_LUT = 0x1

STATUS = {
    0: "OSM_OK",
    -1: "OSM_E_ARG",
    -2: "OSM_E_SHAPE",
    -3: "OSM_E_DTYPE",
    -4: "OSM_E_LAYOUT",
    -5: "OSM_E_WORKSPACE",
    -6: "OSM_E_HIP",
    -7: "OSM_E_FAULT",
}
# Raised by the Python layer (not returned by the library) when a workspace's
# fault word shows that a launch's look-back wait gave up.
OSM_E_FAULT = -7

# Every function the header declares; tests check the library exports each.
EXPORTS = (
    "osm_abi_version",
    "osm_last_error",
    "osm_workspace_bytes",
    "osm_workspace_init",
    "osm_workspace_status",
    "osm_cheby_ema_fwd",
    "osm_cheby_ema_fwd_static",
    "osm_cheby_ema_ttt",
    "osm_cheby_ema_bwd",
    "osm_v10_chunked_ttt",
    "osm_cheby_ema_lut_fwd",
)


class ChebyArgs(ctypes.Structure):
    """Mirror of ``osm_cheby_args`` (same field order and C types)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("B", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("hd", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int32),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_s", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int32),
        ("out_stride_b", ctypes.c_int64),
        ("out_stride_s", ctypes.c_int64),
        ("coeffs", ctypes.c_void_p),
        ("c_stride_b", ctypes.c_int64),
        ("c_stride_h", ctypes.c_int64),
        ("c_stride_k", ctypes.c_int64),
        ("damping", ctypes.c_void_p),
        ("lam", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("g_stride_b", ctypes.c_int64),
        ("g_stride_s", ctypes.c_int64),
        ("g_stride_h", ctypes.c_int64),
        ("lam_shift", ctypes.c_float),
        ("lam_min", ctypes.c_float),
        ("lam_max", ctypes.c_float),
        ("ema_init", ctypes.c_void_p),
        ("ema_final", ctypes.c_void_p),
    ]


class BwdArgs(ctypes.Structure):
    """Mirror of ``osm_cheby_bwd_args``."""

    _fields_ = [
        ("grad_out", ctypes.c_void_p),
        ("go_stride_b", ctypes.c_int64),
        ("go_stride_s", ctypes.c_int64),
        ("grad_state", ctypes.c_void_p),
        ("grad_x", ctypes.c_void_p),
        ("gx_stride_b", ctypes.c_int64),
        ("gx_stride_s", ctypes.c_int64),
        ("grad_coeffs", ctypes.c_void_p),
        ("grad_init", ctypes.c_void_p),
        ("z_saved", ctypes.c_void_p),
        ("z_stride_b", ctypes.c_int64),
        ("z_stride_s", ctypes.c_int64),
    ]


class V10Args(ctypes.Structure):
    """Mirror of ``osm_v10_args``."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("B", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("hd", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("chunk", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int32),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_s", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("out_stride_b", ctypes.c_int64),
        ("out_stride_s", ctypes.c_int64),
        ("coeffs", ctypes.c_void_p),
        ("c_stride_b", ctypes.c_int64),
        ("c_stride_h", ctypes.c_int64),
        ("c_stride_k", ctypes.c_int64),
        ("momentum", ctypes.c_void_p),
        ("m_stride_b", ctypes.c_int64),
        ("m_stride_h", ctypes.c_int64),
        ("m_stride_k", ctypes.c_int64),
        ("coeffs_out", ctypes.c_void_p),
        ("momentum_out", ctypes.c_void_p),
        ("lut", ctypes.c_void_p),
        ("lion_lambda", ctypes.c_void_p),
        ("lr_scale", ctypes.c_void_p),
        ("spectral_scale", ctypes.c_void_p),
        ("gate", ctypes.c_void_p),
        ("dyn_lambda", ctypes.c_void_p),
        ("ema_momentum", ctypes.c_float),
        ("base_lr", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("z_save", ctypes.c_void_p),
        ("z_stride_b", ctypes.c_int64),
        ("z_stride_s", ctypes.c_int64),
        ("coeff_hist", ctypes.c_void_p),
        ("ema_momentum_dev", ctypes.c_void_p),
    ]


class LutFwdArgs(ctypes.Structure):
    """Mirror of ``osm_lut_fwd_args``."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("B", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("hd", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("clamp_tile", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int32),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_s", ctypes.c_int64),
        ("coeffs", ctypes.c_void_p),
        ("c_stride_b", ctypes.c_int64),
        ("c_stride_h", ctypes.c_int64),
        ("c_stride_k", ctypes.c_int64),
        ("lut", ctypes.c_void_p),
        ("ema_momentum", ctypes.c_float),
        ("ema_init", ctypes.c_void_p),
        ("init_stride_b", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("out_stride_b", ctypes.c_int64),
        ("out_stride_s", ctypes.c_int64),
        ("x_norm", ctypes.c_void_p),
        ("xn_stride_b", ctypes.c_int64),
        ("xn_stride_s", ctypes.c_int64),
        ("tanh_y", ctypes.c_void_p),
        ("ty_stride_b", ctypes.c_int64),
        ("ty_stride_s", ctypes.c_int64),
        ("ema_final", ctypes.c_void_p),
        ("final_stride_b", ctypes.c_int64),
    ]


class OsmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Loads libosm.so (once) and declares the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"orthossm_amd: native library {LIB_PATH} is missing; build it with "
                "`python -m orthossm_amd.build` (hipcc, gfx950). There is no CPU fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        lib.osm_abi_version.restype = ctypes.c_int
        lib.osm_abi_version.argtypes = []
        lib.osm_last_error.restype = ctypes.c_char_p
        lib.osm_last_error.argtypes = []
        lib.osm_workspace_bytes.restype = ctypes.c_size_t
        lib.osm_workspace_bytes.argtypes = [ctypes.POINTER(ChebyArgs), ctypes.c_int]
        lib.osm_workspace_init.restype = ctypes.c_int
        lib.osm_workspace_init.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.osm_workspace_status.restype = ctypes.c_int
        lib.osm_workspace_status.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        lib.osm_cheby_ema_fwd.restype = ctypes.c_int
        lib.osm_cheby_ema_fwd.argtypes = [ctypes.POINTER(ChebyArgs), ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p]
        lib.osm_cheby_ema_fwd_static.restype = ctypes.c_int
        lib.osm_cheby_ema_fwd_static.argtypes = [ctypes.POINTER(ChebyArgs), ctypes.c_void_p]
        lib.osm_cheby_ema_ttt.restype = ctypes.c_int
        lib.osm_cheby_ema_ttt.argtypes = [ctypes.POINTER(ChebyArgs), ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.osm_cheby_ema_bwd.restype = ctypes.c_int
        lib.osm_cheby_ema_bwd.argtypes = [ctypes.POINTER(ChebyArgs), ctypes.POINTER(BwdArgs), ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_void_p]
        lib.osm_v10_chunked_ttt.restype = ctypes.c_int
        lib.osm_v10_chunked_ttt.argtypes = [ctypes.POINTER(V10Args), ctypes.c_void_p]
        lib.osm_cheby_ema_lut_fwd.restype = ctypes.c_int
        lib.osm_cheby_ema_lut_fwd.argtypes = [ctypes.POINTER(LutFwdArgs), ctypes.c_void_p]
        got = lib.osm_abi_version()
        if got != ABI_VERSION:
            raise ImportError(f"orthossm_amd: library ABI {got} != binding ABI {ABI_VERSION}; rebuild")
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != 0:
        raise OsmError(rc, load().osm_last_error().decode(errors="replace"))
