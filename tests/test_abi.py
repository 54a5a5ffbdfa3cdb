"""C-ABI checks that need no GPU: the library loads, exports every function
include/osm.h declares, its struct layout matches the ctypes mirror, and
argument errors come back as status codes before any HIP call."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from orthossm_amd import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "osm.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(osm_\w+)\s*\(", text)))


def test_library_loads_with_matching_abi():
    lib = nat.load()
    assert lib.osm_abi_version() == nat.ABI_VERSION
    assert lib.osm_last_error() == b""


def test_every_declared_function_is_exported():
    lib = nat.load()
    declared = header_functions()
    assert declared == sorted(nat.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


@pytest.mark.parametrize("cls,cname", [(nat.ChebyArgs, "osm_cheby_args"), (nat.BwdArgs, "osm_cheby_bwd_args"),
                                      (nat.V10Args, "osm_v10_args"), (nat.LutFwdArgs, "osm_lut_fwd_args")])
def test_struct_layout_matches_ctypes(cls, cname):
    fields = [f for f, _ in cls._fields_]
    prog = ['#include <stdio.h>', '#include <stddef.h>', '#include "osm.h"', "int main(void){",
            f'printf("%zu\\n", sizeof({cname}));']
    prog += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    prog += ["return 0;}"]
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "p.c"), os.path.join(d, "p")
        open(src, "w").write("\n".join(prog))
        subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), src, "-o", exe], check=True)
        vals = [int(v) for v in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(cls)
    assert len(vals) == len(fields) + 1
    for f, off in zip(fields, vals[1:]):
        assert getattr(cls, f).offset == off, f


def _args(**kw):
    a = nat.ChebyArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.S, a.H, a.hd, a.K = 4, 16384, 8, 64, 8
    a.x = a.out = a.coeffs = a.damping = a.lam = 0x10000   # never dereferenced: every case below is invalid
    a.x_stride_b, a.x_stride_s = 16384 * 512, 512
    a.out_stride_b, a.out_stride_s = 16384 * 512, 512
    a.c_stride_b, a.c_stride_h, a.c_stride_k = 8 * 8 * 64, 8 * 64, 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_workspace_bytes_formula():
    lib = nat.load()
    a = _args()
    # 2048-byte header + one 8-byte word per (lane-block, tile, lane): static
    # lambda uses 512-token tiles of 64-lane lane-blocks (4 x 8 lane-blocks,
    # 32 tiles each at S=16384)
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 2048 + 32 * 32 * 64 * 8
    # dynamic lambda: the same 512-token tiles, two words (A and B) per lane
    a.g = 0x10000
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 2048 + 32 * 32 * 64 * 16
    # more than 8 coefficients, or rows off 4-element boundaries, or a head
    # size that is not a multiple of 4: the one-lane geometry, 128-token tiles
    a.K = 9
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 2048 + 32 * 128 * 64 * 16
    a.K, a.g = 8, None
    a.x_stride_s = 514
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 2048 + 32 * 128 * 64 * 8
    a.x_stride_s, a.hd = 512, 62              # D = 496: 8 lane-blocks per row, the last one partial
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 2048 + 32 * 128 * 64 * 8
    a.hd, a.K = 64, 17                        # the Chebyshev form up to 32 terms: the same geometry
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 2048 + 32 * 128 * 64 * 8
    a.K = 33
    assert lib.osm_workspace_bytes(ctypes.byref(a), 0) == 0


def test_workspace_bytes_without_pointers():
    """A shapes-only forward query with x or out NULL does not know their
    alignment and is sized for the one-lane geometry (128-token tiles), the
    largest: a later call with rows off 4-element boundaries (which takes
    that geometry) fits the workspace so sized."""
    lib = nat.load()
    one_lane = 2048 + 32 * 128 * 64 * 8
    assert lib.osm_workspace_bytes(ctypes.byref(_args(x=0, out=0)), 0) == one_lane
    assert lib.osm_workspace_bytes(ctypes.byref(_args(out=0)), 0) == one_lane
    # a view one element off the 4-element boundary asks for the same size
    assert lib.osm_workspace_bytes(ctypes.byref(_args(x=0x10004)), 0) == one_lane
    assert lib.osm_workspace_bytes(ctypes.byref(_args()), 0) == 2048 + 32 * 32 * 64 * 8


def test_ttt_workspace_bytes_formula():
    """TTT: the forward's header and look-back words for 192-token tiles of
    64 lanes (one word per lane, static lambda), 256-byte aligned, then per
    lane 2K+2 floats per tile (the tile records) and per chunk of 16 tiles
    (their merges), then K floats per lane (the per-launch coefficient
    table), with K padded to 4 or 8, then one word per lane-block (the
    table's form: monomial or Chebyshev)."""
    lib = nat.load()
    a = _args()
    n_lb, n_tiles = 4 * 8, -(-16384 // 192)
    n_chunks = -(-n_tiles // 16)

    def want(kpad, words):
        slots = 2048 + n_lb * n_tiles * 64 * 8 * words
        slots = -(-slots // 256) * 256
        return slots + ((n_lb * n_tiles + n_lb * n_chunks) * (2 * kpad + 2) + n_lb * kpad) * 64 * 4 + n_lb * 4

    assert lib.osm_workspace_bytes(ctypes.byref(a), 1) == want(8, 1)
    a.K = 3
    assert lib.osm_workspace_bytes(ctypes.byref(a), 1) == want(4, 1)
    a.K, a.g = 8, 0x10000
    assert lib.osm_workspace_bytes(ctypes.byref(a), 1) == want(8, 2)


def test_flag_values_match_the_header():
    text = open(os.path.join(ROOT, "include", "osm.h")).read()
    for name in ("NO_CLAMP", "NAN_ZERO_U", "FULL_JACOBIAN", "TIMING_JITTER", "POLL_LIMIT_ZERO"):
        m = re.search(rf"#define OSM_FLAG_{name} (0x[0-9a-fA-F]+)", text)
        assert m and int(m.group(1), 16) == getattr(nat, f"FLAG_{name}"), name
    lib = nat.load()
    # the test aids are accepted by the forward, TTT and backward
    for op in (nat.OP_FWD, nat.OP_TTT, nat.OP_BWD):
        for flag in (nat.FLAG_TIMING_JITTER, nat.FLAG_POLL_LIMIT_ZERO):
            assert lib.osm_workspace_bytes(ctypes.byref(_args(flags=flag)), op) > 0


def test_coefficient_limits_per_entry_point():
    lib = nat.load()
    for K in (9, 16):
        assert lib.osm_workspace_bytes(ctypes.byref(_args(K=K)), nat.OP_FWD) > 0
        assert lib.osm_workspace_bytes(ctypes.byref(_args(K=K)), nat.OP_BWD) > 0
        assert lib.osm_workspace_bytes(ctypes.byref(_args(K=K)), nat.OP_TTT) == 0     # the TTT takes K <= 8
        assert b"TTT" in lib.osm_last_error()
    assert nat.MAX_K == 32 and nat.MAX_K_TTT == 8


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=99), -1),
    (dict(flags=0x100), -1),
    (dict(K=0), -2),
    (dict(K=33), -2),
    (dict(hd=0), -2),
    (dict(H=0), -2),
    (dict(S=-1), -2),
    (dict(x_dtype=7), -3),
    (dict(out_dtype=2), -3),
    (dict(x=0), -1),
    (dict(x=0x10002), -4),          # not aligned to one fp32 element
    (dict(x_stride_s=-512), -4),
    (dict(out_stride_b=-4), -4),
])
def test_argument_errors(kw, code):
    lib = nat.load()
    a = _args(**kw)
    assert lib.osm_cheby_ema_fwd(ctypes.byref(a), None, 0, None) == code
    assert lib.osm_last_error() != b""


def test_workspace_errors():
    lib = nat.load()
    a = _args()
    assert lib.osm_cheby_ema_fwd(ctypes.byref(a), None, 0, None) == -5
    assert lib.osm_cheby_ema_fwd(ctypes.byref(a), ctypes.c_void_p(0x10000), 100, None) == -5
    assert b"needs" in lib.osm_last_error()
    assert lib.osm_cheby_ema_fwd(ctypes.byref(a), ctypes.c_void_p(0x10010), 1 << 30, None) == -5   # misaligned


def test_ttt_argument_errors():
    lib = nat.load()
    a = _args()
    assert lib.osm_cheby_ema_ttt(ctypes.byref(a), None, 0, None, 0, None) == -1        # grad NULL
    assert lib.osm_cheby_ema_ttt(ctypes.byref(a), ctypes.c_void_p(0x10000), 5, None, 0, None) == -1  # target
    assert lib.osm_workspace_bytes(ctypes.byref(a), 1) > lib.osm_workspace_bytes(ctypes.byref(a), 0)


def test_bwd_workspace_bytes_formula():
    lib = nat.load()
    a = _args()
    # 192-token tiles (n_tiles = 86 at S=16384), two look-back words per
    # lane, then K-padded partials per tile.
    slots = (2048 + 32 * 86 * 64 * 16 + 255) // 256 * 256
    assert lib.osm_workspace_bytes(ctypes.byref(a), nat.OP_BWD) == slots + 32 * 86 * 8 * 64 * 4
    # more than 8 coefficients: 96-token tiles (171 at S=16384), 16 padded
    a.K = 12
    slots = (2048 + 32 * 171 * 64 * 16 + 255) // 256 * 256
    assert lib.osm_workspace_bytes(ctypes.byref(a), nat.OP_BWD) == slots + 32 * 171 * 16 * 64 * 4
    # more than 16: 32-token tiles (512 at S=16384), 32 padded
    a.K = 20
    slots = (2048 + 32 * 512 * 64 * 16 + 255) // 256 * 256
    assert lib.osm_workspace_bytes(ctypes.byref(a), nat.OP_BWD) == slots + 32 * 512 * 32 * 64 * 4
    assert lib.osm_workspace_bytes(ctypes.byref(a), 3) == 0
    assert b"osm_op" in lib.osm_last_error()


def _bwd(**kw):
    b = nat.BwdArgs()
    b.grad_out = b.grad_x = 0x10000
    b.go_stride_b = b.gx_stride_b = 16384 * 512
    b.go_stride_s = b.gx_stride_s = 512
    for k, v in kw.items():
        setattr(b, k, v)
    return b


@pytest.mark.parametrize("akw,bkw,code", [
    ({}, dict(grad_out=0), -1),
    ({}, dict(grad_x=0), -1),
    ({}, dict(grad_x=0x10002), -4),          # not aligned to one element
    ({}, dict(go_stride_s=-512), -4),
    ({}, dict(gx_stride_s=256), -4),          # rows overlap
    ({}, dict(gx_stride_b=512), -4),          # batches overlap
    (dict(out=0), {}, -1),                    # the clamp mask needs the saved output
    (dict(out=0, flags=nat.FLAG_NO_CLAMP), {}, -5),   # ... unless there is no clamp: reaches the workspace check
    (dict(K=33), {}, -2),
    (dict(K=9), dict(z_saved=0x20000, z_stride_b=16384 * 512, z_stride_s=512), -1),   # the saved z needs K <= 8
])
def test_bwd_argument_errors(akw, bkw, code):
    lib = nat.load()
    a = _args(**akw)
    b = _bwd(**bkw)
    assert lib.osm_cheby_ema_bwd(ctypes.byref(a), ctypes.byref(b), None, 0, None) == code
    assert lib.osm_last_error() != b""
    assert lib.osm_cheby_ema_bwd(ctypes.byref(_args()), None, None, 0, None) == -1


def _v10(**kw):
    a = nat.V10Args()
    a.abi_version = nat.ABI_VERSION
    a.flags = nat.V10_USE_LUT
    a.B, a.S, a.H, a.hd, a.K, a.chunk = 2, 1000, 4, 16, 8, 256
    a.x = a.out = a.coeffs = a.momentum = a.coeffs_out = a.momentum_out = 0x10000
    a.lut = a.lion_lambda = a.lr_scale = a.spectral_scale = 0x10000
    a.x_stride_b = a.out_stride_b = 1000 * 64
    a.x_stride_s = a.out_stride_s = 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=3), -1),
    (dict(flags=0x10), -1),
    (dict(K=9), -2),
    (dict(chunk=0), -2),
    (dict(S=0), -2),
    (dict(x_dtype=5), -3),
    (dict(lut=0), -1),                 # LUT mode needs the table
    (dict(momentum=0), -1),
    (dict(out_stride_s=32), -4),       # rows overlap
    (dict(x_stride_s=1 << 22), -4),    # 257 rows over 2 GiB
    (dict(ema_momentum_dev=0x10002), -4),   # device momentum not float-aligned
])
def test_v10_argument_errors(kw, code):
    lib = nat.load()
    assert lib.osm_v10_chunked_ttt(ctypes.byref(_v10(**kw)), None) == code
    assert lib.osm_last_error() != b""


def _lut(**kw):
    a = nat.LutFwdArgs()
    a.abi_version = nat.ABI_VERSION
    a.flags = nat.V10_USE_LUT
    a.B, a.S, a.H, a.hd, a.K, a.clamp_tile = 2, 256, 8, 8, 4, 128
    a.x = a.out = a.coeffs = a.lut = 0x10000
    a.x_stride_b = a.out_stride_b = 256 * 64
    a.x_stride_s = a.out_stride_s = 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=3), -1),
    (dict(flags=0x10), -1),
    (dict(K=9), -2),
    (dict(K=0), -2),
    (dict(clamp_tile=8), -2),          # the carried state is clamped between waves of 16 tokens
    (dict(clamp_tile=40), -2),
    (dict(x_dtype=5), -3),
    (dict(lut=0), -1),                 # LUT mode needs the table
    (dict(out=0), -1),
    (dict(out_stride_s=32), -4),       # rows overlap
    (dict(x_norm=0x10000, xn_stride_b=256 * 64, xn_stride_s=32), -4),
    (dict(tanh_y=0x10002, ty_stride_b=256 * 64, ty_stride_s=64), -4),   # misaligned
    (dict(ema_final=0x10000, final_stride_b=32), -4),                   # final rows overlap
    (dict(x_stride_s=1 << 22), -4),    # 257 rows over 2 GiB
])
def test_lut_fwd_argument_errors(kw, code):
    lib = nat.load()
    assert lib.osm_cheby_ema_lut_fwd(ctypes.byref(_lut(**kw)), None) == code
    assert lib.osm_last_error() != b""
    assert lib.osm_cheby_ema_lut_fwd(None, None) == -1


def test_lut_fwd_empty_batch_is_a_no_op():
    # B = 0 returns before any pointer is looked at (no GPU work)
    lib = nat.load()
    assert lib.osm_cheby_ema_lut_fwd(ctypes.byref(_lut(B=0, x=0, out=0, coeffs=0)), None) == 0


def test_error_messages_are_thread_local():
    import threading
    lib = nat.load()
    a = _args(K=33)
    assert lib.osm_cheby_ema_fwd(ctypes.byref(a), None, 0, None) == -2
    seen = []
    t = threading.Thread(target=lambda: seen.append(lib.osm_last_error()))
    t.start()
    t.join()
    assert seen == [b""] and b"K=33" in lib.osm_last_error()


def _doc_struct(name):
    """The ctypes structure `name` from the binding stubs of the integration guide."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(rf"^class {name}\(ctypes\.Structure\):.*?\]\n", text, flags=re.S | re.M)
    assert m, f"{name} not found in INTEGRATION.md"
    ns = {"ctypes": ctypes}
    exec(m.group(0), ns)
    return ns[name]


@pytest.mark.parametrize("doc_name,cls", [("_Args", nat.ChebyArgs), ("_BwdArgs", nat.BwdArgs)])
def test_integration_stub_structs_match_the_header(doc_name, cls):
    # the stubs a maintainer would paste must lay the structs out as osm.h does
    doc = _doc_struct(doc_name)
    assert ctypes.sizeof(doc) == ctypes.sizeof(cls)
    assert [f for f, _ in doc._fields_] == [f for f, _ in cls._fields_]
    for f, _ in cls._fields_:
        assert getattr(doc, f).offset == getattr(cls, f).offset, f
