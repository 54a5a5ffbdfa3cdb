"""osm_cheby_ema_fwd_static (the forward with its look-back workspace in the
library's static device array, no allocation) through the C ABI: the same
bits as osm_cheby_ema_fwd with a caller workspace on two calls in a row, the
second with a smaller input, static and dynamic lambda, with the EMA carry;
a seeded sequence of twelve calls of changing layouts gives the same bits
as well; its fault word (osm_workspace_status with a NULL workspace) stays
zero; a shape whose workspace exceeds the static array is refused before
any launch."""
import ctypes

import pytest
import torch

from helpers import inputs, to_dev
from orthossm_amd import _native as nat
from orthossm_amd import ops

pytestmark = pytest.mark.gpu

STATIC_BYTES = 32 << 20


def args_for(d, out, fin, init):
    """osm_cheby_args for the inputs d (on the device), output out and state
    buffers, built as ops does."""
    a, _, keep = ops._prepare(d["x"], d["coeffs"], d["damping"], d["lam"], d.get("g"), 0.004, 0.9, 0.9999, init,
                              True, out.dtype, out)
    a.ema_final = fin.data_ptr()
    return a, keep


def run_both(lib, dev, d, init):
    stream = torch.cuda.current_stream(dev).cuda_stream
    B, S, D = d["x"].shape
    out_s = torch.full((B, S, D), float("nan"), device=dev)
    out_w = torch.full((B, S, D), float("nan"), device=dev)
    fin_s = torch.full((B, D), float("nan"), device=dev)
    fin_w = torch.full((B, D), float("nan"), device=dev)
    a_s, keep_s = args_for(d, out_s, fin_s, init)
    a_w, keep_w = args_for(d, out_w, fin_w, init)
    nat.check(lib.osm_cheby_ema_fwd_static(ctypes.byref(a_s), ctypes.c_void_p(stream)))
    nbytes = lib.osm_workspace_bytes(ctypes.byref(a_w), nat.OP_FWD)
    assert 0 < nbytes <= STATIC_BYTES
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    nat.check(lib.osm_cheby_ema_fwd(ctypes.byref(a_w), ctypes.c_void_p(ws.data_ptr()), nbytes,
                                    ctypes.c_void_p(stream)))
    torch.cuda.synchronize()
    del keep_s, keep_w
    return (out_s, fin_s), (out_w, fin_w)


def static_status(lib, dev):
    st = torch.full((2,), -1, dtype=torch.int32, device=dev)
    nat.check(lib.osm_workspace_status(None, ctypes.c_void_p(st.data_ptr()), 0,
                                       ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    return [int(v) & 0xFFFFFFFF for v in st.cpu().tolist()]


@pytest.mark.parametrize("dynamic", [False, True])
def test_static_scratch_matches_workspace_entry_point(dev, dynamic):
    lib = nat.load()
    # two calls in a row, the second with a smaller input (another layout)
    for B, S, seed in ((3, 9000, 70), (1, 2500, 71)):
        inp = inputs(B, S, 8, 64, seed=seed + dynamic, dynamic=dynamic)
        d = to_dev(inp, dev)
        init = (torch.rand(B, 512, generator=torch.Generator().manual_seed(seed)) - 0.5).to(dev)
        (out_s, fin_s), (out_w, fin_w) = run_both(lib, dev, d, init)
        assert not torch.isnan(out_s).any()
        assert torch.equal(out_s, out_w), (B, S)
        assert torch.equal(fin_s, fin_w), (B, S)
    fault, launches = static_status(lib, dev)
    assert fault == 0 and launches >= 2


def test_static_scratch_repeated_same_layout(dev):
    lib = nat.load()
    d = to_dev(inputs(2, 4000, 8, 64, seed=72), dev)
    first = None
    for _ in range(3):
        (out_s, fin_s), (out_w, _) = run_both(lib, dev, d, None)
        assert torch.equal(out_s, out_w)
        if first is None:
            first = out_s.clone()
        assert torch.equal(out_s, first)
    assert static_status(lib, dev)[0] == 0


def test_static_scratch_refuses_shapes_beyond_its_size(dev):
    lib = nat.load()
    # dynamic lambda, 64 lanes, 512-token tiles: 1.7e7 tokens need 33204 tiles
    # x 64 lanes x 2 words x 8 bytes > 32 MiB of look-back words.  x and g
    # are broadcast (stride 0); out is real memory, so nothing could go out
    # of bounds even if the size check were missing.
    S, H, hd = 17_000_000, 1, 64
    x = torch.randn(1, 1, H * hd, device=dev).to(torch.bfloat16).expand(1, S, H * hd)
    out = torch.empty(1, S, H * hd, device=dev, dtype=torch.bfloat16)
    g = torch.zeros(1, 1, H, device=dev).expand(1, S, H)
    c = torch.zeros(1, H, 8, hd, device=dev)
    lam = torch.full((H,), 0.9, device=dev)
    a, _, keep = ops._prepare(x, c, lam, lam, g, 0.004, 0.9, 0.9999, None, True, torch.bfloat16, out)
    assert lib.osm_workspace_bytes(ctypes.byref(a), nat.OP_FWD) > STATIC_BYTES
    out.fill_(7.0)
    rc = lib.osm_cheby_ema_fwd_static(ctypes.byref(a), None)
    assert rc == -5 and b"static scratch" in lib.osm_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())          # nothing was launched
    del keep


def test_static_scratch_random_sequence_of_layouts(dev):
    """A seeded sequence of calls whose layouts change from call to call
    (batch, length, heads, head size, terms, static or dynamic lambda, an
    initial state): every call gives the bits of the workspace entry point."""
    import numpy as np

    lib = nat.load()
    r = np.random.default_rng(73)
    for i in range(12):
        H = int(r.choice((1, 2, 4, 8)))
        hd = int(r.choice((8, 16, 32, 64)))
        B = int(r.integers(1, 4))
        S = int(r.integers(1, 6000))
        K = int(r.integers(1, 9))
        dyn = bool(r.random() < 0.4)
        d = to_dev(inputs(B, S, H, hd, K, seed=100 + i, dynamic=dyn), dev)
        init = None
        if r.random() < 0.5:
            init = (torch.rand(B, H * hd, generator=torch.Generator().manual_seed(i)) - 0.5).to(dev)
        (out_s, fin_s), (out_w, fin_w) = run_both(lib, dev, d, init)
        assert torch.equal(out_s, out_w), (i, B, S, H, hd, K, dyn)
        assert torch.equal(fin_s, fin_w), (i, B, S, H, hd, K, dyn)
    assert static_status(lib, dev)[0] == 0
