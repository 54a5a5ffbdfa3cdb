"""The workspace's fault word through the C ABI (osm_workspace_status): zero
after ordinary launches, a launch counter that grows by one per launch and
keeps growing across a layout change, and a fault left by an earlier launch
(planted from the host into the header) that is reported, that raises under
the per-launch check, and that does not disturb later launches; and a
launch whose look-back waits give up (forced from the host with
OSM_FLAG_POLL_LIMIT_ZERO), which leaves NaN in the outputs that depend on
the lost values instead of plausible numbers."""
import numpy as np
import pytest
import torch

from helpers import assert_close_fp32, inputs, oracle_forward, to_dev
from orthossm_amd import _native as nat
from orthossm_amd import cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt, ops

pytestmark = pytest.mark.gpu


def _fwd_ws(dev):
    stream = torch.cuda.current_stream(dev).cuda_stream
    return ops._ws_cache[(dev.index, stream, nat.OP_FWD)]


def test_counter_grows_and_no_fault(dev):
    inp = inputs(2, 5000, 8, 64, seed=50)
    d = to_dev(inp, dev)
    cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
    ws = _fwd_ws(dev)
    f0, e0 = ops.workspace_status(ws)
    for _ in range(3):
        cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
    f1, e1 = ops.workspace_status(ws)
    assert (f0, f1) == (0, 0)
    assert e1 == e0 + 3
    # another (smaller) layout on the same workspace: its look-back words are
    # cleared, the counter is not reset
    cheby_ema_forward(d["x"][:1, :2000], d["coeffs"][:1], d["damping"], d["lam"])
    f2, e2 = ops.workspace_status(ws)
    assert f2 == 0 and e2 == e1 + 1


def test_planted_old_fault_is_reported_and_harmless(dev):
    inp = inputs(2, 5000, 8, 64, seed=51)
    d = to_dev(inp, dev)
    want = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
    ws = _fwd_ws(dev)
    _, epoch = ops.workspace_status(ws)
    # the fault tag an earlier launch would have left: (epoch << 2) | 3
    tag = (((epoch - 1) & 0x3FFFFFFF) << 2) | 3
    torch.cuda.synchronize()
    ws.view(torch.int32)[3] = tag - (1 << 32) if tag >= (1 << 31) else tag
    # later launches are not disturbed by it (their waits give up only on
    # their own launch's tag) ...
    for _ in range(3):
        got = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
        assert torch.equal(got, want)
    assert_close_fp32(got.cpu().numpy(), oracle_forward(inp)[0])
    # ... the word stays until read with reset ...
    assert ops.workspace_status(ws) == (tag, epoch + 3)
    # ... and the per-launch check raises on it, clearing it
    old = ops.set_fault_check(True)
    try:
        with pytest.raises(nat.OsmError, match="look-back wait gave up"):
            cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
        got = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])   # cleared: passes
    finally:
        ops.set_fault_check(old)
    assert torch.equal(got, want)
    assert ops.workspace_status(ws)[0] == 0


def test_status_argument_errors(dev):
    lib = nat.load()
    import ctypes
    st = torch.empty(2, dtype=torch.int32, device=dev)
    ws = torch.zeros(4096, dtype=torch.uint8, device=dev)
    assert lib.osm_workspace_status(ctypes.c_void_p(ws.data_ptr() + 4), ctypes.c_void_p(st.data_ptr()), 0,
                                    None) == -5
    assert lib.osm_workspace_status(ctypes.c_void_p(ws.data_ptr()), None, 0, None) == -1


def _equal_or_nan(got, want, what):
    """Every element of `got` is NaN or bit-equal to `want`; returns the NaN mask."""
    g = got.float().cpu().numpy()
    w = want.float().cpu().numpy()
    nan = np.isnan(g)
    assert not np.isnan(w).any(), f"{what}: the reference launch has NaN"
    assert np.array_equal(g[~nan].view(np.uint32), w[~nan].view(np.uint32)), \
        f"{what}: an element that is not NaN differs from the normal launch"
    return nan


def _run_case(case, d, dev):
    """One launch of `case`; returns (tensors, workspace op)."""
    if case == "fwd_static":
        out, fin = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], return_state=True)
        return (out, fin), nat.OP_FWD
    if case == "fwd_dynamic":
        out, fin = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], g=d["g"], return_state=True)
        return (out, fin), nat.OP_FWD
    if case == "ttt":
        out, grad = cheby_ema_ttt(d["x"], d["coeffs"], d["damping"], d["lam"], g=d.get("g"))
        return (out, grad), nat.OP_TTT
    out = d["out_saved"]
    gx, gc, gi = cheby_ema_backward(d["x"], d["coeffs"], d["damping"], d["lam"], out, d["go"], need_init=True)
    return (gx, gc, gi), nat.OP_BWD


@pytest.mark.parametrize("case", ["fwd_static", "fwd_dynamic", "ttt", "bwd"])
def test_poll_limit_zero_poisons_the_dependent_outputs(dev, case):
    """OSM_FLAG_POLL_LIMIT_ZERO (with the timing jitter, so that tiles
    publish late): a look-back word not yet published at its first read
    gives up at once, as a wait past its poll limit does.  Every kernel
    exits; the fault word holds the launch's fault tag; each output element
    is NaN or bit-equal to a normal launch's (outputs downstream of a lost
    carry are NaN, the rest unaffected); the next normal launch is clean."""
    dyn = case == "fwd_dynamic"
    B, S = (2, 40000) if case.startswith("fwd") else (2, 24000)
    inp = inputs(B, S, 8, 64, seed=60, dynamic=dyn)
    d = to_dev(inp, dev)
    if case == "bwd":
        d["out_saved"] = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
        d["go"] = torch.randn(B, S, 512, generator=torch.Generator().manual_seed(61)).to(dev)
    ref, op = _run_case(case, d, dev)
    ref = [t.clone() for t in ref]
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = ops._ws_cache[(dev.index, stream, op)]
    assert ops.workspace_status(ws)[0] == 0
    old_j, old_p = ops.set_timing_jitter(True), ops.set_poll_limit_zero(True)
    try:
        # a give-up depends on timing: up to four launches until one happens
        for _ in range(4):
            _, epoch = ops.workspace_status(ws)
            got, _ = _run_case(case, d, dev)
            fault, _ = ops.workspace_status(ws, reset=True)
            if fault:
                break
    finally:
        ops.set_timing_jitter(old_j)
        ops.set_poll_limit_zero(old_p)
    assert fault == (((epoch & 0x3FFFFFFF) << 2) | 3), f"fault word {fault:#x} after launch {epoch}"
    masks = [_equal_or_nan(g, w, f"{case}[{i}]") for i, (g, w) in enumerate(zip(got, ref))]
    assert masks[0].any(), "the fault word is set but no output is NaN"
    print(f"{case}: {masks[0].mean():.4f} of the first output NaN", flush=True)
    # the next launch is clean and equal to the normal one
    again, _ = _run_case(case, d, dev)
    for i, (g, w) in enumerate(zip(again, ref)):
        assert torch.equal(g, w), f"{case}[{i}] after the poisoned launch"
    assert ops.workspace_status(ws)[0] == 0


def test_status_read_on_another_stream(dev):
    """workspace_status(stream=...) for a workspace used on a side stream,
    called while the default stream is current: the counter it returns
    counts every launch made on that stream."""
    inp = to_dev(inputs(1, 3000, 8, 64, seed=62), dev)
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        cheby_ema_forward(inp["x"], inp["coeffs"], inp["damping"], inp["lam"])
    ws = ops._ws_cache[(dev.index, side.cuda_stream, nat.OP_FWD)]
    _, e0 = ops.workspace_status(ws, stream=side.cuda_stream)
    with torch.cuda.stream(side):
        for _ in range(5):
            cheby_ema_forward(inp["x"], inp["coeffs"], inp["damping"], inp["lam"])
    assert ops.workspace_status(ws, stream=side.cuda_stream) == (0, e0 + 5)


def test_layout_change_repairs_stale_counters(dev):
    """Completion counters left non-zero in the header (what two calls that
    overlap on one workspace, a misuse, can leave) are cleared by the next
    layout change, which keeps the launch counter and the fault word: later
    launches count correctly and match the oracle."""
    a = to_dev(inputs(2, 5000, 8, 64, seed=63), dev)
    b_in = inputs(1, 7000, 8, 64, seed=64)
    b = to_dev(b_in, dev)
    cheby_ema_forward(a["x"], a["coeffs"], a["damping"], a["lam"])
    ws = _fwd_ws(dev)
    _, e0 = ops.workspace_status(ws)
    torch.cuda.synchronize()
    words = ws.view(torch.int32)
    words[16] = 3                       # done_all (byte 64)
    for c in range(8):
        words[32 + 32 * c] = 5 + c      # cls[c].done (byte 128 + 128 c)
    torch.cuda.synchronize()
    # another layout: its clear zeroes the counters
    for i in range(3):
        got = cheby_ema_forward(b["x"], b["coeffs"], b["damping"], b["lam"])
    assert ops.workspace_status(ws) == (0, e0 + 3)
    assert_close_fp32(got.cpu().numpy(), oracle_forward(b_in)[0])
