"""The workspace's fault word through the C ABI (osm_workspace_status): zero
after ordinary launches, a launch counter that grows by one per launch and
keeps growing across a layout change, and a fault left by an earlier launch
(planted from the host into the header) that is reported, that raises under
the per-launch check, and that does not disturb later launches."""
import pytest
import torch

from helpers import assert_close_fp32, inputs, oracle_forward, to_dev
from orthossm_amd import _native as nat
from orthossm_amd import cheby_ema_forward, ops

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
