"""The entry points under HIP graph capture (torch.cuda.CUDAGraph): a captured
forward, TTT step, backward and full path replay several times, with eager launches of
the same entry points and host synchronisations in between, and every replay
equals the eager result bit for bit.  The workspaces of the capture stream
are created by a warm-up on that stream before capture, so the graphs hold
only the library's kernels (no memset nodes); launches keep their state in
the workspace (epoch, look-back words), not on the host."""
import pytest
import torch

from helpers import inputs, to_dev
from orthossm_amd import cheby_ema_backward, cheby_ema_forward, cheby_ema_ttt

pytestmark = pytest.mark.gpu


def _capture(fn, stream):
    """Warm fn up on `stream`, then capture it there; returns the graph."""
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            fn()
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("dynamic", [False, True])
def test_forward_graph_replays_match_eager(dev, dynamic):
    d = to_dev(inputs(2, 5000, 8, 64, seed=31, dynamic=dynamic), dev)
    other = to_dev(inputs(1, 3000, 8, 64, seed=32, dynamic=dynamic), dev)
    init = torch.randn(2, 512, device=dev) * 0.3
    want, want_fin = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], g=d.get("g"), ema_init=init,
                                       return_state=True)
    out = torch.empty_like(want)
    fin = torch.empty_like(want_fin)

    def step():
        cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"], g=d.get("g"), ema_init=init, out=out,
                          return_state=True, state_out=fin)

    g = _capture(step, torch.cuda.Stream())
    for i in range(4):
        out.fill_(float("nan"))
        g.replay()
        # eager work of the same entry point on the default stream in between
        cheby_ema_forward(other["x"], other["coeffs"], other["damping"], other["lam"], g=other.get("g"))
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        assert torch.equal(fin, want_fin), f"replay {i} ema_final"


def test_ttt_graph_replays_match_eager(dev):
    inp = inputs(2, 3000, 8, 64, seed=33)
    d = to_dev(inp, dev)
    xb = d["x"].to(torch.bfloat16)
    want_out, want_grad = cheby_ema_ttt(xb, d["coeffs"], d["damping"], d["lam"])
    out = torch.empty_like(want_out)
    grad = torch.empty_like(want_grad)

    def step():
        cheby_ema_ttt(xb, d["coeffs"], d["damping"], d["lam"], out=out, grad_out=grad)

    g = _capture(step, torch.cuda.Stream())
    for i in range(4):
        grad.zero_()
        g.replay()
        cheby_ema_ttt(xb[:1, :1000], d["coeffs"][:1], d["damping"], d["lam"])
        torch.cuda.synchronize()
        assert torch.equal(out, want_out), f"replay {i}"
        assert torch.equal(grad, want_grad), f"replay {i} grad"


def test_backward_graph_replays_match_eager(dev):
    d = to_dev(inputs(2, 4000, 8, 64, seed=34), dev)
    out = cheby_ema_forward(d["x"], d["coeffs"], d["damping"], d["lam"])
    go = torch.randn(out.shape, device=dev, generator=torch.Generator(device=dev).manual_seed(35))
    want = cheby_ema_backward(d["x"], d["coeffs"], d["damping"], d["lam"], out, go, need_init=True)
    gx, gc, gi = (torch.empty_like(t) for t in want)

    def step():
        cheby_ema_backward(d["x"], d["coeffs"], d["damping"], d["lam"], out, go, grad_x_out=gx,
                           grad_coeffs_out=gc, grad_init_out=gi)

    g = _capture(step, torch.cuda.Stream())
    for i in range(4):
        gx.zero_()
        g.replay()
        cheby_ema_backward(d["x"][:1], d["coeffs"][:1], d["damping"], d["lam"], out[:1], go[:1])
        torch.cuda.synchronize()
        for got, w, what in zip((gx, gc, gi), want, ("grad_x", "grad_coeffs", "grad_init")):
            assert torch.equal(got, w), f"replay {i} {what}"


def test_full_path_graph_replays_match_eager(dev):
    from orthossm_amd.ops import v10_chunked_ttt
    gen = torch.Generator().manual_seed(36)
    x = torch.randn(2, 900, 256, generator=gen).to(dev)
    c = (torch.randn(2, 4, 8, 64, generator=gen) * 0.3).to(dev)
    m = (torch.randn(2, 4, 8, 64, generator=gen) * 0.01).to(dev)
    mu = torch.tensor(0.85, device=dev)
    want = v10_chunked_ttt(x, c, m, n_heads=4, ema_momentum=mu)
    res = [None]

    def step():
        res[0] = v10_chunked_ttt(x, c, m, n_heads=4, ema_momentum=mu)

    g = _capture(step, torch.cuda.Stream())
    for i in range(4):
        g.replay()
        v10_chunked_ttt(x[:1, :300], c[:1], m[:1], n_heads=4)
        torch.cuda.synchronize()
        for got, w, what in zip(res[0], want, ("out", "coeffs", "momentum")):
            assert torch.equal(got, w), f"replay {i} {what}"


def test_forward_graph_with_other_layouts_on_the_capture_stream(dev):
    # Between replays an eager call of another shape runs on the capture
    # stream, so on the same workspace with another layout (the library
    # clears its look-back words).  The captured launch then reuses the
    # workspace with no host step; the inputs change before every replay, so
    # a look-back word left by an earlier replay (another payload) that
    # matched a later launch's tag would give a wrong result.
    big = [to_dev(inputs(2, 6000, 8, 64, seed=40 + i), dev) for i in range(4)]
    small = to_dev(inputs(1, 700, 8, 64, seed=39), dev)
    xbuf = big[0]["x"].clone()
    c, damp, lam = big[0]["coeffs"], big[0]["damping"], big[0]["lam"]
    out = torch.empty_like(xbuf)
    cap = torch.cuda.Stream()

    def step():
        cheby_ema_forward(xbuf, c, damp, lam, out=out)

    g = _capture(step, cap)
    for i in range(4):
        xbuf.copy_(big[i]["x"])
        want = cheby_ema_forward(xbuf, c, damp, lam)        # default stream, its own workspace
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        with torch.cuda.stream(cap):
            cheby_ema_forward(small["x"][:, : 300 + 100 * i], small["coeffs"], small["damping"], small["lam"])
        torch.cuda.synchronize()
