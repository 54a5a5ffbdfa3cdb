"""Host logic of the engine's Cheby-RKV call sites (orthossm_amd/engine.py),
checked on the CPU: routing thresholds, the EMA momentum schedule against its
closed form, the state forms the reference engine accepts
(sdpc_engine.py:173-192), parameter names and shapes of the reference
engine's modules, and that a forward off the GPU fails loudly."""
import math

import pytest
import torch

from orthossm_amd import engine as E


def test_route_thresholds():
    # sdpc_engine.py:51-53, 216-225
    assert [E.route(s) for s in (1, 383, 384, 1023, 1024, 16384)] == \
        ["fast", "fast", "hybrid", "hybrid", "full", "full"]


@pytest.mark.parametrize("tokens,want", [(0, 0.9), (25_000_000, 0.7 + 0.1 * (1 + math.cos(math.pi / 4))),
                                         (50_000_000, 0.8), (100_000_000, 0.7), (300_000_000, 0.7)])
def test_ema_momentum_schedule_closed_form(tokens, want):
    # cosine anneal from ema_base (0.9) at 0 tokens to 0.7 at 1e8, flat beyond
    mu = E.ema_momentum_schedule(torch.tensor(tokens), torch.tensor(0.9))
    assert mu.dtype == torch.float32 and mu.dim() == 0
    assert abs(mu.item() - want) < 1e-6


def test_schedule_counts_this_calls_tokens_first():
    # the engine adds S before computing mu (sdpc_engine.py:199-208)
    m = E.ChebyContextPath(64, n_cheby_heads=4)
    m.total_tokens_seen.fill_(99_999_990)
    with pytest.raises(RuntimeError):         # CPU tensors: the kernels refuse
        m(torch.randn(1, 10, 64))
    assert m.total_tokens_seen.item() == 100_000_000


def test_parse_state_forms():
    c = torch.randn(2, 4, 3, 8)
    mom = torch.randn(2, 4, 3, 8)
    got = E.parse_cheby_state((c, mom), 4)
    assert got[0] is c and got[1] is mom and got[2] is None
    got = E.parse_cheby_state((c, mom, torch.zeros_like(mom)), 4)      # (coeffs, m1, m2)
    assert got[0] is c and got[1] is mom and got[2] is None
    ema = torch.randn(2, 32)
    got = E.parse_cheby_state(E.ChebyState(c, mom, ema), 4)
    assert got[2] is ema
    # a bare tensor: zero momentum, K padded up to max_degree
    got = E.parse_cheby_state(c, 4)
    assert got[0].shape == (2, 4, 4, 8) and torch.equal(got[0][:, :, :3], c) and torch.all(got[0][:, :, 3] == 0)
    assert torch.all(got[1] == 0) and got[1].shape == got[0].shape
    # [B,K,hd] gains a head axis
    got = E.parse_cheby_state(torch.randn(2, 4, 8), 4)
    assert got[0].shape == (2, 1, 4, 8)


def test_parameter_names_and_shapes_follow_the_engine():
    # names and shapes of the reference engine's modules on this path
    # (sdpc_engine.py:83, 92-105, 151, 159-160; sdpc_kernel.py:1822-1827)
    D, H, K = 512, 8, 4
    m = E.ChebyContextPath(D, n_cheby_heads=H, max_degree=K)
    want = {
        "complexity_gate.net.0.weight": (D // 4, D), "complexity_gate.net.0.bias": (D // 4,),
        "complexity_gate.net.2.weight": (1, D // 4), "complexity_gate.net.2.bias": (1,),
        "coeff_init_proj.0.weight": (D // 4, D), "coeff_init_proj.0.bias": (D // 4,),
        "coeff_init_proj.2.weight": (H * K * (D // H), D // 4), "coeff_init_proj.2.bias": (H * K * (D // H),),
        "coeff_spectral_scale": (1, 1, K, 1), "input_norm.weight": (D,), "ema_base": (), "total_tokens_seen": (),
    }
    sd = m.state_dict()
    assert {k: tuple(v.shape) for k, v in sd.items()} == want
    assert torch.all(sd["coeff_init_proj.2.weight"] == 0) and torch.all(sd["coeff_init_proj.2.bias"] == 0)
    torch.testing.assert_close(sd["coeff_spectral_scale"].flatten(), 0.1 / torch.arange(1, K + 1).float())


def test_forward_off_gpu_fails_loudly():
    m = E.ChebyContextPath(64, n_cheby_heads=4)
    for S in (50, 500):
        with pytest.raises(RuntimeError, match="GPU"):
            m(torch.randn(1, S, 64))
