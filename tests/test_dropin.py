"""Host-side behaviour of the drop-in apply_cheby_rkv_v10 that needs no GPU:
the paths it does not implement raise instead of changing semantics, and
CPU tensors raise (there is no CPU path)."""
import pytest
import torch

from orthossm_amd import apply_cheby_rkv_core, apply_cheby_rkv_v10


def test_alias():
    assert apply_cheby_rkv_core is apply_cheby_rkv_v10


def test_full_path_needs_the_gpu_and_a_momentum_buffer():
    x = torch.zeros(1, 512, 64)
    c = torch.zeros(1, 4, 4, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        apply_cheby_rkv_v10(x, c, torch.zeros_like(c), n_heads=4, seq_threshold=384)
    with pytest.raises((RuntimeError, ValueError)):
        apply_cheby_rkv_v10(x, c, None, n_heads=4, seq_threshold=0)


def test_full_path_gradients_need_the_gpu_too():
    x = torch.zeros(1, 512, 64, requires_grad=True)
    c = torch.zeros(1, 4, 4, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        apply_cheby_rkv_v10(x, c, torch.zeros_like(c), n_heads=4, seq_threshold=384)


def test_gradient_path_is_gpu_only_too():
    x = torch.zeros(1, 16, 64, requires_grad=True)
    c = torch.zeros(1, 4, 4, 16, requires_grad=True)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        apply_cheby_rkv_v10(x, c, None, n_heads=4)


def test_cpu_tensor_raises():
    x = torch.zeros(1, 16, 64)
    c = torch.zeros(1, 4, 4, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        apply_cheby_rkv_v10(x, c, None, n_heads=4)


def test_fast_path_rejects_more_than_thirty_two_coefficients():
    # the reference's PyTorch fast path takes any number of terms; the
    # fixed-coefficient kernels here take up to 32
    x = torch.randn(1, 16, 32)
    c = torch.randn(1, 4, 33, 8)
    with pytest.raises(ValueError, match="at most 32"):
        apply_cheby_rkv_v10(x, c, torch.zeros_like(c), n_heads=4, seq_threshold=384)
