"""The drop-in module ``orthossm_amd.sdpc_kernel`` carries every name the
reference's callers import from ``sdpc_kernel`` (CPU, no GPU needed), and
``init_chebyshev_coefficients`` / ``get_chebyshev_lut`` are pinned by the
mathematics that fixes them.

Bitwise parity of the initialisation with the reference is unpinned (its
QR signs come from LAPACK), so it is checked through invariants that a
plausible slip breaks: the per-term scale 0.1/(k+1) of the draw, rows that
are mutually orthogonal and keep their norms, the Gram-Schmidt order of the
QR basis, and the polar-factor tight frame of the underdetermined case.
"""
import math

import numpy as np
import pytest
import torch

import orthossm_amd.sdpc_kernel as SK

# The import lines of the reference's callers (names only; the reference is
# not read at run time).  The Triton kernel object ``_fused_clenshaw_ema_kernel``
# (precision_tests.py:33) is excluded: its launch is a C-ABI entry point here.
CALLER_IMPORTS = {
    "sdpc_engine.py:39-43": ["apply_cheby_rkv_v10", "GatedComplexityPredictor", "init_chebyshev_coefficients"],
    "chimera_experiment/chimera_v2_ssm.py:54": ["apply_cheby_rkv_v10", "init_chebyshev_coefficients"],
    "pretrain_real.py:211": ["apply_cheby_rkv_core", "init_chebyshev_coefficients"],
    "benchmark_ortho.py:20": ["apply_cheby_rkv_core", "init_chebyshev_coefficients"],
    "model.py:20": ["init_chebyshev_coefficients"],
    "benchmark_ruler_pg19.py:30": ["init_chebyshev_coefficients"],
    "precision_tests.py:33": ["apply_cheby_rkv_v10", "get_chebyshev_lut", "LUT_TABLE_SIZE"],
    "ortho_diagnostics.py:174": ["get_chebyshev_lut"],
    # attribute uses of ``import sdpc_kernel as K``
    "test_v10.py / gradient_checker.py / benchmark_long_context.py": [
        "apply_cheby_rkv_v10", "apply_cheby_rkv_core", "init_chebyshev_coefficients"],
}


@pytest.mark.parametrize("site", sorted(CALLER_IMPORTS))
def test_caller_import_lines_resolve(site):
    missing = [n for n in CALLER_IMPORTS[site] if not hasattr(SK, n)]
    assert not missing, f"{site}: {missing} missing from orthossm_amd.sdpc_kernel"


def test_constants():
    # sdpc_kernel.py:58-59, 1416
    assert SK.LUT_TABLE_SIZE == 256 and SK.MAX_DEGREE == 8
    assert SK.MULTI_SCALE_LAMBDA == [0.9995, 0.9995, 0.997, 0.997, 0.995, 0.995, 0.97, 0.95]


def test_lut_is_chebyshev_on_the_half_grid():
    lut = SK.get_chebyshev_lut("cpu")
    assert lut.shape == (SK.MAX_DEGREE, SK.LUT_TABLE_SIZE) and lut.dtype == torch.float32
    assert lut.is_contiguous()
    u = np.linspace(0.0, 1.0, SK.LUT_TABLE_SIZE)
    want = np.cos(np.arange(SK.MAX_DEGREE)[:, None] * np.arccos(u)[None, :])   # T_k(cos t) = cos(k t)
    assert np.abs(lut.numpy() - want).max() < 2e-6
    assert SK.get_chebyshev_lut(torch.device("cpu")) is lut   # built once per device


def test_predictor_layout_and_range():
    m = SK.GatedComplexityPredictor(64)
    names = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert names == {"net.0.weight": (16, 64), "net.0.bias": (16,), "net.2.weight": (1, 16), "net.2.bias": (1,)}
    y = m(torch.randn(3, 64))
    assert y.shape == (3, 1) and bool(((y > 0) & (y < 1)).all())


def _raw_draw(seed, B, H, K, hd):
    torch.manual_seed(seed)
    sigma = 0.1 / (torch.arange(K, dtype=torch.float32) + 1.0)
    return torch.randn(B, H, K, hd) * sigma.view(1, 1, K, 1)


def test_single_head_is_the_scaled_draw():
    # No decorrelation with one head: the result is the draw times 0.1/(k+1),
    # from the same generator call.
    torch.manual_seed(7)
    c = SK.init_chebyshev_coefficients(3, 1, 8, 16, "cpu")
    assert torch.equal(c, _raw_draw(7, 3, 1, 8, 16))
    torch.manual_seed(7)
    z = torch.randn(3, 1, 8, 16)
    ratio = (c / z).reshape(3, 8, 16)
    for k in range(8):
        assert torch.allclose(ratio[:, k], torch.full_like(ratio[:, k], 0.1 / (k + 1)), rtol=1e-6)


@pytest.mark.parametrize("B,H,K,hd", [(2, 8, 4, 64), (3, 4, 8, 16), (1, 2, 1, 2), (2, 5, 1, 5)])
def test_qr_branch_orthogonal_rows_with_norms_kept(B, H, K, hd):
    torch.manual_seed(11)
    c = SK.init_chebyshev_coefficients(B, H, K, hd, "cpu")
    raw = _raw_draw(11, B, H, K, hd)
    assert c.shape == (B, H, K, hd) and c.dtype == torch.float32
    rows = c.reshape(B, H, K * hd).double()
    raw_rows = raw.reshape(B, H, K * hd).double()
    # norms preserved
    assert torch.allclose(rows.norm(dim=2), raw_rows.norm(dim=2), rtol=1e-5)
    # mutually orthogonal: the Gram matrix is diagonal
    gram = rows @ rows.transpose(1, 2)
    off = gram - torch.diag_embed(torch.diagonal(gram, dim1=1, dim2=2))
    assert off.abs().max() <= 1e-5 * gram.abs().max()
    # Gram-Schmidt order: head h lies along the part of raw head h orthogonal
    # to raw heads 0..h-1 (up to the sign LAPACK picks).
    for b in range(B):
        basis = []
        for h in range(H):
            v = raw_rows[b, h].clone()
            for e in basis:
                v -= (v @ e) * e
            e_h = v / v.norm()
            basis.append(e_h)
            cos = (rows[b, h] @ e_h) / rows[b, h].norm()
            assert abs(abs(cos.item()) - 1.0) < 1e-5, (b, h, cos.item())


@pytest.mark.parametrize("B,H,K,hd", [(2, 8, 1, 4), (1, 6, 2, 2), (3, 5, 1, 3)])
def test_tight_frame_branch(B, H, K, hd):
    # deg*hd < n_heads: no orthogonal set of H rows exists; the normalised
    # rows become the polar factor times sqrt(H/width), a Parseval frame.
    width = K * hd
    assert width < H
    torch.manual_seed(5)
    c = SK.init_chebyshev_coefficients(B, H, K, hd, "cpu")
    raw = _raw_draw(5, B, H, K, hd).reshape(B, H, width).double()
    norms = raw.norm(dim=2, keepdim=True)
    rows = c.reshape(B, H, width).double()
    frame = rows / norms
    # F^T F = (H / width) I
    ftf = frame.transpose(1, 2) @ frame
    assert torch.allclose(ftf, (H / width) * torch.eye(width, dtype=torch.float64).expand(B, -1, -1), atol=2e-5)
    # the polar factor of the unit rows, W (W^T W)^(-1/2), computed here by
    # an eigendecomposition (no SVD sign conventions involved)
    unit = raw / (norms + 1e-8)
    for b in range(B):
        w = unit[b]
        evals, evecs = torch.linalg.eigh(w.T @ w)
        inv_sqrt = evecs @ torch.diag(evals.rsqrt()) @ evecs.T
        polar = w @ inv_sqrt * math.sqrt(H / width)
        assert torch.allclose(frame[b], polar, atol=2e-5), b


def test_init_device_argument_forms():
    for dev in ("cpu", torch.device("cpu")):
        c = SK.init_chebyshev_coefficients(1, 4, 4, 8, dev)
        assert c.device.type == "cpu"
