"""Recovery map helpers against their definitions (CPU).

`recovery_geometry` forms alpha and beta from R-dimensional quantities; here
they are recomputed from the materialised per-channel response U b_c.
"""

import pytest
import torch

from calibration_free_moe.reader.progressive import recovery_geometry


def test_geometry_equals_the_materialised_response():
    generator = torch.Generator().manual_seed(3)
    experts, hidden, width, rank = 3, 256, 48, 8
    down = (torch.randn(experts, hidden, width, generator=generator) * 0.02).bfloat16()
    down[1, :, 5] = 0  # a zero down column: alpha is 0, beta is |U b|
    encoder_t = (torch.randn(experts, width, rank, generator=generator) * 0.1).bfloat16()
    decoder = torch.linalg.qr(torch.randn(hidden, rank, generator=generator))[0].bfloat16()
    norms = down.float().square().sum(1).sqrt()
    got = recovery_geometry(down, norms, encoder_t, decoder).double()
    for e in range(experts):
        response = encoder_t[e].double() @ decoder.double().T  # [I, H]: U b_c
        column = down[e].double().T  # [I, H]: d_c
        length = column.norm(dim=-1)
        alpha = torch.where(length > 0, (column * response).sum(-1) / length.clamp_min(1e-300), 0.0)
        beta = (response.norm(dim=-1).square() - alpha.square()).clamp_min(0).sqrt()
        torch.testing.assert_close(got[e, :, 0], alpha, rtol=1e-5, atol=1e-7)
        torch.testing.assert_close(got[e, :, 1], beta, rtol=1e-5, atol=1e-7)
    assert got[1, 5, 0] == 0
    # alpha^2 + beta^2 = |U b|^2 (Pythagoras along and across d_c)
    energy = (encoder_t.double() @ decoder.double().T).square().sum(-1)
    torch.testing.assert_close(got[..., 0].square() + got[..., 1].square(), energy,
                               rtol=1e-5, atol=1e-9)


def test_subspace_bank_against_the_singular_vectors():
    """U spans the top-r left singular vectors of the stacked down columns
    (an SVD, not the Gram eigensolver), captured is their energy share, and
    U B_e is the projection of D_e onto that subspace."""
    from calibration_free_moe.recovery import subspace_bank

    generator = torch.Generator().manual_seed(4)
    experts, hidden, width, rank = 5, 96, 40, 6
    # a decaying spectrum so that the top-r subspace is well separated
    basis = torch.linalg.qr(torch.randn(hidden, hidden, generator=generator, dtype=torch.float64))[0]
    scales = torch.logspace(0, -2, hidden, dtype=torch.float64)
    mix = torch.randn(experts, hidden, width, generator=generator, dtype=torch.float64)
    down = ((basis * scales) @ mix).to(torch.bfloat16)
    u, b, captured = subspace_bank(down, rank, chunk=2)
    assert u.shape == (hidden, rank) and b.shape == (experts, rank, width)
    assert u.dtype == b.dtype == torch.float64
    columns = down.double().permute(1, 0, 2).reshape(hidden, -1)
    left, singular, _ = torch.linalg.svd(columns, full_matrices=False)
    top = left[:, :rank]
    torch.testing.assert_close(u @ u.T, top @ top.T, rtol=0, atol=1e-9)
    energy = singular.square()
    assert abs(captured - float(energy[:rank].sum() / energy.sum())) < 1e-12
    torch.testing.assert_close(u.T @ u, torch.eye(rank, dtype=torch.float64), rtol=0, atol=1e-12)
    for e in range(experts):
        projection = top @ (top.T @ down[e].double())
        torch.testing.assert_close(u @ b[e], projection, rtol=0, atol=1e-9)
    # chunking does not change the result
    u2, b2, captured2 = subspace_bank(down, rank, chunk=16)
    torch.testing.assert_close(u2 @ b2[1], u @ b[1], rtol=0, atol=1e-12)
    assert captured2 == pytest.approx(captured, abs=1e-14)
