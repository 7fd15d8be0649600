"""Recovery bank construction on the device against the host FP64 build
(needs an MI355X). The basis is fixed only up to column signs, so the checks
are sign-invariant: the projector U U^T, the captured energy and U B_e."""

import time

import pytest
import torch

from calibration_free_moe.recovery import subspace_bank

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda:0")


@pytest.mark.parametrize("experts,hidden,width", [(16, 512, 256), (128, 2048, 768)])
def test_device_bank_matches_the_host_build(experts, hidden, width):
    generator = torch.Generator().manual_seed(experts + hidden)
    down = (torch.randn(experts, hidden, width, generator=generator) * 0.02).bfloat16()
    rank = 32
    host_u, host_b, host_captured = subspace_bank(down, rank)
    torch.cuda.synchronize()
    begin = time.perf_counter()
    u, b, captured = subspace_bank(down.to(DEVICE), rank)
    torch.cuda.synchronize()
    print(f"device bank E={experts} H={hidden} I={width}: {time.perf_counter() - begin:.3f} s")
    assert u.device == DEVICE and u.dtype == torch.float64
    u, b = u.cpu(), b.cpu()
    torch.testing.assert_close(u @ u.T, host_u @ host_u.T, rtol=0, atol=1e-8)
    assert captured == pytest.approx(host_captured, rel=1e-10)
    for e in (0, experts // 2, experts - 1):
        torch.testing.assert_close(u @ b[e], host_u @ host_b[e], rtol=0, atol=1e-9)
