"""Device sketch construction (cfmoe_build_sketch) against the torch build.

The HIP kernel (`build_sketch(..., device_kernel=True)`) builds the reference's
resident sketch format (sketch.py:84-150) from device weights; the default
`build_sketch` runs the torch construction on any device (the default reader
constructor uses it, test_progressive_reader.py:803-805 of the reference). The rotation is the same FP32 operations in the same order, so
the rotated values agree bit for bit; the sums behind mean|v|, the scale and
the residual run in a different order. The check therefore follows the
reference's own comparison of two sketch builds (codes exact, statistics
atol 1e-4 / rtol 1e-3, test_progressive_reader.py:803-809), with one stated
allowance: a trit may differ only where |v| lies within 2e-5 (relative) of
0.7 mean|v| computed in float64, and the statistics of such a (row, block)
are left out of the tolerance check. Shapes cover the block-paired 16-byte
tails (width 512), an odd block count (hidden 384: the last tail half is
padding), a width that is not a multiple of five, and unrotated blocks.
"""

import pytest
import torch

from calibration_free_moe.reader.sketch import (
    block_hadamard_signs,
    build_sketch,
    rotate_blocks,
    unpack_sketch,
)

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda:0")


@pytest.mark.parametrize(
    "experts,width,hidden,rotated",
    [(4, 256, 512, True), (2, 512, 2048, True), (3, 96, 384, True), (2, 72, 256, False)],
)
def test_device_sketch_matches_torch_build(experts, width, hidden, rotated):
    generator = torch.Generator().manual_seed(experts * 1000 + width + hidden)
    weights = (torch.randn(experts, 2 * width, hidden, generator=generator) * 0.02).to(torch.bfloat16)
    signs = block_hadamard_signs(hidden, "cpu") if rotated else None
    want_codes, want_stats = build_sketch(weights, signs)
    got_codes, got_stats = build_sketch(
        weights.to(DEVICE), None if signs is None else signs.to(DEVICE), device_kernel=True
    )
    torch.cuda.synchronize()
    got_codes, got_stats = got_codes.cpu(), got_stats.cpu()
    assert got_codes.shape == want_codes.shape and got_stats.shape == want_stats.shape
    rows = 2 * width
    got_trits = unpack_sketch(got_codes, rows, hidden)
    want_trits = unpack_sketch(want_codes, rows, hidden)
    # the allowance: near-threshold coordinates, from the FP32 rotated values
    value = rotate_blocks(weights, signs).reshape(experts, rows, hidden // 128, 128).double()
    magnitude = value.abs()
    threshold = 0.7 * magnitude.mean(-1, keepdim=True)
    near = ((magnitude - threshold).abs() <= 2e-5 * threshold).reshape(experts, rows, hidden)
    differ = got_trits != want_trits
    assert not (differ & ~near).any(), "a trit differs away from the TWN threshold"
    assert int(differ.sum()) <= max(8, differ.numel() // 10000)
    # every byte without a flipped trit is identical (padding bytes included)
    assert int((got_codes != want_codes).sum()) <= int(differ.sum())
    # statistics [E, 2 I, blocks, 2] to the reference's tolerance, outside
    # the (row, block) cells that hold a flipped trit
    flipped = differ.reshape(experts, rows, hidden // 128, 128).any(-1)
    clean = ~flipped
    torch.testing.assert_close(got_stats.float()[clean], want_stats.float()[clean],
                               rtol=1e-3, atol=1e-4)


def test_default_build_on_the_device_is_the_torch_construction():
    """Without device_kernel, device weights get the torch construction: the
    same codes as the build on the host, and statistics to the reference's
    tolerance (its reductions run in the device's order)."""
    generator = torch.Generator().manual_seed(77)
    weights = (torch.randn(3, 2 * 96, 384, generator=generator) * 0.02).to(torch.bfloat16)
    signs = block_hadamard_signs(384, "cpu")
    want_codes, want_stats = build_sketch(weights, signs)
    got_codes, got_stats = build_sketch(weights.to(DEVICE), signs.to(DEVICE))
    torch.cuda.synchronize()
    assert torch.equal(got_codes.cpu(), want_codes)
    torch.testing.assert_close(got_stats.cpu(), want_stats, atol=1e-4, rtol=1e-3)
