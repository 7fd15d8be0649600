"""Resident sketch: format, decoding and rotation (reference tests/test_sketch.py,
tests/test_progressive_reader.py:33-99)."""

import numpy as np
import pytest
import torch

from calibration_free_moe.reader.budget import compile_budget
from calibration_free_moe.reader.sketch import (
    block_hadamard_signs,
    build_sketch,
    differentiable_sketch_feature,
    mask_rotated_blocks,
    rotate_blocks,
    unpack_sketch,
)

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


def independent_unpack(codes, rows, hidden):
    """Decode codes by reassembling coordinate runs (no library offsets)."""
    stride = (2 * ((rows // 2 + 4) // 5) + 15) // 16 * 16
    body, blocks = stride // 32 * 32, hidden // 128
    runs = codes[..., : blocks * 128 * body].reshape(codes.shape[0], blocks, 128, body)
    if stride % 32:
        tails = codes[..., blocks * 128 * body:].reshape(-1, (blocks + 1) // 2, 128, 2, 16)
        tails = tails.transpose(2, 3).reshape(-1, (blocks + 1) // 2 * 2, 128, 16)[:, :blocks]
        runs = torch.cat((runs, tails), dim=-1)
    row = torch.arange(rows)
    channel = row % (rows // 2)
    trits = (runs[..., 2 * (channel // 5) + row // (rows // 2)].long() // (3 ** (channel % 5))) % 3 - 1
    return trits.movedim(-1, -3).flatten(-2)


def hadamard128():
    block = torch.ones(1, 1, dtype=torch.float64)
    while len(block) < 128:
        block = torch.cat((torch.cat((block, block), 1), torch.cat((block, -block), 1)), 0)
    return block


def test_signs_match_committed_fixture():
    signs = block_hadamard_signs(2048, "cpu")
    assert set(signs.unique().tolist()) == {-1, 1}
    expected = np.load(f"{GOLDEN}/signs_2048.npy")
    assert np.array_equal(signs.numpy(), expected)
    assert torch.equal(block_hadamard_signs(256, "cpu"), signs[:256])


def test_ternary_packing_and_residual_variance():
    # Unrotated known answer (reference test_progressive_reader.py:81-99).
    torch.manual_seed(33)
    weights = torch.randn(2, 8, 256).bfloat16()
    codes, metadata = build_sketch(weights)
    original = weights.float().reshape(2, 8, 2, 128)
    keep = original.abs() > 0.7 * original.abs().mean(-1, keepdim=True)
    expected_scale = (original.abs() * keep).sum(-1) / keep.sum(-1)
    expected_codes = torch.where(keep, original.sign(), 0).reshape_as(weights)
    assert torch.equal(independent_unpack(codes, 8, 256), expected_codes.long())
    assert torch.equal(unpack_sketch(codes, 8, 256).long(), expected_codes.long())
    assert torch.equal(metadata[..., 0], expected_scale.half())
    residual = original - expected_codes.reshape_as(original) * expected_scale[..., None]
    assert torch.equal(metadata[..., 1], residual.square().mean(-1).half())
    assert codes.numel() + metadata.numel() * 2 == 2 * 2 * (128 * 16 + 8 * 4)
    assert metadata.stride() == (4 * 4 * 2, 1, 4 * 4, 2 * 4)


@pytest.mark.parametrize("width,hidden", [(512, 384), (704, 256), (48, 256)])
def test_sector_tiled_sketch_preserves_rows_and_prices_loads(width, hidden):
    """Half-sector widths, an odd final block; walks every byte request."""
    torch.manual_seed(83)
    weights = torch.randn(1, 2 * width, hidden).bfloat16()
    codes, _ = build_sketch(weights)
    original = weights.float().reshape(1, 2 * width, hidden // 128, 128)
    keep = original.abs() > 0.7 * original.abs().mean(-1, keepdim=True)
    signed = torch.where(keep, original.sign(), 0)
    assert torch.equal(unpack_sketch(codes, 2 * width, hidden), signed.flatten(-2).to(torch.int8))
    assert torch.equal(independent_unpack(codes, 2 * width, hidden), signed.flatten(-2).long())
    useful = 2 * ((width + 4) // 5)
    stride = (useful + 15) // 16 * 16
    body = stride // 32 * 32
    blocks = hidden // 128
    sectors = 0
    for block in range(blocks):
        for coordinate in range(80):
            for start in range(0, useful, 32):
                byte = torch.arange(start, min(start + 32, useful))
                if start < body:
                    address = (block * 128 + coordinate) * body + byte
                else:
                    address = (blocks * 128 * body + (block // 2 * 128 + coordinate) * 32
                               + block % 2 * 16 + byte - body)
                assert len(set((address // 32).tolist())) == 1
                sectors += 1
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=1, retention=0.1,
                          screen_keep=0.625)
    assert plan.sketch_read_bytes(residual=False) == sectors * 32 + blocks * 4 * width


def test_padding_byte_is_zero_code():
    codes, _ = build_sketch(torch.randn(1, 2 * 48, 256).bfloat16())
    stride = 32  # 2 * ceil(48 / 5) = 20 useful bytes, padded to 32
    rows = codes.reshape(-1)[: 2 * 128 * stride].reshape(2 * 128, stride)
    assert torch.all(rows[:, 20:] == 121)


def test_rotation_is_the_scaled_sylvester_transform():
    signs = block_hadamard_signs(256, "cpu")
    matrix = torch.block_diag(hadamard128(), hadamard128()) * signs.double()[None, :]
    # Small dyadic integers: every butterfly sum is exact in FP32.
    x = torch.randint(-4, 5, (5, 256)).float()
    exact = (x.double() @ matrix.T) * float(np.float32(1 / np.sqrt(128)))
    assert torch.equal(rotate_blocks(x, signs).double(), exact.float().double())
    y = torch.randn(7, 256)
    torch.testing.assert_close(
        rotate_blocks(y, signs).double(), (y.double() @ matrix.T) / 128**0.5, rtol=1e-5, atol=1e-5
    )
    # Orthogonality
    z = rotate_blocks(torch.eye(256), signs).double()
    torch.testing.assert_close(z @ z.T, torch.eye(256, dtype=torch.float64), atol=1e-6, rtol=0)


def test_mask_keeps_largest_with_coordinate_ties():
    x = torch.randint(-3, 4, (6, 256)).float()
    kept = mask_rotated_blocks(x, 80).reshape(-1, 128)
    for row, values in enumerate(x.reshape(-1, 128).tolist()):
        order = sorted(range(128), key=lambda c: (-abs(values[c]), c))[:80]
        expected = torch.zeros(128)
        expected[order] = torch.tensor(values)[order]
        assert torch.equal(kept[row], expected)


@pytest.mark.parametrize("keep", [80, 128])
@pytest.mark.parametrize("input_is_rotated", [False, True])
def test_sketch_feature_matches_kept_coordinate_reference(keep, input_is_rotated):
    torch.manual_seed(71)
    hidden, width = 256, 16
    signs = block_hadamard_signs(hidden, "cpu")
    codes, statistics = build_sketch(torch.randn(1, 2 * width, hidden) * 0.1, signs=signs)
    x = torch.randint(-3, 4, (3, hidden)).float().requires_grad_()
    rotated = x if input_is_rotated else rotate_blocks(x, signs)
    blocks = rotated.reshape(-1, 128)
    mask = torch.zeros_like(blocks, dtype=torch.bool)
    for row, values in enumerate(blocks.detach().tolist()):
        order = sorted(range(128), key=lambda c: (-abs(values[c]), c))
        mask[row, order[:keep]] = True
    kept = torch.where(mask, blocks, 0.0).reshape(3, 2, 128)
    trits = unpack_sketch(codes, 2 * width, hidden)[0].float().reshape(2 * width, 2, 128)
    projection = (torch.einsum("tbc,rbc->trb", kept, trits) * statistics[0, ..., 0].float()).sum(-1)
    g, u = projection.chunk(2, dim=-1)
    expected = (torch.nn.functional.silu(g.bfloat16().float()) * u.bfloat16().float()).bfloat16()
    actual = differentiable_sketch_feature(
        x, codes[0], statistics[0], signs, input_is_rotated=input_is_rotated,
        screen_coordinates=keep,
    )
    torch.testing.assert_close(actual, expected)
    expected_grad = torch.autograd.grad(expected.float().sum(), x)[0]
    actual_grad = torch.autograd.grad(actual.float().sum(), x)[0]
    torch.testing.assert_close(actual_grad, expected_grad)
    if input_is_rotated:
        assert torch.count_nonzero(actual_grad.reshape_as(mask)[~mask]) == 0


def test_rotated_build_matches_unrotated_build_of_rotated_rows():
    torch.manual_seed(7)
    signs = block_hadamard_signs(256, "cpu")
    weights = torch.randn(3, 2 * 32, 256).bfloat16()
    codes, stats = build_sketch(weights, signs)
    rotated = rotate_blocks(weights.float().reshape(-1, 256), signs).reshape(3, 64, 256)
    codes2, stats2 = build_sketch(rotated)
    assert torch.equal(codes, codes2)
    assert torch.equal(stats, stats2)


def test_chunked_build_is_chunk_independent():
    weights = torch.randn(5, 2 * 64, 256).bfloat16()
    signs = block_hadamard_signs(256, "cpu")
    a = build_sketch(weights, signs, chunk=1)
    b = build_sketch(weights, signs, chunk=8)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
