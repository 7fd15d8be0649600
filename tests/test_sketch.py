"""Resident sketch: rotation, mask, packed format, statistics and the sketch
feature, each against a construction written here from its definition.

* Rotation: the Sylvester Hadamard matrix as an explicit float64 matrix.
* Mask: a sort of (|v| descending, coordinate ascending).
* Format: a numpy decoder that locates every trit by address (`stored_address`
  of tests/test_budget.py) and reads its base-3 digit.
* Ternarisation: a hand-made block with known trits, scale and residual, and
  float64 restatements on random weights.
* Feature: explicit float64 matrices for the projection and its gradient.
"""

import os

import numpy as np
import pytest
import torch

from calibration_free_moe.reader.budget import sketch_storage_bytes
from calibration_free_moe.reader.sketch import (
    ZERO_CODE,
    block_hadamard_signs,
    build_sketch,
    differentiable_sketch_feature,
    mask_rotated_blocks,
    rotate_blocks,
    unpack_sketch,
)
from tests.test_budget import stored_address

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def sylvester(size: int = 128) -> np.ndarray:
    matrix = np.ones((1, 1))
    while len(matrix) < size:
        matrix = np.block([[matrix, matrix], [matrix, -matrix]])
    return matrix


def rotation_matrix(signs: np.ndarray) -> np.ndarray:
    """blockdiag(H128) diag(signs) / sqrt(128), float64."""
    blocks = len(signs) // 128
    h = sylvester()
    full = np.zeros((len(signs), len(signs)))
    for b in range(blocks):
        full[128 * b:128 * (b + 1), 128 * b:128 * (b + 1)] = h
    return full * signs[None, :].astype(np.float64) / np.sqrt(128.0)


def decode_by_address(codes: np.ndarray, width: int, hidden: int) -> np.ndarray:
    """Trits [E, 2 width, hidden] read one byte address at a time."""
    experts = codes.shape[0]
    rows = 2 * width
    out = np.zeros((experts, rows, hidden), np.int8)
    for row in range(rows):
        plane, channel = divmod(row, width)
        byte = 2 * (channel // 5) + plane
        power = 3 ** (channel % 5)
        for coordinate in range(hidden):
            address = stored_address(width, hidden, coordinate // 128, coordinate % 128, byte)
            out[:, row, coordinate] = (codes[:, address].astype(np.int64) // power) % 3 - 1
    return out


def twn(values: np.ndarray):
    """Float64 TWN rule of one block: trits, scale, mean squared residual."""
    magnitude = np.abs(values)
    keep = magnitude > 0.7 * magnitude.mean()
    trits = np.where(keep, np.sign(values), 0)
    scale = magnitude[keep].mean() if keep.any() else 0.0
    return trits, scale, np.mean((values - trits * scale) ** 2)


def test_signs_match_committed_fixture():
    signs = block_hadamard_signs(2048, "cpu")
    assert np.array_equal(signs.numpy(), np.load(os.path.join(GOLDEN, "signs_2048.npy")))
    assert set(signs.tolist()) == {-1, 1}
    # a prefix of a wider model's signs is the narrower model's signs
    assert torch.equal(block_hadamard_signs(384, "cpu"), signs[:384])


def test_rotation_is_the_explicit_hadamard_matrix():
    signs = block_hadamard_signs(384, "cpu")
    matrix = rotation_matrix(signs.numpy())
    generator = torch.Generator().manual_seed(5)
    # small integers: every butterfly sum is exact, so only the final FP32
    # scaling rounds, once
    x = torch.randint(-6, 7, (4, 384), generator=generator).float()
    integer = np.rint(matrix * np.sqrt(128.0)).astype(np.int64)  # +-1 entries
    exact = x.numpy().astype(np.int64) @ integer.T
    want = exact.astype(np.float32) * np.float32(1 / np.sqrt(128.0))
    assert np.array_equal(rotate_blocks(x, signs).numpy(), want)
    y = torch.randn(3, 384, generator=generator)
    np.testing.assert_allclose(rotate_blocks(y, signs).double().numpy(),
                               y.double().numpy() @ matrix.T, rtol=0, atol=2e-6)
    # the rotation is orthogonal: it keeps every row's norm
    np.testing.assert_allclose(np.linalg.norm(rotate_blocks(y, signs).numpy(), axis=1),
                               np.linalg.norm(y.numpy(), axis=1), rtol=1e-6)
    assert torch.equal(rotate_blocks(y, None), y)


@pytest.mark.parametrize("keep", [1, 80, 127, 128])
def test_mask_keeps_the_largest_magnitudes_lower_coordinates_first(keep):
    generator = torch.Generator().manual_seed(keep)
    # many exact ties in magnitude, including across signs
    x = torch.randint(-3, 4, (5, 256), generator=generator).float()
    got = mask_rotated_blocks(x, keep).reshape(-1, 128).numpy()
    for row, values in enumerate(x.reshape(-1, 128).numpy()):
        order = sorted(range(128), key=lambda c: (-abs(values[c]), c))
        want = np.zeros(128, np.float32)
        want[order[:keep]] = values[order[:keep]]
        assert np.array_equal(got[row], want)


def test_known_block_ternarisation():
    """One block whose trits, scale and residual are fixed by hand.

    32 values of magnitude 4, 32 of 2, 64 of 1/2: mean |v| = 1.75, threshold
    1.225, so the 4s and 2s are kept (scale 3) and the halves dropped; the
    residual is (32 * 1 + 32 * 1 + 64 * 0.25) / 128 = 0.625.
    """
    block = np.array([4.0] * 32 + [2.0] * 32 + [0.5] * 64)
    sign = np.where(np.arange(128) % 3 == 0, -1.0, 1.0)
    values = np.zeros((1, 2, 256))
    values[0, 0, :128] = block * sign  # gate row, block 0
    values[0, 1, 128:] = -block * sign  # up row, block 1
    codes, statistics = build_sketch(torch.from_numpy(values).bfloat16())
    trits = decode_by_address(codes.numpy(), 1, 256)
    assert np.array_equal(trits[0, 0, :128], np.where(block > 1.225, sign, 0))
    assert np.array_equal(trits[0, 1, 128:], -np.where(block > 1.225, sign, 0))
    assert not trits[0, 0, 128:].any() and not trits[0, 1, :128].any()
    stats = statistics.float().numpy()  # [E, 2 I, blocks, 2]
    assert stats[0, 0, 0].tolist() == [3.0, 0.625]
    assert stats[0, 1, 1].tolist() == [3.0, 0.625]
    assert stats[0, 0, 1].tolist() == [0.0, 0.0]
    assert statistics.stride() == (4 * 2, 1, 4, 2)


@pytest.mark.parametrize("width,hidden,rotated", [(8, 256, False), (48, 384, True),
                                                  (40, 128, False), (24, 512, True)])
def test_codes_and_statistics_follow_the_rule(width, hidden, rotated):
    """Random weights: the address decoder, the library decoder and a float64
    TWN restatement agree; statistics to FP16 rounding. A trit may differ from
    the float64 rule only where |v| sits within FP32 rounding of the threshold."""
    generator = torch.Generator().manual_seed(width + hidden)
    weights = (torch.randn(2, 2 * width, hidden, generator=generator) * 0.05).bfloat16()
    signs = block_hadamard_signs(hidden, "cpu") if rotated else None
    codes, statistics = build_sketch(weights, signs)
    assert codes.shape == (2, sketch_storage_bytes(2 * width, hidden))
    by_address = decode_by_address(codes.numpy(), width, hidden)
    assert np.array_equal(unpack_sketch(codes, 2 * width, hidden).numpy(), by_address)
    value = weights.double().numpy()
    if rotated:
        value = value @ rotation_matrix(signs.numpy()).T
    blocks = value.reshape(2, 2 * width, hidden // 128, 128)
    trits = by_address.reshape(blocks.shape)
    stats = statistics.float().numpy()
    for e in range(2):
        for row in range(2 * width):
            for b in range(hidden // 128):
                want, scale, residual = twn(blocks[e, row, b])
                near = np.abs(np.abs(blocks[e, row, b]) - 0.7 * np.abs(blocks[e, row, b]).mean())
                differ = trits[e, row, b] != want
                assert (near[differ] < 1e-6).all()
                if not differ.any():
                    np.testing.assert_allclose(stats[e, row, b], [scale, residual],
                                               rtol=2e-3, atol=1e-7)


def test_unused_bytes_hold_the_zero_code():
    """Width 48: 2 ceil(48 / 5) = 20 code bytes per coordinate in a 32-byte
    stride; bytes 20..31 are padding and decode to zero trits."""
    codes, _ = build_sketch(torch.randn(1, 96, 256).bfloat16())
    for coordinate in range(256):
        for byte in range(20, 32):
            address = stored_address(48, 256, coordinate // 128, coordinate % 128, byte)
            assert codes[0, address] == ZERO_CODE


def test_build_is_independent_of_chunking():
    weights = torch.randn(5, 2 * 64, 256).bfloat16()
    signs = block_hadamard_signs(256, "cpu")
    whole = build_sketch(weights, signs, chunk=8)
    split = build_sketch(weights, signs, chunk=2)
    assert torch.equal(whole[0], split[0]) and torch.equal(whole[1], split[1])


@pytest.mark.parametrize("keep", [80, 128])
@pytest.mark.parametrize("input_is_rotated", [False, True])
def test_sketch_feature_and_its_gradient_from_explicit_matrices(keep, input_is_rotated):
    hidden, width, tokens = 256, 16, 3
    generator = torch.Generator().manual_seed(keep + input_is_rotated)
    signs = block_hadamard_signs(hidden, "cpu")
    codes, statistics = build_sketch(
        torch.randn(1, 2 * width, hidden, generator=generator) * 0.1, signs=signs)
    x = torch.randn(tokens, hidden, generator=generator, dtype=torch.float32)
    feature = differentiable_sketch_feature(
        x.clone().requires_grad_(), codes[0], statistics[0], signs,
        input_is_rotated=input_is_rotated, screen_coordinates=keep)
    # explicit matrices: sketch S [2I, H] (trit * block scale), rotation R, mask M(x)
    trits = decode_by_address(codes.numpy(), width, hidden)[0].astype(np.float64)
    scale = np.repeat(statistics[0, :, :, 0].double().numpy(), 128, axis=1)
    sketch = trits * scale
    rotation = np.eye(hidden) if input_is_rotated else rotation_matrix(signs.numpy())
    xs = x.double().numpy()
    for t in range(tokens):
        rotated = rotation @ xs[t]
        kept = np.zeros(hidden, bool)
        for b in range(hidden // 128):
            values = rotated[128 * b:128 * (b + 1)]
            order = sorted(range(128), key=lambda c: (-abs(values[c]), c))[:keep]
            kept[128 * b + np.array(order)] = True
        projection = sketch @ np.where(kept, rotated, 0.0)
        g, u = projection[:width], projection[width:]
        g16 = torch.tensor(g).float().bfloat16().double().numpy()
        u16 = torch.tensor(u).float().bfloat16().double().numpy()
        sigma = 1 / (1 + np.exp(-g16))
        want = g16 * sigma * u16
        np.testing.assert_allclose(feature[t].double().detach().numpy(), want,
                                   rtol=2e-2, atol=1e-3)
        # d sum(phi(g) u) / dx = (A_g^T (phi'(g) u) + A_u^T phi(g)), A = S M R
        a = sketch * kept[None, :] @ rotation
        slope = sigma * (1 + g16 * (1 - sigma))
        gradient = a[:width].T @ (slope * u16) + a[width:].T @ (g16 * sigma)
        xt = x[t:t + 1].clone().requires_grad_()
        value = differentiable_sketch_feature(
            xt, codes[0], statistics[0], signs, input_is_rotated=input_is_rotated,
            screen_coordinates=keep)
        (got,) = torch.autograd.grad(value.float().sum(), xt)
        np.testing.assert_allclose(got[0].double().numpy(), gradient, rtol=3e-2,
                                   atol=3e-3 * np.abs(gradient).max())
        if input_is_rotated:
            assert not got[0].numpy()[~kept].any()
