"""The screen's resident 2-bit layout (cfmoe_pack_trit_planes) against the
sketch codes it repacks (needs an MI355X).

The expected words are built here from `unpack_sketch` (the trits of the
reference's five-per-byte codes, sketch.py:209-232) by the layout rule alone:
for expert e, block b, row tile rt and lane l, word h of uint2
((e B + b) RT + rt) 64 + l holds digit t + 1 of row 16 rt + l % 16 at
coordinate 64 h + 16 (l / 16) + k in bits 8 (k % 4) + 2 (k / 4).
"""

import ctypes

import numpy as np
import pytest
import torch

from calibration_free_moe.reader import _ext
from calibration_free_moe.reader.budget import compile_budget
from calibration_free_moe.reader.progressive import _dims
from calibration_free_moe.reader.sketch import block_hadamard_signs, build_sketch, unpack_sketch

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda:0")


def expected_words(trits: np.ndarray) -> np.ndarray:
    """uint32 words of the layout from int8 trits [E, 2I, H] (rows gate then up)."""
    e, rows, h = trits.shape
    blocks, tiles = h // 128, rows // 16
    digits = (trits.astype(np.int64) + 1).reshape(e, rows, blocks, 128).transpose(0, 2, 1, 3)
    # [e, block, tile, row in tile, half, coordinate group, k]
    digits = digits.reshape(e, blocks, tiles, 16, 2, 4, 16)
    k = np.arange(16)
    shifts = 8 * (k % 4) + 2 * (k // 4)
    words = (digits << shifts).sum(-1)
    # lane = 16 * coordinate group + row in tile; the two halves sit together
    words = words.transpose(0, 1, 2, 5, 3, 4)
    return words.reshape(-1).astype(np.uint32)


@pytest.mark.parametrize("hidden,width,experts",
                         [(256, 256, 3), (384, 320, 2), (384, 256, 2), (2048, 512, 2)])
def test_trit_planes_match_unpacked_codes(hidden, width, experts):
    g = torch.Generator().manual_seed(hidden + width)
    gate_up = (torch.randn(experts, 2 * width, hidden, generator=g) * 0.02).bfloat16().to(DEVICE)
    codes, _ = build_sketch(gate_up, block_hadamard_signs(hidden, DEVICE))
    trits = unpack_sketch(codes.cpu(), 2 * width, hidden).numpy()
    assert set(np.unique(trits)) <= {-1, 0, 1}
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=2, retention=0.1,
                          screen_keep=0.625)
    dims = _dims(plan, experts, 0)
    size = _ext.trit_plane_bytes(dims)
    assert size == experts * (hidden // 128) * width * 64
    planes = torch.full((size // 4,), -1, dtype=torch.int32, device=DEVICE)
    _ext.check(_ext.library().cfmoe_pack_trit_planes(
        ctypes.byref(dims), codes.data_ptr(), planes.data_ptr(),
        torch.cuda.current_stream(DEVICE).cuda_stream))
    torch.cuda.synchronize()
    got = planes.cpu().numpy().view(np.uint32)
    want = expected_words(trits)
    mismatch = np.flatnonzero(got != want)
    assert mismatch.size == 0, f"{mismatch.size} of {got.size} words differ, first at {mismatch[:5]}"
    # the inverse repacking gives back every code byte, the bytes that carry
    # no channel (121, five zero trits) included
    back = torch.zeros_like(codes)
    _ext.check(_ext.library().cfmoe_unpack_trit_planes(
        ctypes.byref(dims), planes.data_ptr(), back.data_ptr(),
        torch.cuda.current_stream(DEVICE).cuda_stream))
    torch.cuda.synchronize()
    differ = np.flatnonzero((back != codes).cpu().numpy().reshape(-1))
    assert differ.size == 0, f"{differ.size} of {codes.numel()} code bytes differ, first at {differ[:5]}"


def test_reader_keeps_planes_and_rebuilds_codes():
    """A screened reader holds no copy of the codes: `sketch_codes` rebuilds
    them from the resident planes, equal to the codes it was given."""
    from calibration_free_moe.reader.progressive import ProgressiveReader, channel_major_down

    hidden, width, experts = 512, 256, 4
    g = torch.Generator().manual_seed(5)
    gate_up = (torch.randn(experts, 2 * width, hidden, generator=g) * 0.02).bfloat16().to(DEVICE)
    down = (torch.randn(experts, hidden, width, generator=g) * 0.02).bfloat16().to(DEVICE)
    codes, statistics = build_sketch(gate_up, block_hadamard_signs(hidden, DEVICE))
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=2, retention=0.123,
                          screen_keep=0.625)
    reader = ProgressiveReader(gate_up, channel_major_down(down), None, None, plan, 4,
                               sketch=(codes, statistics))
    assert reader._sketch_codes is None and reader.sketch_trit_planes.numel() > 0
    rebuilt = reader.sketch_codes
    assert torch.equal(rebuilt, codes)
    # a held rebuild is returned again (no second unpack); once released, a
    # read rebuilds it
    assert reader.sketch_codes is rebuilt
    del rebuilt
    assert torch.equal(reader.sketch_codes[1], codes[1])
    # resident: the planes (64 I B bytes per expert) and the FP16 statistics
    planes_bytes = experts * 64 * width * (hidden // 128)
    assert reader.sketch_trit_planes.numel() * 4 == planes_bytes
    assert reader.sketch_resident_bytes == planes_bytes + statistics.numel() * 2
    dense = ProgressiveReader(gate_up, channel_major_down(down), None, None,
                              compile_budget(hidden_size=hidden, expert_width=width, top_k=2,
                                             retention=1.0), 4, sketch=(codes, statistics))
    assert dense.sketch_codes is codes and dense.sketch_trit_planes.numel() == 0
    assert dense.sketch_resident_bytes == codes.numel() + statistics.numel() * 2
