"""Read plans and their per-token byte prices.

Two kinds of check:

* a byte-level model built here from the packed layout itself: the code bytes
  of every kept coordinate are located by address in the stored format and the
  32-byte sectors they touch are counted, then compared with the plan's closed
  forms over a grid of shapes (odd block counts, tail strides, widths that are
  not multiples of five);
* known answers stated by the reference (its tests/test_budget.py:6-82 and the
  per-token totals of the benchmark configurations), kept here as data only.
"""

import json
from math import ceil

import pytest

from calibration_free_moe.reader.budget import (
    PaidRound,
    compile_budget,
    load_layer_budgets,
    sketch_code_stride,
    sketch_storage_bytes,
)

SECTOR = 32


def stored_address(width: int, hidden: int, block: int, coordinate: int, byte: int) -> int:
    """Address of code byte `byte` of (block, coordinate) in one expert's codes,
    from the storage rule: whole 32-byte tiles coordinate-major per block, a
    16-byte remainder in rows shared by the block pair (block // 2)."""
    stride = sketch_code_stride(2 * width)
    body = stride // SECTOR * SECTOR
    blocks = hidden // 128
    if byte < body:
        return (block * 128 + coordinate) * body + byte
    return blocks * 128 * body + ((block // 2) * 128 + coordinate) * 32 + (block % 2) * 16 + byte - body


def walked_sketch_bytes(width: int, hidden: int, top_k: int, keep: int, residual: bool,
                        sectors: bool) -> int:
    """One token's screen reads, counted byte by byte from the layout."""
    useful = 2 * ceil(width / 5)  # gate and up bytes of five channels each
    per_expert = 0
    for block in range(hidden // 128):
        for coordinate in range(keep):
            addresses = [stored_address(width, hidden, block, coordinate, b) for b in range(useful)]
            if sectors:
                per_expert += SECTOR * len({a // SECTOR for a in addresses})
            else:
                per_expert += len(addresses)
        plane = 2 * 2 * width  # fp16 value per gate/up row
        plane = -(-plane // SECTOR) * SECTOR if sectors else plane
        per_expert += plane * (2 if residual else 1)
    return top_k * per_expert


GRID = [(h, i) for h in (128, 384, 2048) for i in (16, 48, 80, 512, 704, 768, 1024)]


@pytest.mark.parametrize("hidden,width", GRID)
def test_layout_fits_the_storage_and_never_splits_a_sector(hidden, width):
    storage = sketch_storage_bytes(2 * width, hidden)
    useful = 2 * ceil(width / 5)
    seen = set()
    for block in range(hidden // 128):
        for coordinate in (0, 1, 77, 127):
            addresses = [stored_address(width, hidden, block, coordinate, b) for b in range(useful)]
            assert max(addresses) < storage
            # a 32-byte run of one coordinate stays inside one sector
            for start in range(0, useful, SECTOR):
                run = addresses[start:start + SECTOR]
                assert len({a // SECTOR for a in run}) == 1
            assert not seen.intersection(addresses)
            seen.update(addresses)


@pytest.mark.parametrize("hidden,width", GRID)
@pytest.mark.parametrize("keep", [0.625, 1.0])
def test_sketch_price_equals_the_walked_layout(hidden, width, keep):
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=3, retention=0.25,
                          screen_keep=keep)
    coordinates = plan.screen_coordinates
    assert coordinates == ceil(128 * keep)
    for residual in (False, True):
        for sectors in (False, True):
            assert plan.sketch_read_bytes(residual=residual, sectors=sectors) == \
                walked_sketch_bytes(width, hidden, 3, coordinates, residual, sectors)


# Known answers. Each row: plan arguments, then {method call: value}.
OLMOE = dict(hidden_size=2048, expert_width=1024, top_k=8, retention=0.15)
KNOWN_PRICES = [
    (dict(OLMOE, screen_keep=1.0), {
        "sketch": 8 * 16 * (128 * 416 + 2 * 4096),
        "sketch_logical": 8 * 16 * (128 * 410 + 2 * 4096),
        "sketch_point": 8 * 16 * (128 * 416 + 4096),
    }),
    (dict(OLMOE, screen_keep=0.625), {
        "sketch": 8 * 16 * (80 * 416 + 2 * 4096),
        "sketch_logical": 8 * 16 * (80 * 410 + 2 * 4096),
        "sketch_point": 8 * 16 * (80 * 416 + 4096),
    }),
]


def priced(plan, name):
    return {
        "sketch": lambda: plan.sketch_read_bytes(),
        "sketch_logical": lambda: plan.sketch_read_bytes(sectors=False),
        "sketch_point": lambda: plan.sketch_read_bytes(residual=False),
    }[name]()


@pytest.mark.parametrize("arguments,answers", KNOWN_PRICES)
def test_known_sketch_prices(arguments, answers):
    plan = compile_budget(**arguments)
    for name, value in answers.items():
        assert priced(plan, name) == value, name
    n, h, f = 8192, 2048, plan.final_count
    assert plan.rounds == (PaidRound(0, 0, n, f), PaidRound(0, h, f, f))
    assert (plan.selected_weight_bytes(), plan.selection_read_bytes(), plan.native_read_bytes(),
            plan.recovery_read_bytes(32)) == (6 * h * f, 12 * n, 6 * n * h, 64 * (n - f + h))


# Per-token sector-priced read cost at T = 1 of the benchmark configurations
# (point score, rank-32 map, H = 2048, K = 8): width, retention, keep, total.
KNOWN_TOTALS = [
    (1024, 0.123, 0.625, 17_796_096),
    (768, 0.123, 0.625, 13_462_272),
    (768, 0.06, 0.625, 8_731_584),
    (768, 0.25, 0.625, 22_996_992),
    (512, 0.123, 0.625, 9_128_448),
    (512, 0.123, 1.0, 10_504_704),
]


@pytest.mark.parametrize("width,retention,keep,total", KNOWN_TOTALS)
def test_known_totals_at_the_benchmark_shapes(width, retention, keep, total):
    plan = compile_budget(hidden_size=2048, expert_width=width, top_k=8, retention=retention,
                          screen_keep=keep)
    parts = (plan.selected_weight_bytes(), plan.recovery_read_bytes(32),
             plan.selection_read_bytes(geometry=False), plan.sketch_read_bytes(residual=False),
             2048)
    assert sum(parts) == total


@pytest.mark.parametrize("width,stride,storage",
                         [(1024, 416, 851_968), (768, 320, 655_360), (512, 208, 425_984)])
def test_known_layout_sizes(width, stride, storage):
    assert (sketch_code_stride(2 * width), sketch_storage_bytes(2 * width, 2048)) == (stride, storage)


def test_final_count_rounds_half_to_even():
    # known answers at N = 32, then the rule over every half-integer target
    for retention, final in ((2.5 / 32, 2), (3.5 / 32, 4), (3 / 32, 3)):
        plan = compile_budget(hidden_size=128, expert_width=16, top_k=2, retention=retention)
        assert plan.final_count == plan.completion_count == final
    for twice in range(3, 64):
        plan = compile_budget(hidden_size=128, expert_width=16, top_k=2, retention=twice / 64)
        half, odd = divmod(twice, 2)
        assert plan.final_count == (half + (half % 2) if odd else half)


def test_full_retention_is_one_dense_stage():
    plan = compile_budget(hidden_size=128, expert_width=32, top_k=4, retention=1)
    assert plan.rounds == (PaidRound(0, 128, 128, 128),)
    assert plan.sketch_read_bytes() == plan.selection_read_bytes() == 0


REJECTED = [
    (dict(hidden_size=0, expert_width=16, top_k=2, retention=0.1), "positive"),
    (dict(hidden_size=64, expert_width=16, top_k=2, retention=0.1), "divisible by 128"),
    (dict(hidden_size=128, expert_width=0, top_k=2, retention=0.1), "positive"),
    (dict(hidden_size=128, expert_width=16, top_k=2, retention=0), r"\(0, 1\]"),
    (dict(hidden_size=128, expert_width=16, top_k=2, retention=float("nan")), r"\(0, 1\]"),
    (dict(hidden_size=128, expert_width=16, top_k=2, retention=0.01), "1 <= F <= N"),
    (dict(hidden_size=128, expert_width=88, top_k=1, retention=0.125), "divisible by 16"),
    (dict(hidden_size=128, expert_width=88, top_k=1, retention=0.125, screen_keep=0.625),
     "divisible by 16"),
    (dict(hidden_size=128, expert_width=16, top_k=2, retention=1.0, screen_keep=0.5),
     "partial-sketch"),
]


@pytest.mark.parametrize("arguments,message", REJECTED)
def test_invalid_plans_raise(arguments, message):
    with pytest.raises(ValueError, match=message):
        compile_budget(**arguments)


def test_layer_allocation_file(tmp_path):
    path = tmp_path / "allocation.json"
    dimensions = {"num_hidden_layers": 2, "hidden_size": 256, "expert_width": 64,
                  "num_experts_per_tok": 4}
    path.write_text(json.dumps({"final_counts": [100, 200], "dimensions": dimensions,
                                "screen_keep": 0.625}))
    shape = dict(hidden_size=256, expert_width=64, top_k=4, screen_keep=0.625)
    plans = load_layer_budgets(path, layers=2, **shape)
    assert [(p.final_count, p.screen_coordinates) for p in plans] == [(100, 80), (200, 80)]
    for layers, keep in ((3, 0.625), (2, 1.0)):
        with pytest.raises(ValueError):
            load_layer_budgets(path, layers=layers, **dict(shape, screen_keep=keep))
    path.write_text(json.dumps({"final_counts": [100, 256]}))
    with pytest.raises(ValueError, match="candidate_count"):
        load_layer_budgets(path, layers=2, **shape)
