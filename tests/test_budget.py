"""Read-plan pricing: the reference's known answers (tests/test_budget.py:6-82)."""

import json

import pytest

from calibration_free_moe.reader.budget import (
    PaidRound,
    compile_budget,
    load_layer_budgets,
    sketch_code_stride,
    sketch_storage_bytes,
)


@pytest.mark.parametrize("screen_keep,coordinates", [(1.0, 128), (0.625, 80)])
def test_sketch_plan_and_paid_reads(screen_keep, coordinates):
    plan = compile_budget(
        hidden_size=2048, expert_width=1024, top_k=8, retention=0.15, screen_keep=screen_keep
    )
    n, h, f = 8192, 2048, plan.final_count
    assert plan.rounds == (PaidRound(0, 0, n, f), PaidRound(0, h, f, f))
    assert plan.sketch_read_bytes() == 8 * 16 * (coordinates * 416 + 2 * 4096)
    assert plan.sketch_read_bytes(sectors=False) == 8 * 16 * (coordinates * 410 + 2 * 4096)
    assert plan.sketch_read_bytes(residual=False) == 8 * 16 * (coordinates * 416 + 4096)
    assert plan.selected_weight_bytes() == 2 * h * 3 * f
    assert plan.selection_read_bytes() == 12 * n
    assert plan.native_read_bytes() == 2 * 3 * n * h
    assert plan.recovery_read_bytes(32) == 64 * (n - f + h)


def test_dense_bypass():
    dense = compile_budget(hidden_size=128, expert_width=32, top_k=4, retention=1)
    assert dense.rounds == (PaidRound(0, 128, 128, 128),)
    assert dense.sketch_read_bytes() == 0
    assert dense.selection_read_bytes() == 0


@pytest.mark.parametrize(("retention", "f"), [(2.5 / 32, 2), (3.5 / 32, 4), (3 / 32, 3)])
def test_nearest_even_rounding(retention, f):
    plan = compile_budget(hidden_size=128, expert_width=16, top_k=2, retention=retention)
    assert (plan.final_count, plan.completion_count) == (f, f)


@pytest.mark.parametrize("screen_keep", [0.625, 1.0])
def test_unaligned_sketch_metadata_width_is_rejected(screen_keep):
    with pytest.raises(ValueError, match=r"divisible by 16.*sketch metadata"):
        compile_budget(
            hidden_size=128, expert_width=88, top_k=1, retention=0.125, screen_keep=screen_keep
        )


@pytest.mark.parametrize(
    ("hidden", "width", "retention"),
    [(0, 16, 0.1), (64, 16, 0.1), (128, 0, 0.1), (128, 16, 0), (128, 16, float("nan")),
     (128, 16, 0.01)],
)
def test_invalid_budgets(hidden, width, retention):
    with pytest.raises(ValueError):
        compile_budget(hidden_size=hidden, expert_width=width, top_k=2, retention=retention)


def test_partial_screen_needs_pruning():
    with pytest.raises(ValueError, match="partial-sketch"):
        compile_budget(hidden_size=128, expert_width=16, top_k=2, retention=1.0,
                       screen_keep=0.5)


@pytest.mark.parametrize(
    "width,stride,storage",
    # OLMoE, Qwen3-30B-A3B and the 256-expert shape at H = 2048 (block-paired tail)
    [(1024, 416, 851_968), (768, 320, 655_360), (512, 208, 425_984)],
)
def test_layout_sizes_at_benchmark_shapes(width, stride, storage):
    assert sketch_code_stride(2 * width) == stride
    assert sketch_storage_bytes(2 * width, 2048) == storage


@pytest.mark.parametrize(
    "width,retention,keep,total",
    # Per-token sector-priced read cost at T = 1 of the benchmark configurations
    # (point score, rank-32 map), as tabulated for the baseline.
    [
        (1024, 0.123, 0.625, 17_796_096),
        (768, 0.123, 0.625, 13_462_272),
        (768, 0.06, 0.625, 8_731_584),
        (768, 0.25, 0.625, 22_996_992),
    ],
)
def test_benchmark_read_cost(width, retention, keep, total):
    h, k, rank = 2048, 8, 32
    plan = compile_budget(hidden_size=h, expert_width=width, top_k=k, retention=retention,
                          screen_keep=keep)
    charged = (
        plan.selected_weight_bytes()
        + plan.recovery_read_bytes(rank)
        + plan.selection_read_bytes(geometry=False)
        + plan.sketch_read_bytes(residual=False)
        + h
    )
    assert charged == total


def test_load_layer_budgets(tmp_path):
    path = tmp_path / "allocation.json"
    path.write_text(json.dumps({
        "final_counts": [100, 200],
        "dimensions": {"num_hidden_layers": 2, "hidden_size": 256, "expert_width": 64,
                       "num_experts_per_tok": 4},
        "screen_keep": 0.625,
    }))
    plans = load_layer_budgets(path, layers=2, hidden_size=256, expert_width=64, top_k=4,
                               screen_keep=0.625)
    assert [p.final_count for p in plans] == [100, 200]
    assert all(p.screen_coordinates == 80 for p in plans)
    with pytest.raises(ValueError):
        load_layer_budgets(path, layers=3, hidden_size=256, expert_width=64, top_k=4,
                           screen_keep=0.625)
