"""Read plans of the sparse expert reader and their per-token byte prices.

Symbols: H hidden size, I intermediate channels per expert, K routed experts
per token, N = K * I candidate channels, F channels kept per token.

Mirrors the plan API of `calibration_free_moe/reader/budget.py` in the
reference (`compile_budget` budget.py:150-206, `BudgetPlan` :52-147,
`PaidRound` :36-49, layout sizes :13-33, `load_layer_budgets` :209-256) so that
runtime bindings construct plans unchanged. Prices are in 32-byte sectors, the
unit the reference's read cost is defined in; the MI355X kernels are measured
against the same algorithmic bytes.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from math import ceil, isfinite
from pathlib import Path

SECTOR = 32


def _sector_ceil(size: int) -> int:
    return -(-size // SECTOR) * SECTOR


def sketch_code_stride(rows: int) -> int:
    """Code bytes of one rotated coordinate of one expert (budget.py:13-19).

    Gate and up channels alternate by byte: byte 2m carries gate channels
    5m..5m+4 and byte 2m+1 the same up channels, one balanced trit each, so a
    coordinate needs 2 * ceil(I / 5) bytes, padded to 16 bytes.
    """
    useful = 2 * ((rows // 2 + 4) // 5)
    return (useful + 15) // 16 * 16


def sketch_storage_bytes(rows: int, hidden: int) -> int:
    """Packed code bytes of one expert (budget.py:22-33).

    Whole 32-byte tiles of every coordinate are stored coordinate-major; a
    16-byte remainder is paired with the same coordinate of the neighbouring
    rotation block so that each tile load stays inside one sector.
    """
    stride = sketch_code_stride(rows)
    blocks = hidden // 128
    body = stride - stride % SECTOR
    tail = stride % SECTOR
    return blocks * 128 * body + ((blocks + 1) // 2) * 128 * 2 * tail


@dataclass(frozen=True)
class PaidRound:
    """One stage of a plan (budget.py:36-49).

    `entering_count` channels enter and the best `retained_count` leave. A stage
    with input_end == 0 is the sketch screen; input_end == hidden_size computes
    the surviving channels exactly from their native rows.
    """

    input_start: int
    input_end: int
    entering_count: int
    retained_count: int


@dataclass(frozen=True)
class BudgetPlan:
    """Token-independent read plan of one MoE layer (budget.py:52-147)."""

    hidden_size: int
    expert_width: int
    top_k: int
    completion_count: int
    final_count: int
    rounds: tuple[PaidRound, ...]
    screen_coordinates: int = 128

    def __post_init__(self) -> None:
        # 80-channel screen tiles read FP16 metadata in whole sectors only when
        # I is a multiple of 16 (budget.py:71-78).
        if self.expert_width % 16:
            raise ValueError(
                "Reader expert width must be divisible by 16 "
                "for sector-aligned sketch metadata"
            )

    @property
    def candidate_count(self) -> int:
        """N = K * I, every channel of the token's routed experts."""
        return self.top_k * self.expert_width

    def native_read_bytes(self) -> int:
        """Dense BF16 gate, up and down bytes of one token's routed experts."""
        return 6 * self.candidate_count * self.hidden_size

    def selected_weight_bytes(self) -> int:
        """BF16 gate/up rows of the exactly computed channels plus down rows of F."""
        return 2 * self.hidden_size * (2 * self.completion_count + self.final_count)

    def sketch_read_bytes(self, residual: bool = True, sectors: bool = True) -> int:
        """Sketch bytes one token's screen reads (budget.py:102-127).

        Per routed expert and rotation block: the kept coordinates' code runs
        (2 * ceil(I / 5) bytes each) and the FP16 scale plane of all 2 I rows,
        plus the residual-variance plane when the score reads it. With
        sectors=True each run is priced in whole 32-byte sectors.
        """
        if self.completion_count == self.candidate_count:
            return 0
        price = _sector_ceil if sectors else (lambda size: size)
        blocks = self.hidden_size // 128
        codes = self.screen_coordinates * price(2 * ((self.expert_width + 4) // 5))
        planes = price(4 * self.expert_width) * (2 if residual else 1)
        return self.top_k * blocks * (codes + planes)

    def recovery_read_bytes(self, rank: int) -> int:
        """BF16 encoder rows of the N - F skipped channels plus the decoder U."""
        return 2 * rank * (self.candidate_count - self.final_count + self.hidden_size)

    def selection_read_bytes(self, geometry: bool = True) -> int:
        """FP32 down-column norm (and two geometry values) per screened candidate."""
        if self.completion_count >= self.candidate_count:
            return 0
        return (12 if geometry else 4) * self.candidate_count


def _check_positive(name: str, value: object) -> None:
    if type(value) is not int or value <= 0:
        raise ValueError(f"{name} must be a positive integer")


def _check_fraction(name: str, value: object) -> None:
    if (
        isinstance(value, bool)
        or not isinstance(value, (int, float))
        or not isfinite(value)
        or not 0 < value <= 1
    ):
        raise ValueError(f"{name} must be finite and in (0, 1]")


def compile_budget(
    *,
    hidden_size: int,
    expert_width: int,
    top_k: int,
    retention: float,
    screen_keep: float = 1.0,
) -> BudgetPlan:
    """Compile a retention fraction into a read plan (budget.py:150-206).

    F = retention * N rounded half to even (Python's `round`); 1 <= F <= N.
    Full retention compiles to a single dense stage without a screen. The
    partial screen keeps ceil(128 * screen_keep) rotated coordinates per block.
    Invalid dimensions or budgets raise ValueError.
    """
    _check_positive("hidden_size", hidden_size)
    _check_positive("expert_width", expert_width)
    _check_positive("top_k", top_k)
    _check_fraction("retention", retention)
    _check_fraction("screen_keep", screen_keep)
    n = top_k * expert_width
    final = round(retention * n)
    if not 1 <= final <= n:
        raise ValueError("Rounded budgets must satisfy 1 <= F <= N")
    if hidden_size % 128:
        raise ValueError("Sketch hidden width must be divisible by 128")
    kept = ceil(screen_keep * 128)
    if kept < 128 and final == n:
        raise ValueError(
            "A partial-sketch screen needs fewer selected than candidate channels"
        )
    if final == n:
        rounds: tuple[PaidRound, ...] = (PaidRound(0, hidden_size, n, final),)
    else:
        rounds = (PaidRound(0, 0, n, final), PaidRound(0, hidden_size, final, final))
    return BudgetPlan(hidden_size, expert_width, top_k, final, final, rounds, kept)


def load_layer_budgets(
    path: str | Path,
    *,
    layers: int,
    hidden_size: int,
    expert_width: int,
    top_k: int,
    screen_keep: float,
) -> list[BudgetPlan]:
    """Compile one plan per MoE layer from an allocation JSON (budget.py:209-256).

    The file holds "final_counts" (one F per layer, 1 <= F < N) and optionally
    "dimensions" and "screen_keep", which must match the model and reader.
    """
    allocation = json.loads(Path(path).read_text())
    counts = allocation["final_counts"]
    if not isinstance(counts, list) or len(counts) != layers:
        raise ValueError("Layer allocation must give one count per MoE layer")
    expected = {
        "num_hidden_layers": layers,
        "hidden_size": hidden_size,
        "expert_width": expert_width,
        "num_experts_per_tok": top_k,
    }
    dimensions = allocation.get("dimensions")
    if dimensions is not None and any(
        dimensions.get(key) != value for key, value in expected.items()
    ):
        raise ValueError("Layer allocation dimensions do not match the model")
    if "screen_keep" in allocation and ceil(128 * allocation["screen_keep"]) != ceil(
        128 * screen_keep
    ):
        raise ValueError("Layer allocation screen_keep does not match the reader")
    n = top_k * expert_width
    if any(type(f) is not int or not 1 <= f < n for f in counts):
        raise ValueError("Layer counts must be integers in [1, candidate_count)")
    return [
        compile_budget(
            hidden_size=hidden_size,
            expert_width=expert_width,
            top_k=top_k,
            retention=f / n,
            screen_keep=screen_keep,
        )
        for f in counts
    ]
