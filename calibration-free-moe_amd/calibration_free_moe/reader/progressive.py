"""Sparse decode operator for the routed experts of one MoE layer (MI355X).

Drop-in for `calibration_free_moe/reader/progressive.py` of the reference
(AidenGeunGeun/calibration-free-moe): same `ProgressiveReader` constructor,
call signature, attributes and `report()`, same `ReaderWorkspace`, same module
names. The device work is done by hand-written HIP kernels for gfx950 in
libcfmoe_reader.so (C ABI: include/cfmoe_reader.h), called through ctypes on
the caller's current stream (`prepare_input` on a side stream that the next
call joins). There is no Triton, no CPU fallback: without the library every
call raises RuntimeError.

Stages of one call (reference progressive.py:13-24):

1. Sort each token's K experts by id; rotate the input by the block-Hadamard
   transform and keep each block's largest |R x| coordinates.
2. Screen: score every candidate channel from the resident ternary sketch.
3. Keep the top-F channels per token (or those above a threshold).
4. Compute the kept channels exactly from the native BF16 gate/up rows.
5. Down projection of the kept channels.
6. Recovery: encode the skipped channels' sketch activations into a rank-R
   latent; decode it with U and mix experts by router weight.

Numerics. The screen's per-block dot products are formed exactly (integer sums
of trits times the rotated input on a 21-bit grid relative to the block
maximum) and rounded once to FP32, so the selected channels are the same at
every batch size and in the CPU oracle (oracle/). FP32 chains after that have
one fixed order.
"""

from __future__ import annotations

import ctypes
import weakref
from math import ceil
from typing import Literal

import torch
from torch import Tensor

from calibration_free_moe.activation import GatedActivation
from calibration_free_moe.reader import _ext
from calibration_free_moe.reader.budget import (
    BudgetPlan,
    sketch_code_stride,
    sketch_storage_bytes,
)
from calibration_free_moe.reader.sketch import block_hadamard_signs, build_sketch


def channel_major_down(weight: Tensor) -> Tensor:
    """One physical [E, I, H] allocation viewed as the logical [E, H, I] weight.

    Each channel's H outputs are contiguous (progressive.py:56-62), which is the
    layout the down kernel streams.
    """
    return weight.transpose(1, 2).contiguous().transpose(1, 2)


# (token, expert) pairs per expert-major block (progressive.py:80-81).
GROUP_ROWS = 16
# Batch size from which the kept channels are computed expert-major (the
# reference's crossover, progressive.py:82-86, is 32 on its GPUs; on MI355X
# the grouped rows already pay at 16 tokens). The screen is expert-major at
# every batch size here, so GROUPED_SCREEN_TOKENS only keeps the API.
GROUPED_TOKENS = 16
GROUPED_SCREEN_TOKENS = 64
# Radix selection constants of the reference's small-batch path
# (progressive.py:106-114); reported by `report()`.
RADIX_BITS = 12
RADIX_HASH_BITS = 8
RADIX_CAPACITY = 128
RADIX_TOKENS = 4
SelectionScore = Literal["recovery-aware", "point"]
# Kept-channel tile of the down kernel and of the reference's tile_starts.
DOWN_TILE = 32
REFERENCE_DOWN_TILE = 128
ENCODER_TILE = 64
# Recovery rank whose encoder runs inside the exact launch (tile-major coefficients).
DIRECT_RANK = 32


def aligned_pairs(pairs: int, experts: int) -> int:
    """Pair capacity of the expert sort after padding to GROUP_ROWS blocks."""
    padded = pairs + experts * (GROUP_ROWS - 1)
    return min(pairs * GROUP_ROWS, padded) if pairs < experts else padded


def aligned_blocks(pairs: int, experts: int) -> int:
    """Number of GROUP_ROWS blocks the expert sort may fill."""
    return (aligned_pairs(pairs, experts) + GROUP_ROWS - 1) // GROUP_ROWS


@torch.no_grad()
def recovery_geometry(down: Tensor, norms: Tensor, encoder_t: Tensor, decoder: Tensor) -> Tensor:
    """Where the recovery map sends each channel, relative to its down column.

    Channel c of expert e has down column d = D_e[:, c] and recovery response
    r = U b, with b = encoder_t[e, c] (the rank-R encoder row) and U the
    decoder [H, R]. alpha = <d, r> / |d| is the response along d (0 when
    d = 0) and beta = sqrt(max(|r|^2 - alpha^2, 0)) its part across d, the
    quantities of the recovery-aware score (progressive.py:3347-3373). Both are
    formed from R-dimensional quantities, <d, U b> = b . (U^T d) and
    |U b|^2 = b^T (U^T U) b, in float64 one expert at a time, so no [I, H]
    response is materialised. Returns float32 [E, I, 2].
    """
    u = decoder.double()
    gram = u.T @ u  # [R, R]
    geometry = torch.empty(
        (down.shape[0], down.shape[2], 2), device=down.device, dtype=torch.float32
    )
    for expert in range(down.shape[0]):
        b = encoder_t[expert].double()  # [I, R]
        along = (b * (down[expert].double().T @ u)).sum(-1)  # <d_c, U b_c>
        norm = norms[expert].double()
        alpha = torch.where(norm > 0, along / torch.where(norm > 0, norm, 1.0), 0.0)
        energy = ((b @ gram) * b).sum(-1)  # |U b_c|^2
        geometry[expert, :, 0] = alpha.float()
        geometry[expert, :, 1] = (energy - alpha.square()).clamp_min(0).sqrt().float()
    return geometry


def _next_power_of_2(value: int) -> int:
    return 1 if value <= 1 else 1 << (value - 1).bit_length()


def _screen_splits(hidden: int) -> int:
    return min(8, hidden // 128)


def _dims(plan: BudgetPlan, experts: int, rank: int, flags: int = 0,
          grouped_tokens: int = GROUPED_TOKENS) -> _ext.Dims:
    return _ext.Dims(
        plan.hidden_size,
        plan.expert_width,
        plan.top_k,
        experts,
        rank,
        plan.final_count,
        plan.screen_coordinates,
        flags,
        grouped_tokens,
    )


def _pointer(tensor: Tensor | None) -> int | None:
    if tensor is None or tensor.numel() == 0:
        return None
    return tensor.data_ptr()


class ReaderWorkspace:
    """Device scratch of one reader call, shareable by layers run in sequence.

    Mirrors progressive.py:2868-3121. The `BudgetPlan` fixes the largest
    shapes; a screened layer with a smaller final_count may share it. `bytes` is
    the total allocation, reported once by the first reader bound to it. Every
    buffer a call reads is written earlier in the same call, so layers run
    back to back on one stream may share it; calls must not overlap.
    """

    @torch.no_grad()
    def __init__(
        self,
        plan: BudgetPlan,
        experts: int,
        rank: int,
        capacity: int,
        device: torch.device,
        grouped_tokens: int = GROUPED_TOKENS,
        grouped_screen_tokens: int = GROUPED_SCREEN_TOKENS,
        radix_select: bool = True,
        screen_block_splits: int = 8,
        grouped_screen_splits: int = 2,
    ) -> None:
        if capacity < 1 or grouped_tokens < 2:
            raise ValueError("Workspace needs a positive capacity and grouped size")
        if screen_block_splits not in (1, 2, 4, 8) or grouped_screen_splits not in (
            1, 2, 4, 8
        ):
            raise ValueError("Screen block splits must be 1, 2, 4 or 8")
        device = torch.device(device)
        self.key = (
            plan, experts, rank, capacity, device, grouped_tokens, grouped_screen_tokens
        )
        self.plan = plan
        self.capacity = capacity
        h, i, k, n = (
            plan.hidden_size, plan.expert_width, plan.top_k, plan.candidate_count
        )
        blocks = h // 128
        keep = plan.screen_coordinates
        sizes = _ext.workspace_sizes(_dims(plan, experts, rank), capacity)
        self._sizes = dict(zip((name for name, _ in _ext.WORKSPACE_FIELDS), sizes))
        dtype = {
            "int32": torch.int32, "float32": torch.float32, "bool": torch.bool,
            "bfloat16": torch.bfloat16, "int8": torch.int8,
        }

        def buffer(name: str, shape: tuple[int, ...]) -> Tensor:
            kind = dict(_ext.WORKSPACE_FIELDS)[name]
            tensor = torch.empty(shape, dtype=dtype[kind], device=device)
            if tensor.numel() * tensor.element_size() < self._sizes[name]:
                raise ValueError(f"workspace buffer {name} is smaller than the kernel needs")
            return tensor

        self.screen_splits = _screen_splits(h) if plan.completion_count < n else 1
        self.ids = buffer("ids", (capacity, k))
        self.weights = buffer("weights", (capacity, k))
        self.sketch_planes = buffer("planes", (capacity, blocks, keep))
        self.sketch_coordinates = (
            buffer("coordinates", (capacity, blocks, keep))
            if keep < 128
            else torch.empty(0, dtype=torch.int32, device=device)
        )
        self.sketch_values = buffer("qvals", (capacity, blocks, keep))
        self.sketch_exponents = buffer("qexp", (capacity, blocks))
        self.sketch_sums = buffer("qsums", (capacity, blocks))
        self.sketch_norms = buffer("norm2", (capacity, blocks))
        self.partial = buffer("partial", (capacity, 2, n))
        self.variances = buffer("variances", (capacity, 2, n))
        # the reference's split partials: this build keeps them in registers
        # and LDS inside the screen launch, so the buffers are empty
        self.screen_parts = torch.empty((0, 2, n), dtype=torch.float32, device=device)
        self.screen_variance_parts = torch.empty((0, 2, n), dtype=torch.float32, device=device)
        self.activations = buffer("activations", (capacity, n))
        self.completed = buffer("completed", (capacity, n))
        self.selected = buffer("selected", (capacity, n))
        self.selected.fill_(plan.final_count == n)
        self.candidate_ids = [
            torch.empty((0,), dtype=torch.int32, device=device),
            buffer("next_ids", (capacity, plan.final_count)),
        ]
        self.scores = [buffer("scores", (capacity, n))]
        self.starts = buffer("starts", (capacity, k))
        self.counts = buffer("counts", (capacity, k))
        self.tile_starts = buffer("tile_starts", (capacity, k))
        self.down_tile_starts = buffer("down_tile_starts", (capacity, k))
        self.down_splits = ceil(i / REFERENCE_DOWN_TILE)
        self.encoder_splits = ceil(i / ENCODER_TILE)
        self.down_tiles = ceil(plan.final_count / DOWN_TILE) + k - 1
        self.down_parts = buffer("down_parts", (capacity * self.down_tiles * h,))
        self.encoder_parts = buffer(
            "encoder_parts", (capacity, k, self.encoder_splits, rank)
        )
        self.latent = buffer("latent", (capacity, rank))
        # Expert-major grouping of the call's (token, slot) pairs.
        self.group_experts = buffer("group_experts", (capacity * k,))
        self.group_starts = buffer("group_starts", (capacity * k,))
        self.group_counts = buffer("group_counts", (capacity * k,))
        self.group_pairs = buffer("group_pairs", (capacity * k * GROUP_ROWS,))
        self.group_total = buffer("group_total", (1,))
        self.pair_tiles = buffer("pair_tiles", (capacity * k,))
        self.tile_masks = buffer("tile_masks", (capacity * n,))
        # Down workgroups' items grouped by expert per XCD, and their builders' records.
        self.down_order = buffer("down_order", (self._sizes["down_order"] // 4,))
        # the kept grid values' three 8-bit digits per rotated coordinate
        self.sketch_digits = buffer("digits", (capacity, blocks, 3, 128))
        # The reference's last-arrival counters; these kernels need none but the
        # attributes stay (all zero) for callers that inspect them.
        self.screen_counters = torch.zeros(
            (0, k, ceil(i / 80)), dtype=torch.int32, device=device
        )
        self.recovery_counters = torch.zeros((0,), dtype=torch.int32, device=device)
        self.histogram = torch.empty((0, 1 << RADIX_BITS), dtype=torch.int32, device=device)
        self.bucket_counts = torch.empty(
            (0, 1 << RADIX_HASH_BITS), dtype=torch.int32, device=device
        )
        self.bucket_keys = torch.empty(
            (0, 1 << RADIX_HASH_BITS, RADIX_CAPACITY), dtype=torch.int32, device=device
        )
        self.keys = torch.empty((0, k), dtype=torch.int32, device=device)
        # the reference's expert-sorted pair list and block experts are the
        # grouping's tile slots and tile experts here
        self.pairs = self.group_pairs
        self.block_experts = self.group_experts
        self.padded_pairs = torch.empty((1,), dtype=torch.int32, device=device)
        self.unions = torch.empty((0, 0, i), dtype=torch.int32, device=device)
        self.union_counts = torch.empty((0, 0, 2), dtype=torch.int32, device=device)
        self.sketch_split = torch.empty((0, blocks, 3, 128), dtype=torch.bfloat16, device=device)
        self.screen_coordinate_union = torch.empty((0, h), dtype=torch.bool, device=device)
        self.screen_dense = torch.empty((0, blocks), dtype=torch.bool, device=device)
        buffers = (
            self.ids, self.weights, self.sketch_planes, self.sketch_coordinates,
            self.sketch_values, self.sketch_exponents, self.sketch_sums, self.sketch_norms,
            self.partial,
            self.variances,
            self.activations, self.completed, self.selected, *self.candidate_ids,
            *self.scores, self.starts, self.counts, self.tile_starts,
            self.down_tile_starts, self.down_parts, self.encoder_parts, self.latent,
            self.group_experts, self.group_starts, self.group_counts, self.group_pairs,
            self.group_total, self.pair_tiles, self.tile_masks, self.down_order,
            self.sketch_digits,
        )
        self.bytes = sum(t.numel() * t.element_size() for t in buffers)
        self.charged = False
        # prepare_input's side stream (default priority) and its two events
        # (progressive.py:3113-3121), made on first use; `input_pending` is
        # set while a preparation awaits its consuming call
        self.input_stream: torch.cuda.Stream | None = None
        self.input_ready: torch.cuda.Event | None = None
        self.input_done: torch.cuda.Event | None = None
        self.input_pending = False

    def pointers(self, read_work: Tensor, final_count: int | None = None) -> _ext.WorkspacePointers:
        """C view of the buffers; `final_count` re-views the kept-id list."""
        fields = {name: _pointer(getattr(self, attr)) for name, attr in _WORKSPACE_ATTRS}
        fields["next_ids"] = _pointer(self.candidate_ids[1])
        fields["scores"] = _pointer(self.scores[0])
        return _ext.WorkspacePointers(
            self.capacity, *(fields[name] for name, _ in _ext.WORKSPACE_FIELDS),
            _pointer(read_work),
        )


_WORKSPACE_ATTRS = (
    ("ids", "ids"),
    ("weights", "weights"),
    ("planes", "sketch_planes"),
    ("coordinates", "sketch_coordinates"),
    ("qvals", "sketch_values"),
    ("qexp", "sketch_exponents"),
    ("qsums", "sketch_sums"),
    ("norm2", "sketch_norms"),
    ("partial", "partial"),
    ("variances", "variances"),
    ("selected", "selected"),
    ("completed", "completed"),
    ("activations", "activations"),
    ("starts", "starts"),
    ("counts", "counts"),
    ("tile_starts", "tile_starts"),
    ("down_tile_starts", "down_tile_starts"),
    ("down_parts", "down_parts"),
    ("encoder_parts", "encoder_parts"),
    ("latent", "latent"),
    ("group_experts", "group_experts"),
    ("group_starts", "group_starts"),
    ("group_counts", "group_counts"),
    ("group_pairs", "group_pairs"),
    ("group_total", "group_total"),
    ("pair_tiles", "pair_tiles"),
    ("tile_masks", "tile_masks"),
    ("down_order", "down_order"),
    ("digits", "sketch_digits"),
)


class ProgressiveReader:
    """Sparse decode operator of one MoE layer's routed experts.

    Construct one per layer, then call it once per decode step with the layer's
    hidden rows and router outputs. Native weights are borrowed in place; the
    workspace is reused across calls and is not reentrant (progressive.py:
    3124-3131).
    """

    @torch.no_grad()
    def __init__(
        self,
        gate_up: Tensor,
        down: Tensor,
        encoder: Tensor | None,
        decoder: Tensor | None,
        plan: BudgetPlan,
        max_tokens: int,
        expert_map: Tensor | None = None,
        sketch: tuple[Tensor, Tensor] | None = None,
        activation: GatedActivation = "silu",
        grouped_tokens: int = GROUPED_TOKENS,
        workspace: ReaderWorkspace | None = None,
        grouped_screen_tokens: int = GROUPED_SCREEN_TOKENS,
        selection_score: SelectionScore = "recovery-aware",
        fused_accounting: bool = True,
        radix_select: bool = True,
        screen_block_splits: int = 8,
        grouped_screen_splits: int = 2,
        selection_threshold: float | None = None,
        screen_last_block_reduction: bool = True,
        recovery_last_block_reduction: bool = True,
        pdl: bool = True,
    ) -> None:
        """Prepare the sketch, recovery geometry and workspace of one layer.

        Arguments as progressive.py:3158-3213. gate_up is [E, 2 I, H] BF16
        contiguous; down the channel-major logical [E, H, I] (stride
        (H I, 1, H)); encoder [E, R, I] and decoder [H, R] or both None. The
        scheduling options (grouped sizes, fused accounting, radix selection,
        split counts, last-block reductions, pdl) are accepted for API parity;
        they do not change any result here, since the HIP kernels fix one
        arithmetic for every batch size.
        """
        h, i, k = plan.hidden_size, plan.expert_width, plan.top_k
        e = gate_up.shape[0]
        rank = decoder.shape[1] if decoder is not None else 0
        if selection_threshold is not None and (
            not selection_threshold >= 0
            or selection_threshold == float("inf")
            or not plan.final_count == plan.completion_count < plan.candidate_count
        ):
            raise ValueError(
                "A selection threshold is finite, nonnegative and needs a screened plan"
            )
        thresholded = selection_threshold is not None
        self.selection_threshold = (
            torch.tensor([selection_threshold], device=gate_up.device, dtype=torch.float32)
            if thresholded
            else None
        )
        if screen_block_splits not in (1, 2, 4, 8) or grouped_screen_splits not in (
            1, 2, 4, 8
        ):
            raise ValueError("Screen block splits must be 1, 2, 4 or 8")
        self.batch_screen_splits = min(screen_block_splits, h // 128)
        self.grouped_screen_splits = min(grouped_screen_splits, h // 128)
        self.radix_select = (
            radix_select
            and not thresholded
            and expert_map is None
            and plan.candidate_count >= 1024
            and plan.final_count == plan.completion_count < plan.candidate_count
        )
        self.fused_accounting = (
            fused_accounting
            and not thresholded
            and expert_map is None
            and plan.completion_count == plan.final_count
        )
        if (
            gate_up.shape != (e, 2 * i, h)
            or down.shape != (e, h, i)
            or (encoder is None) != (decoder is None)
            or (encoder is not None and encoder.shape != (e, rank, i))
            or (decoder is not None and (decoder.shape != (h, rank) or rank < 1))
            or not gate_up.is_cuda
            or down.device != gate_up.device
            or gate_up.dtype != torch.bfloat16
            or down.dtype != gate_up.dtype
            or not gate_up.is_contiguous()
            or down.stride() != (h * i, 1, h)
            or (expert_map is None and k > e)
            or max_tokens < 1
            or grouped_tokens < 2
        ):
            raise ValueError(
                "Expected native GU and channel-major D CUDA experts, "
                "matching recovery and capacity"
            )
        if expert_map is not None:
            raise NotImplementedError(
                "Expert parallelism spans several GPUs; this reader runs on one GPU"
            )
        if rank > 64:
            raise ValueError("Recovery rank above 64 is not supported")
        if k > 64 or plan.candidate_count > 16384 or max_tokens * k > 8192:
            raise ValueError(
                "At most 64 routed experts, 16384 candidates per token and 8192 "
                "routed pairs per call"
            )
        self.pdl = False
        self.screen_last_block_reduction = screen_last_block_reduction
        self.recovery_last_block_reduction = recovery_last_block_reduction and rank > 0
        self.selection_score: SelectionScore = selection_score
        self.expert_map = None
        self.ep_group = None
        self.recovery_owner = True
        self.plan, self.max_tokens, self.rank = plan, max_tokens, rank
        self.activation: GatedActivation = activation
        device = gate_up.device
        self.sketch_signs = block_hadamard_signs(h, device)
        if sketch is None:
            sketch = build_sketch(gate_up, self.sketch_signs)
        codes, self.sketch_statistics = sketch
        if (
            codes.shape != (e, sketch_storage_bytes(2 * i, h))
            or codes.dtype != torch.uint8
            or codes.device != device
            or not codes.is_contiguous()
            or self.sketch_statistics.shape != (e, 2 * i, h // 128, 2)
            or self.sketch_statistics.dtype != torch.float16
            or self.sketch_statistics.device != device
            or self.sketch_statistics.stride() != (4 * i * (h // 128), 1, 4 * i, 2 * i)
        ):
            raise ValueError("Sketch must match the local native routed experts")
        # The screen reads the codes through a 2-bit repacking in the order of
        # its matrix-core operands, built once here (64 I H / 128 bytes per
        # expert); the reference streams the codes themselves. Only the planes
        # stay resident: `sketch_codes` rebuilds the codes from them when read.
        # A dense plan never screens: it keeps the codes as given.
        self.sketch_trit_planes = torch.empty(0, dtype=torch.int32, device=device)
        self._sketch_codes: Tensor | None = codes
        if plan.final_count < plan.candidate_count:
            dims = _dims(plan, e, rank)
            self.sketch_trit_planes = torch.empty(
                _ext.trit_plane_bytes(dims) // 4, dtype=torch.int32, device=device
            )
            _ext.check(
                _ext.library().cfmoe_pack_trit_planes(
                    ctypes.byref(dims),
                    codes.data_ptr(),
                    self.sketch_trit_planes.data_ptr(),
                    torch.cuda.current_stream(device).cuda_stream,
                )
            )
            self._sketch_codes = None
        del codes
        # what stays resident: the trit planes (screened plans) or the codes,
        # plus the FP16 statistics
        resident = (
            self.sketch_trit_planes.numel() * 4
            if self._sketch_codes is None
            else self._sketch_codes.numel()
        )
        self.sketch_resident_bytes = resident + self.sketch_statistics.numel() * 2
        self._rebuilt_codes: weakref.ref | None = None
        self.norms = down.float().square().sum(1).sqrt()
        self.native_gu = gate_up.detach()
        self.down = down.detach()
        self.encoder: Tensor | None = None
        self._encoder_tiles: Tensor | None = None
        self.decoder: Tensor | None = None
        self.recovery_geometry: Tensor | None = None
        prepared = False
        if encoder is not None and decoder is not None:
            self.encoder = (
                encoder.to(device=device, dtype=torch.bfloat16).transpose(1, 2).contiguous()
            )
            self.decoder = decoder.to(device=device, dtype=torch.bfloat16).contiguous()
            if self.encoder.shape[2] == DIRECT_RANK:
                # the exact launch's encoder reads each rank's 64 coefficients of
                # a 64-channel tile as one contiguous row: [E, tiles, R, 64]
                tiles = ceil(i / ENCODER_TILE)
                padded = torch.zeros(
                    (e, tiles * ENCODER_TILE, DIRECT_RANK), dtype=torch.bfloat16, device=device
                )
                padded[:, :i] = self.encoder
                self._encoder_tiles = (
                    padded.view(e, tiles, ENCODER_TILE, DIRECT_RANK).transpose(2, 3).contiguous()
                )
            if selection_score != "point":
                prepared = True
                self.recovery_geometry = self._geometry(down)
        n = plan.candidate_count
        if workspace is None:
            workspace = ReaderWorkspace(
                plan, e, rank, max_tokens, device, grouped_tokens, grouped_screen_tokens,
                radix_select=self.radix_select,
                screen_block_splits=screen_block_splits,
                grouped_screen_splits=grouped_screen_splits,
            )
        workspace_plan = workspace.key[0]
        compatible_plan = workspace_plan == plan or (
            workspace_plan.hidden_size == h
            and workspace_plan.expert_width == i
            and workspace_plan.top_k == k
            and workspace_plan.screen_coordinates == plan.screen_coordinates
            and plan.final_count == plan.completion_count
            and workspace_plan.final_count == workspace_plan.completion_count
            and plan.final_count <= workspace_plan.final_count < n
        )
        if not compatible_plan or workspace.key[1:] != (
            e, rank, max_tokens, torch.device(device), grouped_tokens, grouped_screen_tokens
        ):
            raise ValueError("Shared workspace must match the plan, experts and capacity")
        self.workspace = workspace
        self.grouped_tokens = grouped_tokens
        self.grouped_screen_tokens = grouped_screen_tokens
        w = workspace
        self.ids, self.weights, self.partial, self.variances = (
            w.ids, w.weights, w.partial, w.variances
        )
        self.sketch_planes = w.sketch_planes
        self.sketch_coordinates = w.sketch_coordinates
        self.sketch_values = w.sketch_values
        self.sketch_exponents = w.sketch_exponents
        self.sketch_norms = w.sketch_norms
        self.screen_splits = w.screen_splits
        self.screen_parts = w.screen_parts
        self.screen_variance_parts = w.screen_variance_parts
        self.screen_counters = w.screen_counters
        self.activations, self.completed, self.selected = (
            w.activations, w.completed, w.selected
        )
        self.scores = w.scores
        self.candidate_ids = w.candidate_ids
        if workspace_plan != plan:
            # Kernels index packed token * F lists, not tensor strides.
            self.candidate_ids = [
                w.candidate_ids[0],
                w.candidate_ids[1]
                .view(-1)[: max_tokens * plan.final_count]
                .view(max_tokens, plan.final_count),
            ]
        self.starts, self.counts, self.tile_starts = w.starts, w.counts, w.tile_starts
        self.down_tile_starts = w.down_tile_starts
        self.down_splits, self.encoder_splits = w.down_splits, w.encoder_splits
        self.down_parts, self.encoder_parts, self.latent = (
            w.down_parts, w.encoder_parts, w.latent
        )
        self.recovery_counters = w.recovery_counters
        self.workspace_bytes = 0 if w.charged else w.bytes
        w.charged = True
        self.recovery_geometry_bytes = (
            self.recovery_geometry.numel() * 4 if self.recovery_geometry is not None else 0
        )
        self.recovery_geometry_preparation_products = prepared * 2 * e * i * h
        self.recovery_geometry_preparation_reduction_adds = prepared * 2 * e * i * (h - 1)
        self.recovery_response_preparation_macs = prepared * e * i * h * rank
        self.matrix_macs = (
            2 * n * h * (plan.completion_count != n)
            + 2 * plan.completion_count * h
            + h * plan.final_count
            + rank * (n - plan.final_count + h)
        )
        # Read statistics (progressive.py:3507-3515). Logical bytes: 0 native,
        # 1 dense reference, 3 recovery, 4 selection metadata, 5 sketch.
        # Sector-priced: 6 native, 7 recovery, 9 selection, 17 sketch; slot 10
        # rotation signs. Requested: 11 sketch, 12 gate/up, 13 down, 14
        # encoder. 15 grouped tile MACs, 16 grouped rows, 19 thresholded tokens.
        self.read_work = torch.zeros(20, device=device, dtype=torch.float64)
        self._weights_c = _ext.WeightPointers(
            _pointer(self.native_gu),
            _pointer(self.down),
            _pointer(self._sketch_codes),
            _pointer(self.sketch_statistics),
            _pointer(self.norms),
            _pointer(self.recovery_geometry),
            _pointer(self.encoder),
            _pointer(self.decoder),
            _pointer(self.sketch_signs),
            _pointer(self.selection_threshold),
            _pointer(self.sketch_trit_planes),
            _pointer(self._encoder_tiles),
        )
        self._workspace_c = workspace.pointers(self.read_work)
        self._workspace_c.next_ids = _pointer(self.candidate_ids[1])
        # per-token read charges of per-token and of grouped calls; thresholded
        # readers add theirs from the selection (the device still adds its
        # per-tile and union terms)
        charges = (ctypes.c_double * 18)
        self._charges = {
            grouped: charges(*(
                self._fixed_charges(grouped, grouped) if selection_threshold is None
                else (0.0,) * 18))
            for grouped in (False, True)
        }
        _ext.library()

    def _geometry(self, down: Tensor) -> Tensor:
        """alpha, beta of each channel's recovery response (progressive.py:3347-3373)."""
        return recovery_geometry(down, self.norms, self.encoder, self.decoder)

    def _fixed_charges(self, grouped: bool, grouped_screen: bool) -> tuple[float, ...]:
        """Per-token read statistics independent of the selection (slots 0-17).

        Slots 0-10 and 17 follow progressive.py:4492-4524. The requested-byte
        slots 11-16 describe this build's kernels: the screen streams each
        tile's trit planes (slot 11, with its matrix-core MACs in slot 15,
        both added per tile on the device); the exact rows request 4 H bytes
        per kept channel and token, or per channel of a tile's union in grouped
        calls (slot 12, then counted on the device); the down rows request
        2 H bytes per kept channel and token at every batch size (slot 13); the
        recovery encoder requests the 2 R byte rows of all I channels of each
        routed slot (slot 14); slot 16 counts the tokens of grouped calls.
        `grouped_screen` is accepted for the reference's signature.
        """
        p = self.plan
        native = p.selected_weight_bytes()
        recovery = p.recovery_read_bytes(self.rank)
        selection = p.selection_read_bytes(self.recovery_geometry is not None)
        residual = self.selection_score != "point"
        sketch = p.sketch_read_bytes(residual)
        h, unit = p.hidden_size, 2
        encoder = 2 * self.rank * p.candidate_count
        screened = p.completion_count < p.candidate_count
        return tuple(
            float(v)
            for v in (
                native,
                p.native_read_bytes(),
                0,
                recovery,
                selection,
                p.sketch_read_bytes(residual, sectors=False),
                native,
                recovery,
                0,
                selection,
                h if screened else 0,
                0,
                0 if grouped else unit * 2 * h * p.completion_count,
                unit * h * p.final_count,
                encoder,
                0,
                int(grouped),
                sketch,
            )
        )

    def _flags(self, ids: Tensor, weights: Tensor, input_prepared: bool) -> int:
        flags = 0
        if self.selection_score == "point":
            flags |= _ext.POINT
        if self.activation == "gelu_tanh":
            flags |= _ext.GELU
        if self.recovery_geometry is not None:
            flags |= _ext.GEOMETRY
        if self.selection_threshold is not None:
            flags |= _ext.THRESHOLD
        flags |= _ext.ACCOUNT
        if ids.dtype == torch.int64:
            flags |= _ext.IDS_INT64
        if weights.dtype == torch.bfloat16:
            flags |= _ext.WEIGHTS_BF16
        if input_prepared:
            flags |= _ext.INPUT_PREPARED
        return flags

    def _call_dims(self, ids: Tensor, weights: Tensor, input_prepared: bool) -> _ext.Dims:
        """C dimensions and flags of one call with these router outputs."""
        p = self.plan
        screened = p.completion_count < p.candidate_count
        return _dims(
            p,
            self.native_gu.shape[0],
            self.rank,
            self._flags(ids, weights, input_prepared and screened),
            self.grouped_tokens,
        )

    def _validate_input(self, hidden: Tensor, padding: Tensor | None) -> int:
        """Check the hidden rows and padding mask; return the token count."""
        tokens = hidden.shape[0]
        if (
            not 1 <= tokens <= self.max_tokens
            or hidden.shape != (tokens, self.plan.hidden_size)
            or hidden.dtype != torch.bfloat16
            or hidden.device != self.native_gu.device
            or not hidden.is_contiguous()
            or (
                padding is not None
                and (
                    padding.shape != (tokens,)
                    or padding.device != hidden.device
                    or padding.dtype != torch.bool
                    or not padding.is_contiguous()
                )
            )
        ):
            raise ValueError("Sparse input exceeds the prepared token/candidate contract")
        return tokens

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.native_gu.device).cuda_stream

    @property
    def sketch_codes(self) -> Tensor:
        """The sketch codes [E, sketch_storage_bytes(2 I, H)] (progressive.py:3317).

        Screened plans keep only the trit planes resident, so this rebuilds
        the codes from them (one launch); bytes that carry no channel read 121,
        as `build_sketch` leaves them. The rebuilt tensor is held by a weak
        reference: reads while a caller still holds it (or a view of it)
        return that same tensor, and it is freed with the caller's last
        reference. It is a copy: editing it does not change what the screen
        reads.
        """
        if self._sketch_codes is not None:
            return self._sketch_codes
        held = self._rebuilt_codes() if self._rebuilt_codes is not None else None
        if held is not None:
            return held
        p = self.plan
        e = self.native_gu.shape[0]
        codes = torch.empty(
            (e, sketch_storage_bytes(2 * p.expert_width, p.hidden_size)),
            dtype=torch.uint8, device=self.native_gu.device,
        )
        dims = _dims(p, e, self.rank)
        _ext.check(
            _ext.library().cfmoe_unpack_trit_planes(
                ctypes.byref(dims), self.sketch_trit_planes.data_ptr(), codes.data_ptr(),
                self._stream(),
            )
        )
        self._rebuilt_codes = weakref.ref(codes)
        return codes

    @torch.no_grad()
    def prepare_input(self, hidden: Tensor, padding: Tensor | None = None) -> bool:
        """Rotate the input ahead of the router (progressive.py:3829-3873).

        The rotation runs on the workspace's side stream once the current
        stream has reached this point, so it overlaps whatever the caller
        enqueues next (the router). Returns False, launching nothing, for
        unscreened plans. Pass input_prepared=True to the next call with the
        same rows. The next call on the workspace, prepared or not, makes the
        current stream wait for the rotation before its first kernel; the
        workspace stays non-reentrant in between.
        """
        p = self.plan
        if p.completion_count == p.candidate_count:
            return False
        tokens = self._validate_input(hidden, padding)
        dims = _dims(p, self.native_gu.shape[0], self.rank, 0, self.grouped_tokens)
        w = self.workspace
        device = self.native_gu.device
        if w.input_stream is None:
            w.input_stream = torch.cuda.Stream(device=device)
            w.input_ready, w.input_done = torch.cuda.Event(), torch.cuda.Event()
        w.input_ready.record(torch.cuda.current_stream(device))
        w.input_stream.wait_event(w.input_ready)
        _ext.check(
            _ext.library().cfmoe_prepare_input(
                ctypes.byref(dims),
                ctypes.byref(self._weights_c),
                ctypes.byref(self._workspace_c),
                hidden.data_ptr(),
                _pointer(padding),
                tokens,
                w.input_stream.cuda_stream,
            )
        )
        w.input_done.record(w.input_stream)
        w.input_pending = True
        return True

    def _join_input(self) -> None:
        """The current stream waits for a pending prepare_input rotation (any
        call does: the rotation writes rows of the shared workspace)."""
        w = self.workspace
        if w.input_pending:
            torch.cuda.current_stream(self.native_gu.device).wait_event(w.input_done)
            w.input_pending = False

    @torch.no_grad()
    def __call__(
        self,
        hidden: Tensor,
        ids: Tensor,
        weights: Tensor,
        padding: Tensor | None = None,
        out: Tensor | None = None,
        *,
        input_prepared: bool = False,
    ) -> Tensor:
        """Routed-expert output [tokens, H] of a batch (progressive.py:3876-4472).

        hidden BF16 [tokens, H]; ids (int32/int64) and weights (fp32/bf16)
        [tokens, K]; padding bool [tokens] marks rows that read no weights and
        add no read statistics. Writes `out` (allocated if None) and adds the
        call's read statistics to `read_work`.
        """
        tokens = self._validate_input(hidden, padding)
        p = self.plan
        k = p.top_k
        if (
            ids.shape != (tokens, k)
            or weights.shape != ids.shape
            or ids.device != hidden.device
            or weights.device != hidden.device
            or ids.dtype not in (torch.int32, torch.int64)
            or weights.dtype not in (torch.float32, torch.bfloat16)
            or not ids.is_contiguous()
            or not weights.is_contiguous()
            or (
                out is not None
                and (
                    out.shape != hidden.shape
                    or out.dtype != hidden.dtype
                    or out.device != hidden.device
                    or not out.is_contiguous()
                )
            )
        ):
            raise ValueError("Sparse input exceeds the prepared token/candidate contract")
        if out is None:
            out = torch.empty_like(hidden)
        dims = self._call_dims(ids, weights, input_prepared)
        # any call joins a pending rotation first: it reads or rewrites the
        # same workspace rows
        self._join_input()
        _ext.check(
            _ext.library().cfmoe_forward(
                ctypes.byref(dims),
                ctypes.byref(self._weights_c),
                ctypes.byref(self._workspace_c),
                hidden.data_ptr(),
                ids.data_ptr(),
                weights.data_ptr(),
                _pointer(padding),
                out.data_ptr(),
                tokens,
                self._charges[tokens >= self.grouped_tokens],
                self._stream(),
            )
        )
        if self.selection_threshold is not None:
            self._charge_thresholded(tokens, padding)
        return out

    def launch_stage(
        self,
        stage: str,
        hidden: Tensor,
        ids: Tensor,
        weights: Tensor,
        padding: Tensor | None,
        out: Tensor,
    ) -> None:
        """Relaunch one kernel of the last call (`_ext.STAGES`) for timing.

        Reads the workspace state the earlier stages of a call left, so it is
        meaningful only after a full call with the same arguments. Accounting is
        not repeated.
        """
        tokens = hidden.shape[0]
        flags = self._flags(ids, weights, False) & ~_ext.ACCOUNT
        dims = _dims(self.plan, self.native_gu.shape[0], self.rank, flags, self.grouped_tokens)
        self._join_input()
        _ext.check(
            _ext.library().cfmoe_launch_stage(
                _ext.STAGES.index(stage),
                ctypes.byref(dims),
                ctypes.byref(self._weights_c),
                ctypes.byref(self._workspace_c),
                hidden.data_ptr(),
                ids.data_ptr(),
                weights.data_ptr(),
                _pointer(padding),
                out.data_ptr(),
                tokens,
                None,
                self._stream(),
            )
        )

    def _charge_thresholded(self, tokens: int, padding: Tensor | None) -> None:
        """Selection-dependent read statistics of a thresholded call.

        Enqueued torch ops on the current stream (no host sync): the kept count
        varies per token, so charges follow progressive.py:2189-2225 with the
        per-token selected counts. The device adds the per-tile screen terms
        (slots 11, 15) and, in grouped calls, the union rows (slot 12).
        """
        p = self.plan
        h, i, k, n, rank = (
            p.hidden_size, p.expert_width, p.top_k, p.candidate_count, self.rank
        )
        active = (
            torch.ones(tokens, dtype=torch.float64, device=self.read_work.device)
            if padding is None
            else (~padding).to(torch.float64)
        )
        selected = self.selected[:tokens].sum(1).to(torch.float64) * active
        completed = self.completed[:tokens].sum(1).to(torch.float64) * active
        count = active.sum()
        kept = selected.sum()
        done = completed.sum()
        geometry = self.recovery_geometry is not None
        residual = self.selection_score != "point"
        candidates = count * n
        native = 2 * (2 * done * h + kept * h)
        recovery = 2 * rank * (candidates - kept + count * h)
        selection = (12 if geometry else 4) * candidates + 4 * count
        physical_selection = (12 if geometry else 4) * candidates + 32 * count
        sketch = count * p.sketch_read_bytes(residual, sectors=False)
        physical_sketch = count * p.sketch_read_bytes(residual)
        work = self.read_work
        work[0] += native
        work[1] += count * p.native_read_bytes()
        work[3] += recovery
        work[4] += selection
        work[5] += sketch
        work[6] += native
        work[7] += recovery
        work[9] += physical_selection
        work[10] += count * h
        if tokens >= self.grouped_tokens:
            work[16] += count
        else:
            work[12] += 2 * 2 * h * done
        work[13] += 2 * h * kept
        work[14] += 2 * rank * candidates
        work[17] += physical_sketch
        work[19] += count

    def report(self) -> dict[str, float | None]:
        """Accumulated read statistics and work counters (progressive.py:3517-3803).

        Reads `read_work` back to the host (a device sync). "charged_bytes" is
        the sector-priced read cost, "read_fraction" its ratio to the dense
        reference; "logical_*" price exact bytes; "issued_*" are requested
        bytes.
        """
        (
            native, reference, _, recovery, selection, sketch, physical_native,
            physical_recovery, _, physical_selection, rotation_signs, issued_sketch,
            issued_gate_up, issued_down, issued_encoder, grouped_macs, grouped_rows,
            physical_sketch, _, threshold_tokens,
        ) = self.read_work.cpu().tolist()
        p = self.plan
        h, n, k, i = p.hidden_size, p.candidate_count, p.top_k, p.expert_width
        logical = native + recovery + selection + sketch + rotation_signs
        charged = (
            physical_native + physical_recovery + physical_selection + physical_sketch
            + rotation_signs
        )
        screened = float(p.completion_count != n)
        input_sparse = screened * (p.screen_coordinates < 128)
        point = self.selection_score == "point"
        splits = _screen_splits(h)
        planes = 1 + (not point)
        # both screens reduce their block splits on chip (registers, or LDS
        # inside one workgroup): no split partial crosses HBM
        split_io = 0.0
        split_adds = float(2 * (splits - 1) * n * planes) * screened
        return {
            "charged_bytes": charged,
            "reference_bytes": reference,
            "native_expert_coefficient_bytes": native,
            "physical_native_expert_coefficient_bytes": physical_native,
            "recovery_bytes": recovery,
            "physical_recovery_bytes": physical_recovery,
            "selection_parameter_bytes": selection,
            "physical_selection_parameter_bytes": physical_selection,
            "sketch_bytes": sketch,
            "physical_sketch_bytes": physical_sketch,
            "sketch_resident_bytes": float(self.sketch_resident_bytes),
            "selection_threshold_resident_bytes": 4.0 * (self.selection_threshold is not None),
            "rotation_sign_bytes": rotation_signs,
            "rotation_sign_resident_bytes": float(h),
            # The routing launch sorts each token's K ids once (not per screen CTA).
            "early_screen_route_metadata_io_bytes_per_token_upper_bound": float(12 * k) * screened,
            "early_screen_route_compare_exchanges_per_token_upper_bound": float(k * (k - 1) // 2)
            * screened,
            "early_screen_route_reduction_adds_per_token_upper_bound": float(k * (k - 1))
            * screened,
            "rotation_input_io_bytes_per_token": float(
                2 * h + ((12 if input_sparse else 8) * p.screen_coordinates + 8) * (h // 128)
            )
            * screened,
            "rotation_arithmetic_per_token": float(11 * h) * screened,
            # one rotation launch serves every batch size
            "grouped_rotation_input_io_bytes_per_token": float(
                2 * h + ((12 if input_sparse else 8) * p.screen_coordinates + 8) * (h // 128)
            )
            * screened,
            "grouped_rotation_arithmetic_per_token": float(11 * h) * screened,
            # The mask's cutoff is a 31-step binary search over magnitude bits
            # (two ballots per step) rather than a sort.
            "screen_ranking_compare_exchanges_per_token": float(h // 128 * 31 * 128)
            * input_sparse,
            "screen_mask_arithmetic_per_token": float(h // 128 * 9 * 128) * input_sparse,
            "screen_compaction_scan_adds_per_token": float(h // 128 * 127) * input_sparse,
            # The expert-major screen runs at every batch size and sums each
            # row's block splits in order on chip; there are no arrival
            # counters. Its workgroups read each pair's three 128-byte digit
            # planes per block once per workgroup of the pair's tile: I / 16
            # workgroups per tile below the grouped size, I / 64 from it.
            "batch_one_screen_split_io_bytes": split_io,
            "batched_screen_split_io_bytes_per_token": split_io,
            "batched_screen_split_adds_per_token": split_adds,
            "batch_one_screen_counter_io_bytes": 0.0,
            "batched_screen_counter_io_bytes_per_token": 0.0,
            "batch_one_screen_counter_sector_bytes_upper_bound": 0.0,
            "batched_screen_counter_sector_bytes_per_token_upper_bound": 0.0,
            "grouped_screen_split_io_bytes_per_token": split_io,
            "grouped_screen_split_adds_per_token": split_adds,
            "grouped_screen_union_io_bytes_per_token_upper_bound": float(
                384 * k * (h // 128) * -(-i // 64)
            )
            * screened,
            "per_token_screen_dot_terms": float(
                k * 2 * i * (h // 128) * p.screen_coordinates
            )
            * screened,
            "read_fraction": charged / reference if reference else None,
            "logical_charged_bytes": logical,
            "logical_read_fraction": logical / reference if reference else None,
            "issued_sketch_bytes": issued_sketch,
            "issued_gate_up_bytes": issued_gate_up,
            "issued_down_bytes": issued_down,
            "issued_recovery_encoder_bytes": issued_encoder,
            "grouped_rows": grouped_rows,
            "grouped_issued_matrix_macs": grouped_macs,
            "workspace_bytes": float(self.workspace_bytes),
            # Below the grouped size an exact workgroup is one wave per kept
            # channel with no LDS; at rank 32 the encoder workgroups of the
            # same launch stage two items' 64 channel values (512 B).
            "batch_one_completion_shared_bytes_per_cta_upper_bound": float(
                512 * (self.rank == DIRECT_RANK)
            ),
            # No arrival counters (kernel boundaries order the stages), and the
            # selection's radix histograms live in LDS: these global-scratch
            # request counts are zero here.
            "small_batch_recovery_counter_io_bytes_per_token": 0.0,
            "small_batch_recovery_counter_sector_bytes_per_token_upper_bound": 0.0,
            "small_batch_radix_scratch_io_bytes_per_token_upper_bound": 0.0,
            "small_batch_radix_atomic_adds_per_token": 0.0,
            "small_batch_radix_scratch_sector_bytes_per_token_upper_bound": 0.0,
            "small_batch_radix_scan_adds_per_token_upper_bound": 0.0,
            # One selection workgroup per token reads its N scores once.
            "small_batch_final_selection_score_io_bytes_per_token": float(4 * n) * screened,
            "matrix_macs_per_token": float(self.matrix_macs)
            if self.selection_threshold is None
            else self._threshold_matrix_macs(native, reference, threshold_tokens),
        }

    def _threshold_matrix_macs(self, native: float, reference: float, tokens: float) -> float:
        """Realized MACs per active token of a thresholded reader (progressive.py:4474-4490)."""
        if not tokens:
            return 0.0
        p = self.plan
        h, i = p.hidden_size, p.expert_width
        slots = reference / (p.native_read_bytes() // p.top_k)
        kept = native / (2 * 3 * h)
        local = 2 * h * i * slots + 3 * h * kept + self.rank * (i * slots - kept)
        return local / tokens + self.rank * h


__all__ = [
    "GROUPED_SCREEN_TOKENS",
    "GROUPED_TOKENS",
    "GROUP_ROWS",
    "ProgressiveReader",
    "ReaderWorkspace",
    "SelectionScore",
    "aligned_blocks",
    "aligned_pairs",
    "channel_major_down",
    "sketch_code_stride",
]
