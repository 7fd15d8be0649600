"""Resident ternary sketch of the native gate/up rows, read by the screen.

Mirrors `calibration_free_moe/reader/sketch.py` of the reference: the rotation
signs (sketch.py:22-35), the block-Hadamard rotation (:38-50), the kept-
coordinate mask (:53-68), the packed sketch format (:84-150), its decoder
(:209-232), the differentiable sketch feature (:153-206) and the recovery-map
acquisition check (:71-81). The packed format is an interface shared with
prebuilt sketches and offline recovery fitting, so its byte layout follows the
reference exactly. The torch construction here (on the weights' device,
vectorised over experts in chunks) is the default and gives the reference's
codes; `build_sketch(..., device_kernel=True)` sketches BF16 GPU weights in one
HIP launch instead (cfmoe_build_sketch in the reader's library).

Layout of one expert's codes (rows = 2 I, blocks = H / 128, stride =
`sketch_code_stride(rows)`, body = stride rounded down to 32, tail = stride %
32): byte g of coordinate c in block b packs five consecutive channels
5 (g // 2) .. 5 (g // 2) + 4 of the gate (g even) or up (g odd) rows as
121 + sum_d t_d 3**d, t_d in {-1, 0, 1}. Bytes [0, body) of each coordinate
sit at (b * 128 + c) * body; bytes [body, stride) at
blocks * 128 * body + ((b // 2) * 128 + c) * 32 + (b % 2) * 16. The FP16
statistics are [E, 2 I, blocks, 2] (scale, residual variance) over a physical
[E, blocks, 2, 2 I] allocation.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from calibration_free_moe.activation import GatedActivation, activate
from calibration_free_moe.reader.budget import sketch_code_stride, sketch_storage_bytes

# Acquisition rule a nonzero recovery map must declare (sketch.py:17-19).
ACQUISITION = "ternary-hadamard-sketch-v1"

# 121 = 1 + 3 + 9 + 27 + 81 encodes five zero trits.
ZERO_CODE = 121
_POWERS = (1, 3, 9, 27, 81)
# FP32 value of 1 / sqrt(128), applied after the seven butterfly stages.
ROTATION_SCALE = 1.0 / math.sqrt(128.0)


def block_hadamard_signs(hidden: int, device: torch.device | str) -> Tensor:
    """Model-wide +-1 int8 rotation signs, drawn from a seed-0 CPU generator.

    The same seed-0 draw as sketch.py:22-35, so prebuilt sketches and offline
    recovery fitting share the rotation.
    """
    if hidden % 128:
        raise ValueError("Hadamard sketch requires hidden width divisible by 128")
    bits = torch.randint(0, 2, (hidden,), generator=torch.Generator().manual_seed(0))
    return (2 * bits - 1).to(device=device, dtype=torch.int8)


def _butterflies(value: Tensor) -> Tensor:
    """Seven in-place-order butterfly stages over the last dim (128).

    Stage w pairs coordinates c and c + w (c with bit w clear) into
    (left + right, left - right), as the kernel's lane exchange does.
    """
    lead = value.shape[:-1]
    for width in (1, 2, 4, 8, 16, 32, 64):
        pairs = value.reshape(*lead, 128 // (2 * width), 2, width)
        left = pairs[..., 0, :]
        right = pairs[..., 1, :]
        value = torch.stack((left + right, left - right), dim=-2).reshape(*lead, 128)
    return value


def rotate_blocks(x: Tensor, signs: Tensor | None) -> Tensor:
    """blockdiag(H128)/sqrt(128) diag(signs) x in FP32; identity for None."""
    if signs is None:
        return x.float()
    blocks = signs.numel() // 128
    value = x.float().reshape(-1, blocks, 128) * signs.float().reshape(blocks, 128)
    return (_butterflies(value) * ROTATION_SCALE).reshape(x.shape)


def mask_rotated_blocks(x: Tensor, keep: int = 128) -> Tensor:
    """Zero all but each block's `keep` largest |x|; ties go to lower coordinates.

    Membership carries no gradient; kept values pass gradients through.
    """
    if keep == 128:
        return x
    blocks = x.reshape(*x.shape[:-1], -1, 128)
    with torch.no_grad():
        magnitude = blocks.abs()
        cutoff = torch.topk(magnitude, keep, dim=-1).values[..., -1:]
        above = magnitude > cutoff
        tied = magnitude == cutoff
        room = keep - above.sum(dim=-1, keepdim=True)
        kept = above | (tied & (tied.cumsum(dim=-1) <= room))
    return torch.where(kept, blocks, torch.zeros_like(blocks)).reshape_as(x)


def require_sketch_acquisition(bank: dict[str, object]) -> None:
    """Reject a nonzero recovery map fitted to another acquisition rule."""
    decoder, encoder = bank["decoder"], bank["encoder"]
    if not isinstance(decoder, Tensor) or not isinstance(encoder, Tensor):
        raise TypeError("Recovery bank parameters must be tensors")
    if bool(torch.count_nonzero(decoder)) or bool(torch.count_nonzero(encoder)):
        plan = bank.get("plan")
        if not isinstance(plan, dict) or plan.get("acquisition") != ACQUISITION:
            raise ValueError(f"Nonzero recovery bank requires {ACQUISITION} acquisition")


def _ternarise(value: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """TWN rule per 128-block: keep |v| > 0.7 mean|v|; scale = mean kept |v|.

    Returns the trits (int16 in {-1,0,1}), the FP32 scale and the FP32 mean
    squared residual of `value` [..., 128].
    """
    magnitude = value.abs()
    keep = magnitude > 0.7 * magnitude.mean(dim=-1, keepdim=True)
    scale = (magnitude * keep).sum(-1) / keep.sum(-1).clamp_min(1)
    trit = torch.where(keep, value.sign(), torch.zeros_like(value))
    residual = (value - trit * scale.unsqueeze(-1)).square().mean(-1)
    return trit.to(torch.int16), scale, residual


def _pack_bytes(trit: Tensor, width: int, stride: int) -> Tensor:
    """Pack trits [chunk, 2, width, blocks, 128] into [chunk, blocks, 128, stride]."""
    chunk, _, _, blocks, _ = trit.shape
    groups = (width + 4) // 5
    digits = torch.ones(
        (chunk, blocks, 128, groups * 5, 2), dtype=torch.int16, device=trit.device
    )
    digits[:, :, :, :width, :] = (trit + 1).permute(0, 3, 4, 2, 1)
    powers = torch.tensor(_POWERS, dtype=torch.int16, device=trit.device)
    packed = (digits.reshape(chunk, blocks, 128, groups, 5, 2) * powers[:, None]).sum(4)
    out = torch.full(
        (chunk, blocks, 128, stride), ZERO_CODE, dtype=torch.uint8, device=trit.device
    )
    out[..., : 2 * groups] = packed.reshape(chunk, blocks, 128, 2 * groups).to(torch.uint8)
    return out


def build_sketch(
    weights: Tensor, signs: Tensor | None = None, *, chunk: int = 8, device_kernel: bool = False
) -> tuple[Tensor, Tensor]:
    """Build (codes, statistics) from native gate/up rows [E, 2 I, H].

    Each rotated 128-coordinate block of a row is ternarised by the TWN rule
    (sketch.py:84-150) and packed in the layout described in the module
    docstring. `chunk` experts are processed at a time so the FP32 copy stays
    transient. Returns uint8 codes [E, sketch_storage_bytes(2 I, H)] and FP16
    statistics [E, 2 I, H // 128, 2].

    The default is the torch construction on the weights' device, whose codes
    are the reference's. `device_kernel=True` builds BF16 device weights in
    one HIP launch instead (cfmoe_build_sketch, about 20 times faster per
    layer); its sums run in the kernel's order, so a trit can differ from the
    torch construction where |v| lies within an FP32 rounding of 0.7 mean|v|.
    """
    experts, rows, hidden = weights.shape
    if hidden % 128 or rows % 2:
        raise ValueError(
            "Ternary sketch requires 128-coordinate blocks and paired gate/up rows"
        )
    if device_kernel:
        if not (weights.is_cuda and weights.dtype == torch.bfloat16):
            raise ValueError("device_kernel builds BF16 weights on the GPU")
        return _build_sketch_device(weights, signs)
    return _build_sketch_torch(weights, signs, chunk)


def _build_sketch_torch(weights: Tensor, signs: Tensor | None, chunk: int = 8) -> tuple[Tensor, Tensor]:
    """The torch construction of build_sketch (any device), `chunk` experts at a time."""
    experts, rows, hidden = weights.shape
    blocks, width = hidden // 128, rows // 2
    stride = sketch_code_stride(rows)
    body = stride - stride % 32
    tail = stride % 32
    device = weights.device
    codes = torch.full(
        (experts, sketch_storage_bytes(rows, hidden)),
        ZERO_CODE,
        dtype=torch.uint8,
        device=device,
    )
    physical = torch.empty((experts, blocks, 2, rows), dtype=torch.float16, device=device)
    for begin in range(0, experts, chunk):
        end = min(experts, begin + chunk)
        value = weights[begin:end].float().reshape(end - begin, rows, blocks, 128)
        if signs is not None:
            value = rotate_blocks(value, signs)
        trit, scale, residual = _ternarise(value)
        physical[begin:end, :, 0, :] = scale.transpose(1, 2).to(torch.float16)
        physical[begin:end, :, 1, :] = residual.transpose(1, 2).to(torch.float16)
        packed = _pack_bytes(
            trit.reshape(end - begin, 2, width, blocks, 128), width, stride
        )
        codes[begin:end, : blocks * 128 * body] = packed[..., :body].reshape(
            end - begin, -1
        )
        if tail:
            tails = torch.full(
                (end - begin, (blocks + 1) // 2 * 2, 128, tail),
                ZERO_CODE,
                dtype=torch.uint8,
                device=device,
            )
            tails[:, :blocks] = packed[..., body:]
            codes[begin:end, blocks * 128 * body :] = (
                tails.reshape(end - begin, -1, 2, 128, tail)
                .transpose(2, 3)
                .reshape(end - begin, -1)
            )
    return codes, physical.permute(0, 3, 1, 2)


def _build_sketch_device(weights: Tensor, signs: Tensor | None) -> tuple[Tensor, Tensor]:
    """build_sketch of a device tensor: one HIP launch (cfmoe_build_sketch).

    Same format and rule as the torch construction below it; the sums of
    mean|v|, the scale and the residual run in the kernel's order, so a trit
    can differ only for |v| within an FP32 rounding of 0.7 mean|v|. Raises if
    the HIP library is missing (no host fallback for device weights).
    """
    from calibration_free_moe.reader import _ext

    experts, rows, hidden = weights.shape
    device = weights.device
    source = weights.detach().contiguous()
    rotation = None
    if signs is not None:
        rotation = signs.to(device=device, dtype=torch.int8).contiguous()
        if rotation.numel() != hidden:
            raise ValueError("rotation signs must have one entry per hidden coordinate")
    codes = torch.full(
        (experts, sketch_storage_bytes(rows, hidden)), ZERO_CODE, dtype=torch.uint8, device=device
    )
    physical = torch.empty((experts, hidden // 128, 2, rows), dtype=torch.float16, device=device)
    with torch.cuda.device(device):
        _ext.check(
            _ext.library().cfmoe_build_sketch(
                experts, rows // 2, hidden, source.data_ptr(),
                None if rotation is None else rotation.data_ptr(),
                codes.data_ptr(), physical.data_ptr(),
                torch.cuda.current_stream(device).cuda_stream,
            )
        )
    return codes, physical.permute(0, 3, 1, 2)


def code_offsets(rows: int, hidden: int, device: torch.device | str = "cpu") -> Tensor:
    """Byte offset of every (row, coordinate) trit byte: int64 [rows, hidden]."""
    width, blocks = rows // 2, hidden // 128
    stride = sketch_code_stride(rows)
    body, tail = stride - stride % 32, stride % 32
    row = torch.arange(rows, device=device)
    byte = 2 * ((row % width) // 5) + row // width
    coordinate = torch.arange(hidden, device=device)
    block, local = coordinate // 128, coordinate % 128
    offset = (coordinate * body)[None, :] + byte[:, None]
    if tail:
        tail_offset = (
            blocks * 128 * body
            + (((block // 2) * 128 + local) * 32 + (block % 2) * 16)[None, :]
            + (byte - body)[:, None]
        )
        offset = torch.where(byte[:, None] < body, offset, tail_offset)
    return offset


def unpack_sketch(codes: Tensor, rows: int, hidden: int) -> Tensor:
    """Decode packed codes [..., storage] into int8 trits [..., rows, hidden]."""
    width = rows // 2
    offset = code_offsets(rows, hidden, codes.device)
    digit = (torch.arange(rows, device=codes.device) % width) % 5
    packed = codes[..., offset].to(torch.int32)
    divisor = torch.tensor(_POWERS, device=codes.device, dtype=torch.int32)[digit]
    return ((packed // divisor[:, None]) % 3 - 1).to(torch.int8)


def differentiable_sketch_feature(
    x: Tensor,
    codes: Tensor,
    statistics: Tensor,
    signs: Tensor | None,
    *,
    unpacked: Tensor | None = None,
    checkpoint_cached: bool = False,
    activation: GatedActivation = "silu",
    input_is_rotated: bool = False,
    screen_coordinates: int = 128,
) -> Tensor:
    """BF16 sketch feature phi(g) u of every channel, differentiable in x.

    The feature recovery encodes for a skipped channel (sketch.py:153-206):
    g and u are the sketch projections of the (masked) rotated input, rounded
    to BF16 before phi. Gradients reach x only.
    """
    blocks = statistics.shape[-2]
    rows = statistics.shape[-3]

    def project(input_x: Tensor) -> Tensor:
        trits = unpacked if unpacked is not None else unpack_sketch(codes, rows, blocks * 128)
        trits = trits.float().reshape(rows, blocks, 128)
        rotated = input_x if input_is_rotated else rotate_blocks(input_x, signs)
        kept = mask_rotated_blocks(rotated, screen_coordinates).reshape(-1, blocks, 128)
        per_block = torch.einsum("tbc,rbc->trb", kept, trits)
        projection = (per_block * statistics[..., 0].float()[None]).sum(-1)
        g, u = projection.chunk(2, dim=-1)
        return (activate(g.bfloat16().float(), activation) * u.bfloat16().float()).bfloat16()

    if unpacked is None or checkpoint_cached:
        return checkpoint(project, x, use_reentrant=False)
    return project(x)
