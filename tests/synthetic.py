"""Seeded synthetic MoE layers for the tests, the smoke check and the bench.

Shapes and distributions follow the benchmark configurations: BF16 weights
N(0, 0.02^2); a BF16 router N(0, 0.02^2) whose logits bf16(x W^T) go through
an FP32 softmax, top-k and renormalisation; hidden states N(0, 1) with a fixed
1 % of dimensions scaled by 20; the rank-R weight-only recovery map of
scripts/build_weight_recovery_bank.py:80-94 in the reference (U = top-R
eigenvectors of sum_e D_e D_e^T, B_e = U^T D_e, both BF16).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from calibration_free_moe.reader.progressive import recovery_geometry
from calibration_free_moe.recovery import subspace_bank
from calibration_free_moe.reader.sketch import block_hadamard_signs, build_sketch


@dataclass
class Layer:
    gate_up: Tensor  # [E, 2I, H] bf16
    down: Tensor  # logical [E, H, I] bf16 (row-major, not yet channel-major)
    encoder: Tensor  # [E, R, I] bf16
    decoder: Tensor  # [H, R] bf16
    codes: Tensor
    statistics: Tensor
    router: Tensor  # [E, H] bf16
    hidden: Tensor  # [T, H] bf16
    ids: Tensor  # [T, K] int64
    weights: Tensor  # [T, K] fp32


def hidden_states(tokens: int, hidden: int, generator: torch.Generator,
                  outlier_fraction: float = 0.01, outlier_scale: float = 20.0,
                  device: str | torch.device = "cpu") -> Tensor:
    x = torch.randn(tokens, hidden, generator=generator)
    count = max(1, round(outlier_fraction * hidden))
    dims = torch.randperm(hidden, generator=generator)[:count]
    x[:, dims] *= outlier_scale
    return x.to(torch.bfloat16).to(device)


def route(x: Tensor, router: Tensor, top_k: int) -> tuple[Tensor, Tensor]:
    """Softmax router: bf16 logits, FP32 softmax, top-k, renormalised weights."""
    logits = (x.float() @ router.float().T).to(torch.bfloat16).float()
    probabilities = torch.softmax(logits, dim=-1)
    weights, ids = probabilities.topk(top_k, dim=-1)
    return ids.to(torch.int64), (weights / weights.sum(-1, keepdim=True)).float()


def zipf_route(tokens: int, experts: int, top_k: int, generator: torch.Generator,
               s: float = 1.2) -> tuple[Tensor, Tensor]:
    """Skewed routing: Gumbel-top-k on log p_e with p_e proportional to rank^-s."""
    rank = torch.arange(1, experts + 1, dtype=torch.float64)
    popularity = rank.pow(-s)
    permutation = torch.randperm(experts, generator=generator)
    log_p = torch.log(popularity / popularity.sum())[permutation]
    gumbel = -torch.log(-torch.log(torch.rand(tokens, experts, generator=generator, dtype=torch.float64)))
    scores = log_p[None, :] + gumbel
    ids = scores.topk(top_k, dim=-1).indices
    weights = torch.softmax(scores.gather(1, ids), dim=-1).float()
    return ids.to(torch.int64), weights


def recovery_bank(down: Tensor, rank: int) -> tuple[Tensor, Tensor]:
    """B [E, R, I] and U [H, R] of the down weights [E, H, I], cast to BF16
    (the package's subspace_bank, on the device of `down`)."""
    u, b, _ = subspace_bank(down, rank)
    return b.to(torch.bfloat16), u.to(torch.bfloat16)


def make_layer(*, hidden: int, width: int, experts: int, top_k: int, rank: int,
               tokens: int, seed: int, std: float = 0.02, zipf: float | None = None,
               device: str | torch.device = "cpu") -> Layer:
    """One seeded layer plus a batch of routed decode tokens."""
    generator = torch.Generator().manual_seed(seed)
    gate_up = (torch.randn(experts, 2 * width, hidden, generator=generator) * std).to(
        torch.bfloat16
    )
    down = (torch.randn(experts, hidden, width, generator=generator) * std).to(torch.bfloat16)
    router = (torch.randn(experts, hidden, generator=generator) * std).to(torch.bfloat16)
    x = hidden_states(tokens, hidden, generator)
    if zipf is None:
        ids, weights = route(x, router, top_k)
    else:
        ids, weights = zipf_route(tokens, experts, top_k, generator, zipf)
    gate_up, down, router = gate_up.to(device), down.to(device), router.to(device)
    encoder, decoder = recovery_bank(down, rank)
    codes, statistics = build_sketch(gate_up, block_hadamard_signs(hidden, device))
    return Layer(gate_up, down, encoder, decoder, codes, statistics, router,
                 x.to(device), ids.to(device), weights.to(device))


def make_routed_layer(*, hidden: int, width: int, experts: int, top_k: int, rank: int,
                      tokens: int, seed: int, std: float = 0.02) -> Layer:
    """A full-width layer whose weights exist only for the routed experts.

    The router and hidden states come first; then each expert some token routes
    to gets its own seeded N(0, std^2) gate/up and down rows, the others stay
    zero (their sketch codes are the zero code). The recovery map is the bank
    of the routed experts. A token's computation reads nothing else, so this
    is the per-token work of a benchmark shape at a fraction of the set-up
    cost (CPU only).
    """
    generator = torch.Generator().manual_seed(seed)
    router = (torch.randn(experts, hidden, generator=generator) * std).to(torch.bfloat16)
    x = hidden_states(tokens, hidden, generator)
    ids, weights = route(x, router, top_k)
    gate_up = torch.zeros(experts, 2 * width, hidden, dtype=torch.bfloat16)
    down = torch.zeros(experts, hidden, width, dtype=torch.bfloat16)
    used = sorted(set(ids.reshape(-1).tolist()))
    for e in used:
        own = torch.Generator().manual_seed(seed * 100003 + e)
        gate_up[e] = (torch.randn(2 * width, hidden, generator=own) * std).to(torch.bfloat16)
        down[e] = (torch.randn(hidden, width, generator=own) * std).to(torch.bfloat16)
    index = torch.tensor(used)
    encoder_used, decoder = recovery_bank(down[index], rank)
    encoder = torch.zeros(experts, rank, width, dtype=torch.bfloat16)
    encoder[index] = encoder_used
    codes_used, stats_used = build_sketch(gate_up[index], block_hadamard_signs(hidden, "cpu"))
    codes = torch.full((experts, codes_used.shape[1]), 121, dtype=torch.uint8)
    codes[index] = codes_used
    statistics = torch.zeros((experts, hidden // 128, 2, 2 * width), dtype=torch.float16)
    statistics[index] = stats_used.permute(0, 2, 3, 1)
    statistics = statistics.permute(0, 3, 1, 2)
    return Layer(gate_up, down, encoder, decoder, codes, statistics, router, x, ids, weights)


def bits(tensor: Tensor) -> np.ndarray:
    """uint16 bit patterns of a BF16/FP16 tensor (CPU copy)."""
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_weights(layer: Layer, reader) -> "object":
    """The oracle's view of exactly the tensors the GPU reader holds."""
    from oracle import oracle

    statistics = reader.sketch_statistics.detach().cpu()
    physical = statistics.permute(0, 2, 3, 1).contiguous()  # [E, B, 2, 2I]
    geometry = reader.recovery_geometry
    return oracle.Weights(
        gate_up=bits(reader.native_gu),
        down=bits(reader.down.transpose(1, 2)),
        codes=reader.sketch_codes.detach().cpu().contiguous().numpy(),
        stats=bits(physical),
        norms=reader.norms.detach().cpu().contiguous().numpy(),
        signs=reader.sketch_signs.detach().cpu().contiguous().numpy(),
        encoder_t=None if reader.encoder is None else bits(reader.encoder),
        decoder=None if reader.decoder is None else bits(reader.decoder),
        geometry=None if geometry is None else geometry.detach().cpu().contiguous().numpy(),
    )


def cpu_weights(layer: Layer, point: bool = True):
    """The oracle's weights built on the CPU the way the reader builds them."""
    from oracle import oracle

    down = layer.down.float()
    norms = down.square().sum(1).sqrt()
    encoder_t = layer.encoder.transpose(1, 2).contiguous()
    geometry = None
    if not point:
        geometry = recovery_geometry(layer.down, norms, encoder_t, layer.decoder)
    physical = layer.statistics.permute(0, 2, 3, 1).contiguous()
    hidden = layer.gate_up.shape[2]
    return oracle.Weights(
        gate_up=bits(layer.gate_up),
        down=bits(layer.down.transpose(1, 2)),
        codes=layer.codes.contiguous().numpy(),
        stats=bits(physical),
        norms=norms.contiguous().numpy(),
        signs=block_hadamard_signs(hidden, "cpu").numpy(),
        encoder_t=bits(encoder_t),
        decoder=bits(layer.decoder),
        geometry=None if geometry is None else geometry.contiguous().numpy(),
    )
