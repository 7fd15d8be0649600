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
    """U [H, R] and B [E, R, I] from the down weights [E, H, I] (BF16 outputs)."""
    d = down.double() if down.device.type == "cpu" else down.float()
    gram = torch.zeros(d.shape[1], d.shape[1], dtype=d.dtype, device=d.device)
    for expert in range(d.shape[0]):
        gram += d[expert] @ d[expert].T
    try:
        _, vectors = torch.linalg.eigh(gram)
    except RuntimeError:  # no device eigensolver: solve on the host
        _, vectors = torch.linalg.eigh(gram.double().cpu())
        vectors = vectors.to(d.device, d.dtype)
    u = vectors[:, -rank:].flip(-1)
    b = torch.einsum("hr,ehi->eri", u, d)
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
        decoder_float = layer.decoder.float().T
        geometry = torch.zeros(down.shape[0], down.shape[2], 2)
        for expert in range(down.shape[0]):
            response = encoder_t[expert].float() @ decoder_float
            original = down[expert].T
            norm = norms[expert]
            alpha = (original * response).sum(-1) / torch.where(norm > 0, norm, torch.ones_like(norm))
            beta = (response.square().sum(-1) - alpha.square()).clamp_min(0).sqrt()
            geometry[expert, :, 0] = alpha
            geometry[expert, :, 1] = beta
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
