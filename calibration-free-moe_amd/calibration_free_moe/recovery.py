"""Weight-only recovery bank of one layer: the rank-r subspace of its down columns.

Mirrors `subspace_bank` of the reference (scripts/build_weight_recovery_bank.py:
80-94): U holds the top-r left singular vectors of the layer's down columns
[H, E I] -- the eigenvectors of their Gram matrix D D^T -- and B_e = U^T D_e.
The reader adds U B_e p, the rank-r projection of the skipped channels'
estimated output, so only the subspace U U^T matters; each column of U is
fixed up to its sign, and a flipped column flips the matching row of every
B_e, leaving U B_e unchanged.

On the device the Gram matrix is accumulated in FP64 a few experts at a time
(one FP64 GEMM per chunk, so no [H, E I] FP64 copy of the layer is made) and
decomposed by the FP64 symmetric eigensolver on the same device; a device
without one raises instead of falling back to the host.
"""

from __future__ import annotations

import torch
from torch import Tensor


@torch.no_grad()
def subspace_bank(down: Tensor, rank: int, chunk: int = 16) -> tuple[Tensor, Tensor, float]:
    """Return (U [H, r], B = U^T D_e [E, r, I], captured energy) for down [E, H, I].

    FP64 outputs on the device of `down`; `captured` is the fraction of the
    squared Frobenius norm of the down columns that the r directions hold.
    `chunk` experts enter the Gram matrix per GEMM.
    """
    if down.dim() != 3:
        raise ValueError("down must be [experts, hidden, width]")
    experts, hidden, width = down.shape
    if not 1 <= rank <= hidden or chunk < 1:
        raise ValueError("rank must be in [1, hidden] and chunk positive")
    gram = torch.zeros(hidden, hidden, dtype=torch.float64, device=down.device)
    for begin in range(0, experts, chunk):
        columns = down[begin:begin + chunk].double().permute(1, 0, 2).reshape(hidden, -1)
        gram.addmm_(columns, columns.T)
    eigenvalues, eigenvectors = torch.linalg.eigh(gram)  # ascending
    decoder = eigenvectors[:, hidden - rank:].flip(-1).contiguous()
    total = eigenvalues.clamp_min(0).sum()
    captured = float(eigenvalues[hidden - rank:].clamp_min(0).sum() / total) if total > 0 else 0.0
    encoder = torch.empty(experts, rank, width, dtype=torch.float64, device=down.device)
    for begin in range(0, experts, chunk):
        end = min(experts, begin + chunk)
        encoder[begin:end] = torch.matmul(decoder.T, down[begin:end].double())
    return decoder, encoder, captured


__all__ = ["subspace_bank"]
