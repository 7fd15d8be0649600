"""Gated expert activations (reference `calibration_free_moe/activation.py:1-28`)."""

from __future__ import annotations

from typing import Literal

import torch.nn.functional as F
from torch import Tensor

GatedActivation = Literal["silu", "gelu_tanh"]


def model_activation(config: object) -> GatedActivation:
    """Map a Hugging Face config's `hidden_activation` to a gate activation.

    Configs without the field (OLMoE, Qwen) use SiLU (activation.py:11-21).
    """
    name = getattr(config, "hidden_activation", "silu")
    if name in ("gelu_pytorch_tanh", "gelu_tanh"):
        return "gelu_tanh"
    if name in ("silu", "swiglu"):
        return "silu"
    raise ValueError(f"Unsupported routed expert activation: {name}")


def activate(gate: Tensor, activation: GatedActivation) -> Tensor:
    """Apply phi: SiLU, or GELU with the tanh approximation (activation.py:24-28)."""
    if activation == "gelu_tanh":
        return F.gelu(gate, approximate="tanh")
    return F.silu(gate)
