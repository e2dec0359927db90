"""The reference's unfused PyTorch path, kept for API compatibility and comparisons.

`PyTorchMLP`, `flashmlp_torch_fwd` and `flashmlp_torch_bwd` are public in the reference
module (flashmlp.py:619-723; example.py:8 imports PyTorchMLP) and are used there as the
speed/memory baseline: bmm -> activation -> bmm with the (H, B, E) intermediate stored.
They run wherever torch runs. The FlashMLP API (flashmlp_fwd, flashmlp_bwd,
FlashMLPFunction, FlashMLP) never calls them.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np
import torch


def _act(z: torch.Tensor, activation: str) -> torch.Tensor:
    if activation == "leaky_relu":
        return torch.nn.functional.leaky_relu(z, negative_slope=0.01)
    if activation == "silu":
        return torch.nn.functional.silu(z)
    if activation == "sigmoid":
        return torch.sigmoid(z)
    return z


class PyTorchMLP(torch.nn.Module):
    """Unfused multi-head MLP with FlashMLP's interface (reference: flashmlp.py:619-664)."""

    def __init__(self, num_heads: int, hidden_dim: int, intermediate_dim: int,
                 activation: str = "silu", dtype=torch.float16, device="cuda"):
        super().__init__()
        self.num_heads = num_heads
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.activation = activation
        self.w1 = torch.nn.Parameter(
            torch.randn(num_heads, hidden_dim, intermediate_dim, dtype=dtype, device=device) / np.sqrt(intermediate_dim)
        )
        self.w2 = torch.nn.Parameter(
            torch.randn(num_heads, intermediate_dim, hidden_dim, dtype=dtype, device=device) / np.sqrt(hidden_dim)
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() == 2:
            x = x.unsqueeze(0).expand(self.num_heads, -1, -1)
            squeeze_output = True
        else:
            squeeze_output = False
        z = torch.bmm(x, self.w1)
        h = _act(z, self.activation)
        o = torch.bmm(h, self.w2)
        if squeeze_output:
            o = o.mean(dim=0)
        return o


def flashmlp_torch_fwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, activation: str = "") -> torch.Tensor:
    """Unfused forward (reference: flashmlp.py:671-686)."""
    return torch.bmm(_act(torch.bmm(x, w1), activation), w2)


def flashmlp_torch_bwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, do: torch.Tensor,
                       activation: str = "") -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Manual unfused backward (reference: flashmlp.py:689-723), including its Leaky ReLU
    derivative of 1 at Z == 0."""
    z = torch.bmm(x, w1)
    h = _act(z, activation)
    dh = torch.bmm(do, w2.transpose(-1, -2).contiguous())
    dw2 = torch.bmm(h.transpose(-1, -2).contiguous(), do)
    if activation == "leaky_relu":
        dz = dh * torch.where(z >= 0, 1.0, 0.01).to(dh.dtype)
    elif activation == "silu":
        sig = torch.sigmoid(z)
        dz = dh * (sig + z * sig * (1 - sig))
    elif activation == "sigmoid":
        dz = dh * h * (1 - h)
    else:
        dz = dh
    dx = torch.bmm(dz, w1.transpose(-1, -2).contiguous())
    dw1 = torch.bmm(x.transpose(-1, -2).contiguous(), dz)
    return dx, dw1, dw2
