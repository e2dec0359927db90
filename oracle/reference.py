"""Torch fp32 restatement of the reference FlashMLP path (test infrastructure only).

reference forward: flashmlp.py:671-686  (z = bmm(x, w1); h = act(z); o = bmm(h, w2))
activations:       flashmlp.py:676-683  (leaky_relu slope 0.01, silu, sigmoid, else linear)
gradients:         PyTorch autograd of that forward (the north star's oracle), on the CPU.
manual backward:   flashmlp.py:689-723  (kept for cross-checks; Leaky ReLU derivative 1 at 0)
"""
from __future__ import annotations

from typing import Tuple

import torch


def act(z: torch.Tensor, activation: str) -> torch.Tensor:
    """flashmlp.py:676-683"""
    if activation == "leaky_relu":
        return torch.nn.functional.leaky_relu(z, negative_slope=0.01)
    if activation == "silu":
        return torch.nn.functional.silu(z)
    if activation == "sigmoid":
        return torch.sigmoid(z)
    return z


def torch_fwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, activation: str = "") -> torch.Tensor:
    """flashmlp.py:671-686 in the dtype of the inputs."""
    return torch.bmm(act(torch.bmm(x, w1), activation), w2)


def autograd_grads(x, w1, w2, do, activation: str = "", dtype=torch.float32):
    """Forward and autograd gradients on the CPU in `dtype` (default fp32), from the given
    (already io-quantised) inputs. Returns (o, dx, dw1, dw2) in `dtype`."""
    xs = x.detach().to("cpu", dtype).requires_grad_(True)
    a = w1.detach().to("cpu", dtype).requires_grad_(True)
    b = w2.detach().to("cpu", dtype).requires_grad_(True)
    g = do.detach().to("cpu", dtype)
    o = torch_fwd(xs, a, b, activation)
    o.backward(g)
    return o.detach(), xs.grad, a.grad, b.grad


def manual_bwd(x, w1, w2, do, activation: str = "") -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """flashmlp.py:689-723 (note: Leaky ReLU derivative is 1 where z == 0)."""
    z = torch.bmm(x, w1)
    h = act(z, activation)
    dh = torch.bmm(do, w2.transpose(-1, -2))
    dw2 = torch.bmm(h.transpose(-1, -2), do)
    if activation == "leaky_relu":
        dz = dh * torch.where(z >= 0, 1.0, 0.01).to(dh.dtype)
    elif activation == "silu":
        sig = torch.sigmoid(z)
        dz = dh * (sig + z * sig * (1 - sig))
    elif activation == "sigmoid":
        dz = dh * h * (1 - h)
    else:
        dz = dh
    dx = torch.bmm(dz, w1.transpose(-1, -2))
    dw1 = torch.bmm(x.transpose(-1, -2), dz)
    return dx, dw1, dw2
