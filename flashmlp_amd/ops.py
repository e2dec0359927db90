"""torch.library registration of the FlashMLP operators (torch.compile / FakeTensor support).

Two custom operators wrap the same C ABI calls as flashmlp_fwd / flashmlp_bwd:

    torch.ops.flashmlp_amd.fwd(x, w1, w2, activation="") -> o
    torch.ops.flashmlp_amd.bwd(x, w1, w2, do, activation="", accurate_dw=False) -> (dx, dw1, dw2)

Each has a fake (meta) implementation that only checks shapes and allocates outputs, so
FakeTensor tracing, torch.export and torch.compile see through them without launching
anything, and `fwd` carries an autograd formula that calls `bwd` (saving only x, w1, w2,
as FlashMLPFunction does, flashmlp.py:545-557). `flashmlp(x, w1, w2, activation,
accurate_dw=False)` is the differentiable entry point; FlashMLP uses it while torch.compile
traces the module.

The real implementations are registered for the "cuda" device type only (HIP on ROCm):
there is no CPU kernel, and calling the operators on CPU tensors raises.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .flashmlp import flashmlp_bwd, flashmlp_fwd


def _check_shapes(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> None:
    # the reference's shape assertions (flashmlp.py:443-447), as symbolic-shape checks
    torch._check(x.dim() == 3 and w1.dim() == 3 and w2.dim() == 3, lambda: "x, w1, w2 must be 3-D")
    torch._check(x.shape[0] == w1.shape[0], lambda: "Number of heads must match")
    torch._check(x.shape[0] == w2.shape[0], lambda: "Number of heads must match")
    torch._check(x.shape[2] == w1.shape[1], lambda: "Hidden dimension mismatch")
    torch._check(w1.shape[2] == w2.shape[1], lambda: "Intermediate dimension mismatch")
    torch._check(x.shape[2] == w2.shape[2], lambda: "Output dimension mismatch")


@torch.library.custom_op("flashmlp_amd::fwd", mutates_args=(), device_types="cuda")
def fwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, activation: str = "",
        accurate_dw: bool = False) -> torch.Tensor:
    """O = act(x @ w1) @ w2 per head on the gfx950 kernels (flashmlp.py:428-477).
    accurate_dw only selects the backward's dW mode (carried to bwd by the autograd formula)."""
    return flashmlp_fwd(x, w1, w2, activation)


@fwd.register_fake
def _fwd_fake(x, w1, w2, activation="", accurate_dw=False):
    _check_shapes(x, w1, w2)
    return x.new_empty(x.shape)


@torch.library.custom_op("flashmlp_amd::bwd", mutates_args=(), device_types="cuda")
def bwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, do: torch.Tensor,
        activation: str = "", accurate_dw: bool = False) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx, dw1, dw2) with recomputation on the gfx950 kernels (flashmlp.py:480-538)."""
    return flashmlp_bwd(x, w1, w2, do, activation, accurate_dw=accurate_dw)


@bwd.register_fake
def _bwd_fake(x, w1, w2, do, activation="", accurate_dw=False):
    _check_shapes(x, w1, w2)
    torch._check(x.shape == do.shape, lambda: "Gradient shape mismatch")
    return x.new_empty(x.shape), w1.new_empty(w1.shape), w2.new_empty(w2.shape)


def _setup_context(ctx, inputs, output):
    x, w1, w2, activation, accurate_dw = inputs
    ctx.save_for_backward(x, w1, w2)
    ctx.activation = activation
    ctx.accurate_dw = accurate_dw


def _backward(ctx, do):
    x, w1, w2 = ctx.saved_tensors
    dx, dw1, dw2 = bwd(x, w1, w2, do, ctx.activation, ctx.accurate_dw)
    return dx, dw1, dw2, None, None


fwd.register_autograd(_backward, setup_context=_setup_context)


def flashmlp(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, activation: str = "",
             accurate_dw: bool = False) -> torch.Tensor:
    """Differentiable FlashMLP through the registered operator (traceable by torch.compile)."""
    return torch.ops.flashmlp_amd.fwd(x, w1, w2, activation, accurate_dw)
