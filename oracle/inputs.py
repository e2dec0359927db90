"""Seeded inputs for the BASELINE.json configurations (test infrastructure only).

Generation: torch.manual_seed(seed) on the CPU, fp32 draws in the order X, W1, W2, dO,
each cast to the io dtype (round to nearest even), so CPU oracle and GPU kernels see the
same io-representable values. Scales: X ~ N(0, x_std^2), W1 ~ N(0, 1/D), W2 ~ N(0, 1/E),
dO ~ N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    name: str
    H: int
    B: int
    D: int
    E: int
    dtype: torch.dtype
    activation: str
    x_std: float = 1.0


CONFIGS = {
    # cfg1 is the CPU fp32 oracle case; the GPU runs it in fp16 as cfg2
    "cfg1": Config("cfg1", 12, 1024, 64, 768, torch.float32, "silu"),
    "cfg2": Config("cfg2", 12, 1024, 64, 768, torch.float16, "silu"),
    "cfg3": Config("cfg3", 16, 8192, 128, 512, torch.bfloat16, "leaky_relu"),
    "cfg4": Config("cfg4", 32, 16384, 128, 1024, torch.bfloat16, "silu"),
    "cfg5_linear": Config("cfg5_linear", 8, 4097, 64, 2048, torch.float16, "", 2.0),
    "cfg5_sigmoid": Config("cfg5_sigmoid", 8, 4097, 64, 2048, torch.float16, "sigmoid", 2.0),
    # forward-only inference sweep of config 5 at B = 65536 (sigmoid; the tests also run linear)
    "cfg5s": Config("cfg5s", 8, 65536, 64, 2048, torch.float16, "sigmoid", 2.0),
}


def make_inputs(H, B, D, E, dtype=torch.bfloat16, x_std=1.0, seed=0, with_do=True):
    """Returns (x, w1, w2, do) on the CPU in `dtype` (do is None when with_do is False)."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(H, B, D, generator=g) * x_std).to(dtype)
    w1 = (torch.randn(H, D, E, generator=g) / D ** 0.5).to(dtype)
    w2 = (torch.randn(H, E, D, generator=g) / E ** 0.5).to(dtype)
    do = torch.randn(H, B, D, generator=g).to(dtype) if with_do else None
    return x, w1, w2, do


def config_inputs(cfg: Config, seed=0, with_do=True):
    return make_inputs(cfg.H, cfg.B, cfg.D, cfg.E, cfg.dtype, cfg.x_std, seed, with_do)
