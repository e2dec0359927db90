"""FlashMLP for AMD Instinct MI355X (gfx950).

Fused multi-head MLP  O = act(X W1) W2  with a recomputing backward, as hand-written HIP
kernels behind a C ABI (include/flashmlp.h, libflashmlp.so). The Python API mirrors the
reference module `flashmlp`:

    from flashmlp_amd import flashmlp_fwd, flashmlp_bwd, FlashMLPFunction, FlashMLP, PyTorchMLP
"""
from .flashmlp import FlashMLP, FlashMLPFunction, flashmlp_bwd, flashmlp_fwd
from .baseline import PyTorchMLP, flashmlp_torch_bwd, flashmlp_torch_fwd

__all__ = [
    "flashmlp_fwd",
    "flashmlp_bwd",
    "FlashMLPFunction",
    "FlashMLP",
    "PyTorchMLP",
    "flashmlp_torch_fwd",
    "flashmlp_torch_bwd",
]
