"""FlashMLP for AMD Instinct MI355X (gfx950).

Fused multi-head MLP  O = act(X W1) W2  with a recomputing backward, as hand-written HIP
kernels behind a C ABI (include/flashmlp.h, libflashmlp.so). The Python API mirrors the
reference module `flashmlp`:

    from flashmlp_amd import flashmlp_fwd, flashmlp_bwd, FlashMLPFunction, FlashMLP, PyTorchMLP

`flashmlp_amd.flashmlp` (torch.ops.flashmlp_amd.fwd / .bwd) is the same computation as a
registered torch.library operator, for torch.compile and FakeTensor tracing.
"""
from .flashmlp import FlashMLP, FlashMLPFunction, flashmlp_bwd, flashmlp_fwd
from .baseline import PyTorchMLP, flashmlp_torch_bwd, flashmlp_torch_fwd
from . import ops
from .ops import flashmlp

__all__ = [
    "flashmlp_fwd",
    "flashmlp_bwd",
    "FlashMLPFunction",
    "FlashMLP",
    "PyTorchMLP",
    "flashmlp_torch_fwd",
    "flashmlp_torch_bwd",
    "flashmlp",
    "ops",
]
