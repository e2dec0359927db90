"""FlashMLP Python API on MI355X: the reference's interface over the gfx950 HIP library.

Same names, arguments, shapes and assertion messages as the reference module
(flashmlp.py:428-616):

    flashmlp_fwd(x, w1, w2, activation="") -> o                       (H,B,D)
    flashmlp_bwd(x, w1, w2, do, activation="") -> (dx, dw1, dw2)      (H,B,D),(H,D,E),(H,E,D)
    FlashMLPFunction.apply(x, w1, w2, activation)
    FlashMLP(num_heads, hidden_dim, intermediate_dim, activation="silu",
             dtype=torch.float16, device="cuda")

plus one opt-in the reference does not have: accurate_dw=True (flashmlp_bwd keyword,
FlashMLPFunction's fifth argument, FlashMLP constructor argument) computes dW1 and dW2 with
h and dZ split into two io-dtype terms (hi + lo) instead of rounded to the io dtype, for
elementwise agreement with an fp32 computation at large B (twice the dW MFMA work).

O = act(X W1) W2 per head with act in {"", "silu", "leaky_relu", "sigmoid"}; an unknown
activation string means linear, as in the reference. Every call launches the HIP kernels
of libflashmlp.so asynchronously on torch's current stream of the tensors' device; there
is no other execution path.

Differences from the reference, all deliberate:
  * outputs are allocated with torch.empty (the kernels overwrite every element) instead of
    torch.zeros_like (flashmlp.py:462,516-518);
  * flashmlp_bwd also checks the head counts (flashmlp.py:496-499 omits them);
  * Leaky ReLU's derivative at Z == 0 is autograd's 0.01 (flashmlp.py:33-34 uses 1.0);
  * io dtypes are fp16, bf16 and fp32 (fp32 in true fp32, where the reference's tl.dot would
    use its default reduced input precision); other dtypes raise TypeError;
  * strided inputs are accepted: shapes with kernels of their own (16-bit io, D in {64, 128,
    256}, E % 8 == 0) copy them to dense tensors, as the reference's reshape / contiguous does
    (flashmlp.py:453-459,508); every other shape reads the views in place (generic kernels),
    where the reference would copy them or fail its contiguity assertions.
"""
from __future__ import annotations

import functools
from typing import Tuple

import numpy as np
import torch

from . import _lib

try:  # the per-call fast path over the same C ABI (fmlp_py.cpp); the ctypes path otherwise
    from . import _fmlp_fast as _fast
except ImportError:
    _fast = None

_DTYPES = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16,
           torch.float32: _lib.FMLP_DTYPE_F32}


def _act_code(activation: str) -> int:
    return _lib.ACT_CODES.get(activation, 0)


def _check_tensors(*ts: torch.Tensor) -> int:
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"FlashMLP runs on an AMD GPU through HIP; got a tensor on {dev} (move inputs to 'cuda')")
    dt = ts[0].dtype
    if dt not in _DTYPES:
        raise TypeError(f"FlashMLP supports float16, bfloat16 and float32 inputs, got {dt}")
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on one device ({dev} vs {t.device})")
        if t.dtype != dt:
            raise TypeError(f"all tensors must share one dtype ({dt} vs {t.dtype})")
    return _DTYPES[dt]


@functools.lru_cache(maxsize=256)
def _ws_bytes(device_index: int, H: int, B: int, D: int, E: int, dtype: int) -> int:
    # the backward plan depends only on the shapes, the dW mode flag and the device's CU count;
    # asked once per (device, shape, flags)
    return int(_lib.lib().fmlp_bwd_workspace_bytes(H, B, D, E, dtype))


@functools.lru_cache(maxsize=256)
def _fwd_ws_bytes(device_index: int, H: int, B: int, D: int, E: int, dtype: int) -> int:
    # the forward's split tiles (small grids, a short last round of tiles): fp32 partials
    return int(_lib.lib().fmlp_fwd_workspace_bytes(H, B, D, E, dtype))


def _dense(t: torch.Tensor) -> torch.Tensor:
    # the tuned kernels use 16-byte vector accesses on dense tensors: a strided view, or one at
    # a storage offset that is not a multiple of 16 bytes, is copied
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _ptr(t):
    # device address of an output, or NULL for one that is not computed
    return t.data_ptr() if t is not None else None


def _alloc_ws(nbytes: int, device: torch.device):
    # a call's workspace (None when the plan needs none)
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


@functools.lru_cache(maxsize=1024)
def _own_kernels(D: int, E: int, dtype: int) -> bool:
    # shapes with kernels of their own, which take dense 16-byte aligned tensors: the tuned
    # kernels (fmlp_shape_tuned) and the D = 256 programs (16-bit io, E % 8 == 0); views of
    # other shapes go to the generic kernels in place
    if _lib.lib().fmlp_shape_tuned(D, E, dtype):
        return True
    return D == 256 and E % 8 == 0 and dtype in (_lib.FMLP_DTYPE_F16, _lib.FMLP_DTYPE_BF16)


# torch's current HIP stream of a device, as the raw handle the C ABI takes, and the current
# device: the private accessors skip building a torch.cuda.Stream object (about 2 us per call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def _stream_of(index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def _io_code(x: torch.Tensor, *ts: torch.Tensor):
    """The io dtype code when every tensor is a GPU tensor of x's dtype on x's device (the common
    case, checked with the cheapest accessors), else the reason raised by _check_tensors."""
    dt = x.dtype
    d = x.get_device()
    code = _DTYPES.get(dt)
    if d < 0 or code is None or any(t.dtype is not dt or t.get_device() != d for t in ts):
        return _check_tensors(x, *ts)
    return code


def _dense_all(*ts: torch.Tensor):
    # the tuned kernels' inputs: unchanged when all are dense and 16-byte aligned
    if all(t.is_contiguous() and t.data_ptr() % 16 == 0 for t in ts):
        return ts
    return tuple(_dense(t) for t in ts)


def _empty_as(t: torch.Tensor, shape) -> torch.Tensor:
    # a dense output of t's shape, dtype and device (empty_like is the cheapest allocation)
    return torch.empty_like(t) if t.is_contiguous() else t.new_empty(shape)


def _current_device() -> int:
    return _get_device() if _get_device is not None else torch.cuda.current_device()


def flashmlp_fwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, activation: str = "") -> torch.Tensor:
    """FlashMLP forward pass (reference: flashmlp.py:428-477).

    Args:
        x: (H, B, D); w1: (H, D, E); w2: (H, E, D); activation: "silu", "leaky_relu",
        "sigmoid" or "" (linear).
    Returns:
        O = act(x @ w1) @ w2 of shape (H, B, D), dtype of x.
    """
    H, B, D = x.shape
    H1, D1, E = w1.shape
    H2, E2, D2 = w2.shape
    assert H == H1, "Number of heads must match"
    assert H == H2, "Number of heads must match"
    assert D == D1, "Hidden dimension mismatch"
    assert E == E2, "Intermediate dimension mismatch"
    assert D == D2, "Output dimension mismatch"

    if _fast is not None:  # 16-bit, one GPU, dense and aligned, a tuned shape: else None
        r = _fast.fwd(x, w1, w2, _act_code(activation))
        if r is not None:
            if r[0]:
                _lib.check(r[0], "forward")
            return r[1]
    dtype = _io_code(x, w1, w2)
    o = _empty_as(x, (H, B, D))
    L = _lib.lib()
    dev = x.get_device()
    prev = _current_device()
    if prev != dev:  # the library launches on the current device
        torch.cuda.set_device(dev)
    try:
        stream = _stream_of(dev)
        if _own_kernels(D, E, dtype):
            x, w1, w2 = _dense_all(x, w1, w2)
            ws_bytes = _fwd_ws_bytes(dev, H, B, D, E, dtype)
            try:
                ws = _alloc_ws(ws_bytes, x.device)
            except torch.OutOfMemoryError:  # the kernels then run every tile whole
                ws, ws_bytes = None, 0
            st = L.fmlp_fwd_ws(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), o.data_ptr(), H, B, D, E, dtype,
                               _act_code(activation), ws.data_ptr() if ws is not None else None, ws_bytes, stream)
        else:
            st = L.fmlp_fwd_strided(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), o.data_ptr(), H, B, D, E,
                                    _lib.strides(x), _lib.strides(w1), _lib.strides(w2), dtype,
                                    _act_code(activation), stream)
    finally:
        if prev != dev:
            torch.cuda.set_device(prev)
    _lib.check(st, "forward")
    return o


def flashmlp_bwd(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, do: torch.Tensor,
                 activation: str = "", *, accurate_dw: bool = False, recompute: bool = False,
                 _needs: Tuple[bool, bool] = (True, True)) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """FlashMLP backward pass (reference: flashmlp.py:480-538).

    Recomputes Z = x @ w1 and h = act(Z) instead of reading stored activations.
    Returns (dx, dw1, dw2) shaped like (x, w1, w2). For large shapes the library stores dZ in
    a temporary workspace (H x ceil(E/128)*128 x ceil(B/256)*256 io elements) and computes dx
    from it; recompute=True keeps the reference's recompute-only form, whose extra memory is
    at most the fp32 dW partials, and it is also taken when the stored-dZ workspace cannot be
    allocated. accurate_dw=True takes h and dZ into the dW products as
    hi + lo io-dtype terms. Both keywords have no counterpart in the reference. `_needs`
    (need dx, need dw1 and dw2; FlashMLPFunction passes autograd's needs_input_grad) skips the
    programs of a gradient nobody asked for and returns None in its place.
    """
    H, B, D = x.shape
    H1, D1, E = w1.shape
    H2, E2, D2 = w2.shape
    assert H == H1, "Number of heads must match"
    assert H == H2, "Number of heads must match"
    assert D == D1, "Hidden dimension mismatch"
    assert E == E2, "Intermediate dimension mismatch"
    assert D == D2, "Output dimension mismatch"
    assert x.shape == do.shape, "Gradient shape mismatch"

    need_dx, need_dw = bool(_needs[0]), bool(_needs[1])
    flags = (_lib.FMLP_DW_HILO if accurate_dw else 0) | (_lib.FMLP_BWD_RECOMPUTE if recompute else 0)
    if not (need_dx and need_dw):
        flags |= (0 if need_dx else _lib.FMLP_BWD_NO_DX) | (0 if need_dw else _lib.FMLP_BWD_NO_DW)
    if _fast is not None and (need_dx or need_dw):  # as in flashmlp_fwd
        r = _fast.bwd(x, w1, w2, do, _act_code(activation), flags)
        if r is not None:
            if r[0]:
                _lib.check(r[0], "backward")
            return r[1], r[2], r[3]
    dtype = _io_code(x, w1, w2, do)
    flags |= dtype
    dx = _empty_as(x, (H, B, D)) if need_dx else None
    dw1 = _empty_as(w1, (H, D, E)) if need_dw else None
    dw2 = _empty_as(w2, (H, E, D)) if need_dw else None
    if not (need_dx or need_dw):
        return dx, dw1, dw2
    L = _lib.lib()
    dev = x.get_device()
    prev = _current_device()
    if prev != dev:  # the library launches on the current device
        torch.cuda.set_device(dev)
    try:
        stream = _stream_of(dev)
        if _own_kernels(D, E, dtype):
            x, w1, w2, do = _dense_all(x, w1, w2, do)
            ws_bytes = _ws_bytes(dev, H, B, D, E, flags)
            try:
                ws = _alloc_ws(ws_bytes, x.device)
            except torch.OutOfMemoryError:
                if flags & _lib.FMLP_BWD_RECOMPUTE:
                    raise
                # the stored-dZ form's workspace does not fit: the recompute form needs at most
                # the fp32 dW partials (the reference's backward allocates no workspace at all)
                flags |= _lib.FMLP_BWD_RECOMPUTE
                ws_bytes = _ws_bytes(dev, H, B, D, E, flags)
                ws = _alloc_ws(ws_bytes, x.device)
            st = L.fmlp_bwd(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), do.data_ptr(), _ptr(dx),
                            _ptr(dw1), _ptr(dw2), H, B, D, E, flags, _act_code(activation),
                            ws.data_ptr() if ws is not None else None, ws_bytes, stream)
        else:
            # the generic kernels' dW programs split B with fp32 partials in the workspace when
            # it is given; without one (it does not fit) they run unsplit
            ws_bytes = _ws_bytes(dev, H, B, D, E, flags)
            try:
                ws = _alloc_ws(ws_bytes, x.device)
            except torch.OutOfMemoryError:
                ws, ws_bytes = None, 0
            st = L.fmlp_bwd_strided(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), do.data_ptr(), _ptr(dx),
                                    _ptr(dw1), _ptr(dw2), H, B, D, E, _lib.strides(x), _lib.strides(w1),
                                    _lib.strides(w2), _lib.strides(do), flags, _act_code(activation),
                                    ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    finally:
        if prev != dev:
            torch.cuda.set_device(prev)
    _lib.check(st, "backward")
    return dx, dw1, dw2


class FlashMLPFunction(torch.autograd.Function):
    """Autograd binding (reference: flashmlp.py:545-557). Saves only (x, w1, w2)."""

    @staticmethod
    def forward(ctx, x, w1, w2, activation="", accurate_dw=False):
        o = flashmlp_fwd(x, w1, w2, activation)
        ctx.save_for_backward(x, w1, w2)
        ctx.activation = activation
        ctx.accurate_dw = bool(accurate_dw)
        return o

    @staticmethod
    def backward(ctx, do):
        x, w1, w2 = ctx.saved_tensors
        need_x, need_w1, need_w2 = ctx.needs_input_grad[:3]
        # only the programs of the gradients autograd asks for run (an input or weights that
        # need no gradient skip the dX or the dW programs)
        dx, dw1, dw2 = flashmlp_bwd(x, w1, w2, do, ctx.activation, accurate_dw=ctx.accurate_dw,
                                    _needs=(need_x, need_w1 or need_w2))
        return dx, (dw1 if need_w1 else None), (dw2 if need_w2 else None), None, None


class FlashMLP(torch.nn.Module):
    """Multi-head MLP module on the FlashMLP kernels (reference: flashmlp.py:564-616).

    Args:
        num_heads: number of heads H
        hidden_dim: hidden dimension D
        intermediate_dim: intermediate dimension E
        activation: "silu", "leaky_relu", "sigmoid" or ""
        dtype: weight dtype (float16 or bfloat16)
        device: device of the weights
        accurate_dw: dW products with hi + lo terms of h and dZ (no counterpart in the
            reference; see flashmlp_bwd)

    Parameters w1 (H, D, E) ~ randn / sqrt(E) and w2 (H, E, D) ~ randn / sqrt(D), as in
    the reference (flashmlp.py:586-591). A 2-D input (B, D) is expanded to every head and
    the output is the mean over heads (flashmlp.py:603-614).
    """

    def __init__(self, num_heads: int, hidden_dim: int, intermediate_dim: int,
                 activation: str = "silu", dtype=torch.float16, device="cuda", accurate_dw: bool = False):
        super().__init__()
        self.num_heads = num_heads
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.activation = activation
        self.accurate_dw = accurate_dw

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

        if torch.compiler.is_compiling():
            # the registered operator (flashmlp_amd.ops) is what torch.compile traces through
            from .ops import flashmlp as _op
            o = _op(x, self.w1, self.w2, self.activation, self.accurate_dw)
        else:
            o = FlashMLPFunction.apply(x, self.w1, self.w2, self.activation, self.accurate_dw)

        if squeeze_output:
            o = o.mean(dim=0)
        return o
