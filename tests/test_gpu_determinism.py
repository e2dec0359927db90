"""Run-to-run determinism and complete overwrite of the outputs, through the C ABI.

The library allocates its outputs with torch.empty where the reference zero-fills them
(flashmlp.py:462,516-518), and the backward's workspace (fp32 dW partials of a B split, the
stored dZ) is never cleared. So every case here fills the outputs and the workspace with NaN
bytes first, runs the call twice, and asserts that the two results are bitwise equal and
free of NaN: every output element is written, nothing depends on what the workspace held (the
stored-dZ form's padding rows past B and columns past E included), and the B-split reduction
sums its partials in a fixed order (no atomics).

Shapes: B not a multiple of the 256-row dZ tile or of the 32-row subtile, E not a multiple of
32, one B split of the dW programs; both backward forms, D 64 and 128, fp16 and bf16.
"""
import ctypes
import sys

import pytest
import torch

from flashmlp_amd import _lib
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu

_DT = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16}
FORMS = {"recompute": _lib.FMLP_BWD_RECOMPUTE, "stored_dz": _lib.FMLP_BWD_STORE_DZ}
CASES = [
    # H, B, D, E, dtype, act, seed
    (3, 2100, 64, 1000, torch.float16, "sigmoid", 51),
    (2, 8192, 128, 256, torch.bfloat16, "silu", 52),  # B split: fp32 partials, then dZ
    (2, 300, 128, 136, torch.bfloat16, "leaky_relu", 53),
]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _nan_like(shape, dtype):
    t = torch.empty(shape, dtype=dtype, device="cuda")
    t.view(torch.uint8).fill_(0xFF)  # NaN in fp16, bf16 and fp32
    return t


def _fwd(x, w1, w2, act):
    H, B, D = x.shape
    E = w1.shape[2]
    o = _nan_like((H, B, D), x.dtype)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().fmlp_fwd(_p(x), _p(w1), _p(w2), _p(o), H, B, D, E, _DT[x.dtype], _lib.ACT_CODES[act],
                                   stream), "forward")
    torch.cuda.synchronize()
    return o


def _bwd(x, w1, w2, do, act, flags):
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    code = _DT[x.dtype] | flags
    dx = _nan_like((H, B, D), x.dtype)
    dw1 = _nan_like((H, D, E), x.dtype)
    dw2 = _nan_like((H, E, D), x.dtype)
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
    ws = _nan_like((max(n, 16),), torch.uint8)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, code,
                          _lib.ACT_CODES[act], _p(ws), n, stream), "backward")
    torch.cuda.synchronize()
    return dx, dw1, dw2


@pytest.mark.parametrize("H,B,D,E,dt,act,seed", CASES)
def test_forward_deterministic_and_complete(H, B, D, E, dt, act, seed):
    x, w1, w2, _ = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=seed))
    _say(f"[determinism] forward H={H} B={B} D={D} E={E} {dt} act='{act}'")
    o1 = _fwd(x, w1, w2, act)
    o2 = _fwd(x, w1, w2, act)
    assert not torch.isnan(o1).any(), "forward left output elements unwritten"
    assert torch.equal(o1, o2), "forward results differ between two identical calls"


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("H,B,D,E,dt,act,seed", CASES)
def test_backward_deterministic_and_complete(H, B, D, E, dt, act, seed, form):
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=seed))
    _say(f"[determinism] backward {form} H={H} B={B} D={D} E={E} {dt} act='{act}'")
    r1 = _bwd(x, w1, w2, do, act, FORMS[form])
    r2 = _bwd(x, w1, w2, do, act, FORMS[form])
    for name, a, b in zip(("dx", "dw1", "dw2"), r1, r2):
        assert not torch.isnan(a).any(), f"{name}: output elements unwritten or a stale workspace value leaked in"
        assert torch.equal(a, b), f"{name}: results differ between two identical calls"
