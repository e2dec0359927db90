"""The tuned forward at D = 256 (fwd_kernel with four waves of 32 rows, one per SIMD; dense 16-bit
tensors with E % 8 == 0; the backward of such shapes runs on the generic kernels).

Each case checks through the C ABI:
  * the fp32 sums (FMLP_OUT_F32) against the oracle's cast-point emulation at the north star's
    1e-4, and against the generic kernel's sums for the same values passed as a non-dense view
    (so the generic path takes them) within 1e-5 (summation order only);
  * the io output against the fp32 autograd oracle at the parity bar (3e-2 + 3e-2 |ref|),
    every element written (output NaN-filled first).
"""
import ctypes
import sys

import pytest
import torch

from flashmlp_amd import _lib
from oracle import emulate, reference
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu

_DT = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16}
CASES = [(dt, act) for dt in (torch.float16, torch.bfloat16) for act in ("silu", "leaky_relu", "sigmoid", "")]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _normrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _fwd(x, w1, w2, act, code, out_dtype, strided=False):
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    o = torch.full((H, B, D), float("nan"), dtype=out_dtype, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a = _lib.ACT_CODES[act]
    if strided:
        st = L.fmlp_fwd_strided(_ptr(x), _ptr(w1), _ptr(w2), _ptr(o), H, B, D, E, _lib.strides(x), _lib.strides(w1),
                                _lib.strides(w2), code, a, stream)
    else:
        st = L.fmlp_fwd(_ptr(x), _ptr(w1), _ptr(w2), _ptr(o), H, B, D, E, code, a, stream)
    _lib.check(st, "forward")
    torch.cuda.synchronize()
    return o


def _check(H, B, D, E, dt, act, seed):
    code = _DT[dt]
    _say(f"[fwd-d256] H={H} B={B} D={D} E={E} {dt} act='{act}' seed={seed}")
    x, w1, w2, _ = make_inputs(H, B, D, E, dt, 1.0, seed=seed, with_do=False)
    xd, w1d, w2d = (t.cuda() for t in (x, w1, w2))
    # the same X values in a buffer with padded rows: a non-dense view, read by the generic kernel
    xpad = torch.zeros(H, B, D + 8, dtype=dt, device="cuda")
    xpad[:, :, :D] = xd
    xv = xpad[:, :, :D]
    assert not xv.is_contiguous()

    s_tuned = _fwd(xd, w1d, w2d, act, code | _lib.FMLP_OUT_F32, torch.float32)
    s_gen = _fwd(xv, w1d, w2d, act, code | _lib.FMLP_OUT_F32, torch.float32, strided=True)
    e = emulate.emu_fwd(x, w1, w2, act, dt, round_out=False)
    rel_e, rel_g = _normrel(s_tuned.cpu(), e), _normrel(s_tuned, s_gen)
    _say(f"[fwd-d256] fp32 sums rel to emulation {rel_e:.3g}, to the generic kernel {rel_g:.3g}")
    assert torch.isfinite(s_tuned).all()
    assert rel_e <= 1e-4 and rel_g <= 1e-5

    o = _fwd(xd, w1d, w2d, act, code, dt)
    ro = reference.autograd_grads(x, w1, w2, torch.zeros_like(x), act)[0]
    bad = ((o.cpu().float() - ro).abs() > 3e-2 + 3e-2 * ro.abs()).sum().item()
    _say(f"[fwd-d256] io outside 3e-2: {bad}")
    assert torch.isfinite(o.float()).all() and bad == 0


@pytest.mark.parametrize("dt,act", CASES, ids=[f"{str(d).split('.')[-1]}-{a or 'linear'}" for d, a in CASES])
def test_tuned_forward_d256(dt, act):
    _check(2, 300, 256, 136, dt, act, seed=21)  # B tail, E-chunk tail (136 = 4 * 32 + 8)


def test_tuned_forward_d256_larger_and_split():
    _check(4, 1024, 256, 512, torch.bfloat16, "silu", seed=22)
    n = torch.cuda.get_device_properties(0).multi_processor_count
    # one ragged tile past n full ones: the forward's split tiles through fmlp_fwd_ws
    H, B, D, E, dt, act = 1, n * 128 + 1, 256, 256, torch.float16, "sigmoid"
    L = _lib.lib()
    ws_n = L.fmlp_fwd_workspace_bytes(H, B, D, E, _DT[dt])
    _say(f"[fwd-d256] split shape H={H} B={B} ws={ws_n}")
    assert ws_n > 0
    x, w1, w2, _ = make_inputs(H, B, D, E, dt, 1.0, seed=23, with_do=False)
    xd, w1d, w2d = (t.cuda() for t in (x, w1, w2))
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    o = torch.full((H, B, D), float("nan"), dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.fmlp_fwd_ws(_ptr(xd), _ptr(w1d), _ptr(w2d), _ptr(o), H, B, D, E, _DT[dt] | _lib.FMLP_OUT_F32,
                             _lib.ACT_CODES[act], _ptr(ws), ws_n, stream), "forward")
    torch.cuda.synchronize()
    e = emulate.emu_fwd(x, w1, w2, act, dt, round_out=False)
    rel = _normrel(o.cpu(), e)
    _say(f"[fwd-d256] split fp32 sums rel {rel:.3g}")
    assert torch.isfinite(o).all() and rel <= 1e-4
