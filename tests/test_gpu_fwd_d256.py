"""The tuned kernels at D = 256: the forward (fwd_kernel with four waves of 32 rows, one per SIMD)
and the backward's dX programs (dx256_kernel, the same layout), for dense 16-bit tensors with
E % 8 == 0 (the backward's dW programs there, dw256_kernel, have tests of their own).

Each case checks through the C ABI:
  * the fp32 sums (FMLP_OUT_F32) against the oracle's cast-point emulation at the north star's
    1e-4, and against the generic kernel's sums for the same values passed as a non-dense view
    (so the generic path takes them) within 1e-5 (summation order only);
  * the io output against the fp32 autograd oracle at the parity bar (3e-2 + 3e-2 |ref|),
    every element written (output NaN-filled first);
  * for the backward, the fp32 sums of dX, dW1, dW2 against the emulation and the generic
    kernels likewise, and the partial backwards (FMLP_BWD_NO_DW, FMLP_BWD_NO_DX) bitwise equal
    to the full one.
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


def _bwd(x, w1, w2, do, act, code, out_dtype, strided=False):
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    dx = torch.full((H, B, D), float("nan"), dtype=out_dtype, device=x.device)
    dw1 = torch.full((H, D, E), float("nan"), dtype=out_dtype, device=x.device)
    dw2 = torch.full((H, E, D), float("nan"), dtype=out_dtype, device=x.device)
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a = _lib.ACT_CODES[act]
    st = L.fmlp_bwd_strided(_ptr(x), _ptr(w1), _ptr(w2), _ptr(do), _ptr(dx), _ptr(dw1), _ptr(dw2), H, B, D, E,
                            _lib.strides(x), _lib.strides(w1), _lib.strides(w2), _lib.strides(do), code, a, _ptr(ws),
                            n, stream)
    _lib.check(st, "backward")
    torch.cuda.synchronize()
    return dx, dw1, dw2


BWD_CASES = [(torch.float16, "silu", 2, 300, 136), (torch.bfloat16, "sigmoid", 2, 300, 136),
             (torch.bfloat16, "leaky_relu", 3, 1000, 512), (torch.float16, "", 2, 129, 264)]


@pytest.mark.parametrize("dt,act,H,B,E", BWD_CASES, ids=[f"{str(c[0]).split('.')[-1]}-{c[1] or 'linear'}-B{c[3]}"
                                                          for c in BWD_CASES])
def test_tuned_dx_d256(dt, act, H, B, E):
    D = 256
    code = _DT[dt]
    _say(f"[bwd-d256] H={H} B={B} D={D} E={E} {dt} act='{act}'")
    x, w1, w2, do = make_inputs(H, B, D, E, dt, 1.0, seed=31)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    xpad = torch.zeros(H, B, D + 8, dtype=dt, device="cuda")
    xpad[:, :, :D] = xd
    xv = xpad[:, :, :D]  # a non-dense view: the whole backward on the generic kernels

    s = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32)
    sg = _bwd(xv, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32)
    e = emulate.emu_bwd(x, w1, w2, do, act, dt, round_out=False)
    rel = {k: _normrel(g.cpu(), r) for k, g, r in zip(("dx", "dw1", "dw2"), s, e)}
    rel_g = [_normrel(a_, b_) for a_, b_ in zip(s, sg)]
    sums = " ".join(f"{k}={v:.3g}" for k, v in rel.items())
    _say(f"[bwd-d256] fp32 sums rel {sums}, dx/dw1/dw2 to generic {['%.3g' % r for r in rel_g]}")
    assert max(rel.values()) <= 1e-4 and max(rel_g) <= 1e-5

    dx, dw1, dw2 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    _, rdx, _, _ = reference.autograd_grads(x, w1, w2, do, act)
    bad = ((dx.cpu().float() - rdx).abs() > 3e-2 + 3e-2 * rdx.abs()).sum().item()
    _say(f"[bwd-d256] dx outside 3e-2: {bad}")
    assert torch.isfinite(dx.float()).all() and bad == 0
    # partial backwards: the same programs, bitwise
    dxo, _, _ = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_BWD_NO_DW, dt)
    _, dw1o, dw2o = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_BWD_NO_DX, dt)
    assert torch.equal(dx.view(torch.int16), dxo.view(torch.int16))
    assert torch.equal(dw1.view(torch.int16), dw1o.view(torch.int16))
    assert torch.equal(dw2.view(torch.int16), dw2o.view(torch.int16))
