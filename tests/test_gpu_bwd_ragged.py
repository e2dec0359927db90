"""The backward's split ragged dX tiles: when B is not a multiple of the dX programs' rows, each
head's last dX tile holds a few rows but costs a whole program, which can leave a round of H
programs on an otherwise idle device. The plan may split those tiles over E (fp32 partials in
the workspace, summed by a second launch in a fixed order); fmlp_bwd_plan reports it.

Each case (shapes where the plan splits on a 256-CU MI355X) checks, through the C ABI:
  * the fp32 sums (FMLP_OUT_F32) of dX, dW1, dW2 against the oracle's cast-point emulation at
    the north star's 1e-4, with dX and the workspace NaN-filled beforehand;
  * the io dX against the fp32 autograd oracle within the parity bar (3e-2 + 3e-2 |ref|);
  * bitwise equality of two calls (a fixed summation order), and of dX between the default and
    the accuracy dW mode (dX does not depend on the dW mode).
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
CASES = [
    ("cfg5", 8, 4097, 64, 2048, torch.float16, "sigmoid", 2.0, [0, 7]),
    ("D128-bf16", 8, 4100, 128, 512, torch.bfloat16, "silu", 1.0, [0, 7]),
    ("D128-leaky", 16, 2049, 128, 1024, torch.bfloat16, "leaky_relu", 1.0, [3]),
]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _normrel(a, b):
    a = a.double()
    b = b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def plan(H, B, D, E, code, act):
    info = (ctypes.c_int64 * 10)()
    _lib.check(_lib.lib().fmlp_bwd_plan(H, B, D, E, code, _lib.ACT_CODES[act], info, 10), "backward plan")
    keys = ("dz", "nS", "dx_es", "dxs_xs", "dx_first", "n_dw", "n_dx", "n_dxs", "ws_bytes", "act")
    return dict(zip(keys, list(info)))


def _bwd(x, w1, w2, do, act, code, out_dtype, fill_nan=False):
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    dev = x.device
    dx = torch.empty(H, B, D, dtype=out_dtype, device=dev)
    dw1 = torch.empty(H, D, E, dtype=out_dtype, device=dev)
    dw2 = torch.empty(H, E, D, dtype=out_dtype, device=dev)
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=dev)
    if fill_nan:
        dx.fill_(float("nan"))
        ws.view(torch.float32)[: ws.numel() // 4].fill_(float("nan"))
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(L.fmlp_bwd(_ptr(x), _ptr(w1), _ptr(w2), _ptr(do), _ptr(dx), _ptr(dw1), _ptr(dw2), H, B, D, E, code,
                          _lib.ACT_CODES[act], _ptr(ws), n, stream), "backward")
    torch.cuda.synchronize()
    return dx, dw1, dw2


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_ragged_dx_split(case):
    name, H, B, D, E, dt, act, x_std, hs = case
    code = _DT[dt]
    p = plan(H, B, D, E, code, act)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    _say(f"[bwd-ragged] {name}: H={H} B={B} D={D} E={E} {dt} act='{act}' cus={cus} plan={p}")
    if cus == 256:
        assert p["dxs_xs"] >= 2 and p["n_dxs"] == H * p["dxs_xs"], p
    x, w1, w2, do = make_inputs(H, B, D, E, dt, x_std, seed=5)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    sel = lambda t: t[hs].cpu()

    # fp32 sums against the emulation
    sdx, sdw1, sdw2 = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32, fill_nan=True)
    assert torch.isfinite(sdx).all()
    edx, edw1, edw2 = emulate.emu_bwd(sel(x), sel(w1), sel(w2), sel(do), act, dt, round_out=False)
    rel = {k: _normrel(sel(g), e) for k, g, e in (("dx", sdx, edx), ("dw1", sdw1, edw1), ("dw2", sdw2, edw2))}
    _say(f"[bwd-ragged] {name}: fp32 sums rel " + " ".join(f"{k}={v:.3g}" for k, v in rel.items()))
    assert max(rel.values()) <= 1e-4, rel

    # io dX against the fp32 oracle, every element written
    dx, dw1, dw2 = _bwd(xd, w1d, w2d, dod, act, code, dt, fill_nan=True)
    assert torch.isfinite(dx.float()).all()
    _, rdx, _, _ = reference.autograd_grads(sel(x), sel(w1), sel(w2), sel(do), act)
    bad = ((sel(dx).float() - rdx).abs() > 3e-2 + 3e-2 * rdx.abs()).float().mean().item()
    _say(f"[bwd-ragged] {name}: dx outside 3e-2: {bad:.3g}")
    assert bad == 0.0

    # fixed order; dX independent of the dW mode
    dx2, dw12, dw22 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    assert torch.equal(dx.view(torch.int16), dx2.view(torch.int16))
    assert torch.equal(dw1.view(torch.int16), dw12.view(torch.int16))
    assert torch.equal(dw2.view(torch.int16), dw22.view(torch.int16))
    dxh, _, _ = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_DW_HILO, dt)
    assert torch.equal(dx.view(torch.int16), dxh.view(torch.int16))
