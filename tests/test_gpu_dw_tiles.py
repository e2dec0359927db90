"""The backward's 64-column dW programs (D = 64, with the dX programs' E split): twice the dW
programs of the 128-column form, each over half the E-columns, with four row sets of waves
whose partial sums are added through LDS. The plan takes them for grids that leave CUs idle;
fmlp_bwd_plan reports the width (its 11th value).

Each case (shapes where the plan takes 64 columns on a 256-CU MI355X) checks through the C ABI
the fp32 sums (FMLP_OUT_F32) of dX, dW1, dW2 against the oracle's cast-point emulation at the
north star's 1e-4, the io outputs against the fp32 autograd oracle (dX) and the emulation (dW)
at the parity bar (3e-2 + 3e-2 |ref|), bitwise equal repeats, and the dW-only backward
(FMLP_BWD_NO_DX, the same plan) bitwise equal to the full one's dW.
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
    ("cfg2", 12, 1024, 64, 768, torch.float16, "silu"),
    ("bf16-small", 8, 512, 64, 512, torch.bfloat16, "silu"),
    ("leaky-B-tail", 4, 1000, 64, 512, torch.float16, "leaky_relu"),
    ("sigmoid-E-tail", 6, 700, 64, 328, torch.bfloat16, "sigmoid"),
]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _normrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _bad(a, b):
    a, b = a.float(), b.float()
    return ((a - b).abs() > 3e-2 + 3e-2 * b.abs()).sum().item()


def _plan(H, B, D, E, code, act):
    info = (ctypes.c_int64 * 11)()
    _lib.check(_lib.lib().fmlp_bwd_plan(H, B, D, E, code, _lib.ACT_CODES[act], info, 11), "backward plan")
    return list(info)


def _bwd(x, w1, w2, do, act, code, out_dtype, want_dx=True):
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    if not want_dx:
        code |= _lib.FMLP_BWD_NO_DX
    dx = torch.full((H, B, D), float("nan"), dtype=out_dtype, device=x.device) if want_dx else None
    dw1 = torch.full((H, D, E), float("nan"), dtype=out_dtype, device=x.device)
    dw2 = torch.full((H, E, D), float("nan"), dtype=out_dtype, device=x.device)
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.fmlp_bwd(_ptr(x), _ptr(w1), _ptr(w2), _ptr(do), _ptr(dx), _ptr(dw1), _ptr(dw2), H, B, D, E, code,
                          _lib.ACT_CODES[act], _ptr(ws), n, stream), "backward")
    torch.cuda.synchronize()
    return dx, dw1, dw2


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_64_column_dw_programs(case):
    name, H, B, D, E, dt, act = case
    code = _DT[dt]
    p = _plan(H, B, D, E, code, act)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    _say(f"[dw-tiles] {name}: H={H} B={B} D={D} E={E} {dt} act='{act}' cus={cus} plan={p}")
    if cus == 256:
        assert p[10] == 64 and p[0] == 0 and p[2] == 2, p
    x, w1, w2, do = make_inputs(H, B, D, E, dt, 1.0, seed=9)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))

    s = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32)
    e = emulate.emu_bwd(x, w1, w2, do, act, dt, round_out=False)
    rel = {k: _normrel(g.cpu(), r) for k, g, r in zip(("dx", "dw1", "dw2"), s, e)}
    _say(f"[dw-tiles] {name}: fp32 sums rel " + " ".join(f"{k}={v:.3g}" for k, v in rel.items()))
    assert max(rel.values()) <= 1e-4, rel

    dx, dw1, dw2 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    _, rdx, _, _ = reference.autograd_grads(x, w1, w2, do, act)
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
    bad = {"dx": _bad(dx.cpu(), rdx), "dw1": _bad(dw1.cpu(), edw1), "dw2": _bad(dw2.cpu(), edw2)}
    _say(f"[dw-tiles] {name}: outside 3e-2: {bad}")
    assert sum(bad.values()) == 0, bad

    dx2, dw12, dw22 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    assert torch.equal(dx.view(torch.int16), dx2.view(torch.int16))
    assert torch.equal(dw1.view(torch.int16), dw12.view(torch.int16))
    assert torch.equal(dw2.view(torch.int16), dw22.view(torch.int16))
    _, dw13, dw23 = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_BWD_RECOMPUTE, dt, want_dx=False)
    assert torch.equal(dw1.view(torch.int16), dw13.view(torch.int16))
    assert torch.equal(dw2.view(torch.int16), dw23.view(torch.int16))
