"""Both forms of the backward against the oracle, through the C ABI.

The library's backward has two forms (fmlp_bwd in include/flashmlp.h): the reference's
recompute-only one (flashmlp.py:341-421: dX programs recompute Z and dH) and a stored-dZ
one, whose dW programs also store dZ, in the io dtype, to the workspace and whose dX is a
GEMM over it (dxg_kernel). The plan picks one per shape; FMLP_BWD_RECOMPUTE and
FMLP_BWD_STORE_DZ force each, so every case here runs both on the same inputs.

Bars, as in test_gpu_parity.py: dX elementwise |gpu - ref| <= 3e-2 + 3e-2 |ref| against the
fp32 autograd oracle; dW1, dW2 the same against the cast-point emulation (oracle.emulate) and
normwise <= 1e-2 against fp32; with FMLP_OUT_F32 the fp32 sums within 1e-4 normwise of the
emulation's unrounded sums (test_gpu_fp32_sums.py); with FMLP_DW_HILO zero elementwise misses
of dW against fp32 (test_gpu_accurate_dw.py).

Shapes cover B and E tails (partial 32-row subtiles and 256-row dX tiles, E % 32 != 0), one
B split of the dW programs (fp32 partials before dZ in the workspace), D 64 and 128, fp16 and
bf16, every activation.
"""
import ctypes
import sys

import pytest
import torch

from flashmlp_amd import _lib
from oracle import emulate, reference
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu

ATOL = RTOL = 3e-2
_DT = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16}
FORMS = {"recompute": _lib.FMLP_BWD_RECOMPUTE, "stored_dz": _lib.FMLP_BWD_STORE_DZ}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _fail_frac(a, b):
    a, b = a.float(), b.float()
    return ((a - b).abs() > ATOL + RTOL * b.abs()).float().mean().item()


def _normrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def bwd_abi(x, w1, w2, do, act, flags):
    """fmlp_bwd with the io dtype code OR `flags`; fp32 outputs when FMLP_OUT_F32 is set."""
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    code = _DT[x.dtype] | flags
    odt = torch.float32 if flags & _lib.FMLP_OUT_F32 else x.dtype
    dx = torch.empty(H, B, D, dtype=odt, device=x.device)
    dw1 = torch.empty(H, D, E, dtype=odt, device=x.device)
    dw2 = torch.empty(H, E, D, dtype=odt, device=x.device)
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, code,
                          _lib.ACT_CODES[act], _p(ws), n, stream), "backward")
    torch.cuda.synchronize()
    return dx, dw1, dw2, n


CASES = [
    # H, B, D, E, dtype, act, seed
    (3, 300, 64, 264, torch.float16, "silu", 31),
    (2, 33, 128, 136, torch.bfloat16, "sigmoid", 32),
    (4, 4097, 64, 520, torch.bfloat16, "leaky_relu", 33),
    (2, 1, 128, 8, torch.float16, "", 34),
    (5, 700, 128, 40, torch.bfloat16, "silu", 35),
    (2, 8192, 128, 256, torch.bfloat16, "silu", 36),  # 4 dW programs: B split, partials + dZ
    (3, 2100, 64, 1000, torch.float16, "sigmoid", 37),
]


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("H,B,D,E,dt,act,seed", CASES)
def test_form_parity(H, B, D, E, dt, act, seed, form):
    x, w1, w2, do = make_inputs(H, B, D, E, dt, seed=seed)
    _say(f"[forms] {form}: H={H} B={B} D={D} E={E} {dt} act='{act}' seed={seed}")
    dx, dw1, dw2, n = bwd_abi(*(t.cuda() for t in (x, w1, w2, do)), act, FORMS[form])
    _, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
    res = {
        "ws": n,
        "dx_fail": _fail_frac(dx.cpu(), rdx),
        "dw1_emu_fail": _fail_frac(dw1.cpu(), edw1),
        "dw2_emu_fail": _fail_frac(dw2.cpu(), edw2),
        "dw1_rel": _normrel(dw1.cpu(), rdw1),
        "dw2_rel": _normrel(dw2.cpu(), rdw2),
    }
    _say(f"[forms] {form}: " + " ".join(f"{k}={v:.3g}" for k, v in res.items()))
    for t in (dx, dw1, dw2):
        assert torch.isfinite(t.float()).all()
    assert res["dx_fail"] == 0.0, res
    assert res["dw1_emu_fail"] == 0.0 and res["dw2_emu_fail"] == 0.0, res
    assert res["dw1_rel"] <= 1e-2 and res["dw2_rel"] <= 1e-2, res
    if form == "stored_dz":  # dZ itself is in the workspace
        assert n >= H * -(-E // 128) * 128 * -(-B // 256) * 256 * 2


@pytest.mark.parametrize("H,B,D,E,dt,act,seed", [CASES[0], CASES[2], CASES[5]])
def test_stored_dz_fp32_sums(H, B, D, E, dt, act, seed):
    x, w1, w2, do = make_inputs(H, B, D, E, dt, seed=seed)
    _say(f"[forms] stored_dz fp32 sums: H={H} B={B} D={D} E={E} {dt} act='{act}'")
    dx, dw1, dw2, _ = bwd_abi(*(t.cuda() for t in (x, w1, w2, do)), act,
                              _lib.FMLP_BWD_STORE_DZ | _lib.FMLP_OUT_F32)
    edx, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt, round_out=False)
    rel = {k: _normrel(g.cpu(), e) for k, g, e in (("dx", dx, edx), ("dw1", dw1, edw1), ("dw2", dw2, edw2))}
    _say(f"[forms] stored_dz fp32 sums: " + " ".join(f"{k}={v:.3g}" for k, v in rel.items()))
    assert all(v <= 1e-4 for v in rel.values()), rel


def test_stored_dz_accuracy_mode():
    H, B, D, E, dt, act, seed = 2, 8192, 128, 256, torch.bfloat16, "silu", 38
    x, w1, w2, do = make_inputs(H, B, D, E, dt, seed=seed)
    _say(f"[forms] stored_dz + hi/lo dW: H={H} B={B} D={D} E={E} {dt} act='{act}'")
    dx, dw1, dw2, _ = bwd_abi(*(t.cuda() for t in (x, w1, w2, do)), act,
                              _lib.FMLP_BWD_STORE_DZ | _lib.FMLP_DW_HILO)
    _, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    miss = {"dx": _fail_frac(dx.cpu(), rdx), "dw1": _fail_frac(dw1.cpu(), rdw1), "dw2": _fail_frac(dw2.cpu(), rdw2)}
    _say(f"[forms] stored_dz + hi/lo dW misses vs fp32: {miss}")
    assert all(v == 0.0 for v in miss.values()), miss


def test_workspace_sizes_by_form():
    L = _lib.lib()
    for H, B, D, E in ((32, 16384, 128, 1024), (8, 4097, 64, 2048), (3, 300, 64, 264)):
        code = _lib.FMLP_DTYPE_BF16
        lean = L.fmlp_bwd_workspace_bytes(H, B, D, E, code | _lib.FMLP_BWD_RECOMPUTE)
        auto = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
        dz = L.fmlp_bwd_workspace_bytes(H, B, D, E, code | _lib.FMLP_BWD_STORE_DZ)
        need_dz = H * -(-E // 128) * 128 * -(-B // 256) * 256 * 2
        _say(f"[forms] workspace H={H} B={B} D={D} E={E}: recompute {lean}, auto {auto}, stored-dZ {dz}")
        assert lean < need_dz <= dz
        assert lean <= auto <= max(lean, dz)
