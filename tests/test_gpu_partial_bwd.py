"""Partial backward (FMLP_BWD_NO_DX / FMLP_BWD_NO_DW) through every backward entry point of
the C ABI: fmlp_bwd, fmlp_bwd_strided (dense strides: tuned kernels; a strided view: generic
kernels) and fmlp_bwd_noalloc.

For each entry point and flag:
  * the unwanted outputs are passed filled with a sentinel byte pattern and must come back
    unchanged (the header promises they are not written);
  * the wanted outputs are passed filled with NaN bytes and must come back NaN-free and
    bit-identical to the same entry point's full backward: dw1, dw2 of FMLP_BWD_NO_DX to those
    of the same call without it (the dW programs of that call's plan, whichever form it takes;
    with FMLP_BWD_RECOMPUTE as well, to the recompute form's), dx of FMLP_BWD_NO_DW to the
    recompute form's (FMLP_BWD_RECOMPUTE), whose dX programs it runs; two shapes whose plan
    stores dZ with dW programs of another B split or width than the recompute form's make the
    difference between the forms observable;
  * with FMLP_BWD_NO_DW the workspace is at most the split ragged dX tiles' partials (the dX
    programs run as in the recompute form's launch, split parts and their sum included): none,
    and a NULL workspace is accepted, on a shape whose dW programs split B but whose dX tiles
    are whole (where the full backward does need one).
No counterpart in the reference, whose backward always computes all three gradients.
"""
import ctypes
import sys

import pytest
import torch

from flashmlp_amd import _lib
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu

_DT = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16}
SENTINEL = 0x5A  # 0x5A5A: a finite fp16 / bf16 value no gradient here takes


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _filled(shape, dtype, byte):
    t = torch.empty(shape, dtype=dtype, device="cuda")
    t.view(torch.uint8).fill_(byte)
    return t


def _strides(t):
    return (ctypes.c_int64 * 3)(*t.stride())


def _call(entry, x, w1, w2, do, act, flags, outs, ws=None, ws_bytes=0):
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    code = _DT[x.dtype] | flags
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dx, dw1, dw2 = outs
    if entry == "fmlp_bwd":
        st = L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, code,
                        _lib.ACT_CODES[act], _p(ws), ws_bytes, stream)
    elif entry == "fmlp_bwd_strided":
        st = L.fmlp_bwd_strided(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E,
                                _strides(x), _strides(w1), _strides(w2), _strides(do), code,
                                _lib.ACT_CODES[act], _p(ws), ws_bytes, stream)
    else:
        st = L.fmlp_bwd_noalloc(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, code,
                                _lib.ACT_CODES[act], stream)
    _lib.check(st, f"{entry} flags={flags:#x}")
    torch.cuda.synchronize()


def _workspace(entry, x, w1, flags):
    """(tensor or None, bytes) the entry point needs for these flags (none for no-alloc)."""
    if entry == "fmlp_bwd_noalloc":
        return None, 0
    H, B, D = x.shape
    E = w1.shape[2]
    n = _lib.lib().fmlp_bwd_workspace_bytes(H, B, D, E, _DT[x.dtype] | flags)
    return (torch.empty(n, dtype=torch.uint8, device="cuda") if n else None), n


CASES = [
    # H, B, D, E, dtype, act, seed, x transposed (a strided view: generic kernels)
    (2, 4096, 128, 512, torch.bfloat16, "silu", 71, False),      # tuned kernels, B split
    (8, 4097, 64, 2048, torch.float16, "sigmoid", 72, False),    # tuned kernels, tails
    (3, 300, 32, 45, torch.float16, "leaky_relu", 73, False),    # generic kernels (D = 32)
    (2, 260, 64, 136, torch.bfloat16, "silu", 74, True),         # generic kernels (strided X)
    (1, 4096, 128, 1024, torch.bfloat16, "silu", 75, False),     # stored dZ, another B split
    (1, 4096, 64, 2048, torch.float16, "sigmoid", 76, False),    # stored dZ, 128- vs 64-column dW
]
STORED = {(1, 4096, 128, 1024), (1, 4096, 64, 2048)}
ENTRIES = ["fmlp_bwd", "fmlp_bwd_strided", "fmlp_bwd_noalloc"]


@pytest.mark.parametrize("entry", ENTRIES)
@pytest.mark.parametrize("H,B,D,E,dt,act,seed,xt", CASES,
                         ids=["bf16-D128-split", "fp16-D64-tail", "fp16-D32-generic", "bf16-D64-stridedX",
                              "bf16-D128-stored-dz", "fp16-D64-stored-dz"])
def test_partial_backward_writes_only_what_is_asked(entry, H, B, D, E, dt, act, seed, xt):
    if xt and entry != "fmlp_bwd_strided":
        pytest.skip("a strided view goes through fmlp_bwd_strided only")
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=seed))
    if xt:  # same values, X stored as (H, D, B) and viewed as (H, B, D)
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    _say(f"[partial] {entry} H={H} B={B} D={D} E={E} {dt} act='{act}' strided_x={xt}")
    if (H, B, D, E) in STORED and entry == "fmlp_bwd":
        L, code = _lib.lib(), _DT[dt]
        p_own, p_rec = (ctypes.c_int64 * 11)(), (ctypes.c_int64 * 11)()
        _lib.check(L.fmlp_bwd_plan(H, B, D, E, code, _lib.ACT_CODES[act], p_own, 11), "plan")
        _lib.check(L.fmlp_bwd_plan(H, B, D, E, code | _lib.FMLP_BWD_RECOMPUTE, _lib.ACT_CODES[act], p_rec, 11),
                   "plan")
        # the plan stores dZ, with dW programs of another B split or E-tile width than the recompute form's
        assert p_own[0] == 1 and (p_own[1], p_own[10]) != (p_rec[1], p_rec[10]), (list(p_own), list(p_rec))
    full = {}
    for form in (_lib.FMLP_BWD_RECOMPUTE, 0):
        ws, n = _workspace(entry, x, w1, form)
        full[form] = tuple(_filled(s, dt, 0xFF) for s in ((H, B, D), (H, D, E), (H, E, D)))
        _call(entry, x, w1, w2, do, act, form, full[form], ws, n)
        for name, t in zip(("dx", "dw1", "dw2"), full[form]):
            assert not torch.isnan(t).any(), f"full backward (flags {form:#x}) left {name} elements unwritten"

    # dW only: dx is a sentinel-filled buffer that must stay untouched; dw1, dw2 are those of
    # the full call with the same other flags
    for form in (0, _lib.FMLP_BWD_RECOMPUTE):
        flags = _lib.FMLP_BWD_NO_DX | form
        # a strided view of a tuned shape runs on the generic kernels, which split B as far as the
        # workspace holds, while the query sizes the tuned plan's: give them the full call's
        ws, n = _workspace(entry, x, w1, form if xt else flags)
        dx_s = _filled((H, B, D), dt, SENTINEL)
        dw1, dw2 = _filled((H, D, E), dt, 0xFF), _filled((H, E, D), dt, 0xFF)
        _call(entry, x, w1, w2, do, act, flags, (dx_s, dw1, dw2), ws, n)
        assert bool((dx_s.view(torch.uint8) == SENTINEL).all()), "FMLP_BWD_NO_DX wrote dx"
        assert torch.equal(dw1, full[form][1]) and torch.equal(dw2, full[form][2]), f"flags {flags:#x}"
    own, full = full[0], full[_lib.FMLP_BWD_RECOMPUTE]

    # dX only: dw1, dw2 are sentinel-filled and must stay untouched; the workspace holds at most
    # the split ragged tiles' partials
    ws, n = _workspace(entry, x, w1, _lib.FMLP_BWD_NO_DW)
    if entry != "fmlp_bwd_noalloc":
        full_n = _lib.lib().fmlp_bwd_workspace_bytes(H, B, D, E, _DT[dt] | _lib.FMLP_BWD_RECOMPUTE)
        assert n <= full_n, (n, full_n)
    dx = _filled((H, B, D), dt, 0xFF)
    dw1_s, dw2_s = _filled((H, D, E), dt, SENTINEL), _filled((H, E, D), dt, SENTINEL)
    _call(entry, x, w1, w2, do, act, _lib.FMLP_BWD_NO_DW, (dx, dw1_s, dw2_s), ws, n)
    assert bool((dw1_s.view(torch.uint8) == SENTINEL).all()), "FMLP_BWD_NO_DW wrote dw1"
    assert bool((dw2_s.view(torch.uint8) == SENTINEL).all()), "FMLP_BWD_NO_DW wrote dw2"
    assert torch.equal(dx, full[0])

    # NULL for the outputs nobody asked for
    dw1, dw2 = _filled((H, D, E), dt, 0xFF), _filled((H, E, D), dt, 0xFF)
    ws, n = _workspace(entry, x, w1, 0 if xt else _lib.FMLP_BWD_NO_DX)
    _call(entry, x, w1, w2, do, act, _lib.FMLP_BWD_NO_DX, (None, dw1, dw2), ws, n)
    assert torch.equal(dw1, own[1]) and torch.equal(dw2, own[2])
    dx = _filled((H, B, D), dt, 0xFF)
    ws, n = _workspace(entry, x, w1, _lib.FMLP_BWD_NO_DW)
    _call(entry, x, w1, w2, do, act, _lib.FMLP_BWD_NO_DW, (dx, None, None), ws, n)
    assert torch.equal(dx, full[0])


def test_no_dw_needs_no_workspace_where_the_full_backward_does():
    H, B, D, E, dt = 2, 4096, 128, 512, torch.bfloat16
    code = _DT[dt] | _lib.FMLP_BWD_RECOMPUTE
    need = _lib.lib().fmlp_bwd_workspace_bytes(H, B, D, E, code)
    _say(f"[partial] workspace full={need} no_dw={_lib.lib().fmlp_bwd_workspace_bytes(H, B, D, E, code | _lib.FMLP_BWD_NO_DW)}")
    assert need > 0, "this shape should split B in the recompute form"
    assert _lib.lib().fmlp_bwd_workspace_bytes(H, B, D, E, code | _lib.FMLP_BWD_NO_DW) == 0
    # the full backward refuses a NULL workspace here; the dX-only one takes it
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=75))
    outs = tuple(torch.empty(s, dtype=dt, device="cuda") for s in ((H, B, D), (H, D, E), (H, E, D)))
    L = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), *(_p(t) for t in outs), H, B, D, E, code,
                    _lib.ACT_CODES["silu"], None, 0, stream)
    assert st == 4, "the full backward must report FMLP_ERR_WORKSPACE without its workspace"
    st = L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), _p(outs[0]), None, None, H, B, D, E,
                    code | _lib.FMLP_BWD_NO_DW, _lib.ACT_CODES["silu"], None, 0, stream)
    assert st == 0, _lib.lib().fmlp_last_error().decode()
    torch.cuda.synchronize()
    assert not torch.isnan(outs[0]).any()
