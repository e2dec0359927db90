"""The backward's dW programs at D = 256 (dw256_kernel: four waves of 32 E-columns each, one per
SIMD, with the wave's W1 / W2 operands held in registers; B split over programs with fp32
partials summed by a second launch as far as the workspace holds them), for dense 16-bit
tensors with E % 8 == 0. The reference's dW programs are flashmlp.py:247-329.

Each case checks, through the C ABI:
  * the fp32 sums (FMLP_OUT_F32) of dX, dW1, dW2 against the oracle's cast-point emulation at
    the north star's 1e-4, and against the generic kernels' sums for the same values passed as
    non-dense views within 1e-5 (summation order only);
  * the io dW against the emulation and dX against the fp32 autograd oracle at the parity bar
    (3e-2 + 3e-2 |ref|), every element written (outputs NaN-filled first);
  * where B splits: the split (the queried workspace) against no workspace (one program per
    E-tile) within the summation-order difference, two calls bitwise equal, and
    fmlp_bwd_noalloc bitwise equal to fmlp_bwd;
  * the accuracy mode (FMLP_DW_HILO) against the fp32 autograd oracle: every dW element within
    the parity bar, and dX bitwise equal to the default mode's.
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
D = 256


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _normrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _bad(a, b):
    a, b = a.float(), b.float()
    return ((a - b).abs() > 3e-2 + 3e-2 * b.abs()).sum().item()


def _plan(H, B, E, code, act):
    info = (ctypes.c_int64 * 11)()
    _lib.check(_lib.lib().fmlp_bwd_plan(H, B, D, E, code, _lib.ACT_CODES[act], info, 11), "backward plan")
    keys = ("dz", "nS", "dx_es", "dxs_xs", "dx_first", "n_dw", "n_dx", "n_dxs", "ws_bytes", "act", "et_w")
    return dict(zip(keys, list(info)))


def _bwd(x, w1, w2, do, act, code, out_dtype, ws_bytes=None, strided=False, noalloc=False):
    """fmlp_bwd (or fmlp_bwd_strided / fmlp_bwd_noalloc) with NaN-filled outputs; ws_bytes None:
    the queried workspace, 0: none."""
    L = _lib.lib()
    H, B, _ = x.shape
    E = w1.shape[2]
    dev = x.device
    dx = torch.full((H, B, D), float("nan"), dtype=out_dtype, device=dev)
    dw1 = torch.full((H, D, E), float("nan"), dtype=out_dtype, device=dev)
    dw2 = torch.full((H, E, D), float("nan"), dtype=out_dtype, device=dev)
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code) if ws_bytes is None else ws_bytes
    ws = torch.empty(n, dtype=torch.uint8, device=dev) if n else None
    if ws is not None:  # stale partials would show
        ws.view(torch.float32)[: n // 4].fill_(float("nan"))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a = _lib.ACT_CODES[act]
    if noalloc:
        st = L.fmlp_bwd_noalloc(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, code, a, stream)
    elif strided:
        st = L.fmlp_bwd_strided(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, _lib.strides(x),
                                _lib.strides(w1), _lib.strides(w2), _lib.strides(do), code, a, _p(ws), n, stream)
    else:
        st = L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, code, a, _p(ws), n,
                        stream)
    _lib.check(st, "backward")
    torch.cuda.synchronize()
    return dx, dw1, dw2


def _padded(t):
    """The same values in a buffer with padded rows: a non-dense view (the generic kernels)."""
    pad = torch.zeros(*t.shape[:-1], t.shape[-1] + 8, dtype=t.dtype, device=t.device)
    pad[..., : t.shape[-1]] = t
    v = pad[..., : t.shape[-1]]
    assert not v.is_contiguous()
    return v


def _check(H, B, E, dt, act, seed):
    code = _DT[dt]
    p = _plan(H, B, E, code, act)
    _say(f"[dw256] H={H} B={B} D={D} E={E} {dt} act='{act}' seed={seed} plan={p}")
    x, w1, w2, do = make_inputs(H, B, D, E, dt, 1.0, seed=seed)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))

    s = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32)
    sg = _bwd(_padded(xd), w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32, strided=True)
    e = emulate.emu_bwd(x, w1, w2, do, act, dt, round_out=False)
    rel = {k: _normrel(g.cpu(), r) for k, g, r in zip(("dx", "dw1", "dw2"), s, e)}
    rel_g = {k: _normrel(a_, b_) for k, a_, b_ in zip(("dx", "dw1", "dw2"), s, sg)}
    _say(f"[dw256] fp32 sums rel to emulation {rel}, to the generic kernels {rel_g}")
    assert all(torch.isfinite(t).all() for t in s)
    assert max(rel.values()) <= 1e-4 and max(rel_g.values()) <= 1e-5, (rel, rel_g)

    dx, dw1, dw2 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    _, rdx, _, _ = reference.autograd_grads(x, w1, w2, do, act)
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
    bad = {"dx": _bad(dx.cpu(), rdx), "dw1": _bad(dw1.cpu(), edw1), "dw2": _bad(dw2.cpu(), edw2)}
    _say(f"[dw256] io outside 3e-2: {bad}")
    assert all(torch.isfinite(t.float()).all() for t in (dx, dw1, dw2))
    assert sum(bad.values()) == 0, bad
    return p, (xd, w1d, w2d, dod), (dx, dw1, dw2)


CASES = [(dt, act) for dt in (torch.float16, torch.bfloat16) for act in ("silu", "leaky_relu", "sigmoid", "")]


@pytest.mark.parametrize("dt,act", CASES, ids=[f"{str(d).split('.')[-1]}-{a or 'linear'}" for d, a in CASES])
def test_dw256_tails(dt, act):
    # B tail (300 = 9 x 32 + 12) and an E-tile with 8 of its 128 columns (136 = 128 + 8)
    _check(2, 300, 136, dt, act, seed=61)


SPLIT = [("ragged-ranges", 2, 2100, 264, torch.bfloat16, "silu"),
         ("d256-heads", 2, 4096, 1024, torch.float16, "sigmoid")]


@pytest.mark.parametrize("case", SPLIT, ids=[c[0] for c in SPLIT])
def test_dw256_b_split(case):
    name, H, B, E, dt, act = case
    code = _DT[dt]
    p, (xd, w1d, w2d, dod), (dx, dw1, dw2) = _check(H, B, E, dt, act, seed=62)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert p["nS"] > 1 and p["ws_bytes"] > 0, p
    # two calls: bitwise equal (a fixed summation order; the NaN-filled workspace is rewritten)
    dx2, dw12, dw22 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    for a_, b_ in ((dx, dx2), (dw1, dw12), (dw2, dw22)):
        assert torch.equal(a_.view(torch.int16), b_.view(torch.int16))
    # no workspace: one program per E-tile, the same sums up to the order
    s = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32)
    s0 = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_OUT_F32, torch.float32, ws_bytes=0)
    assert torch.equal(s[0], s0[0])  # dX does not depend on the split
    r0 = [_normrel(a_, b_) for a_, b_ in zip(s[1:], s0[1:])]
    _say(f"[dw256] {name}: split vs unsplit dW rel {r0}")
    assert max(r0) <= 1e-5
    # the no-allocation entry point: the same plan (the partials fit its scratch), bitwise
    if p["ws_bytes"] <= 64 << 20:
        na = _bwd(xd, w1d, w2d, dod, act, code, dt, noalloc=True)
        for a_, b_ in zip((dx, dw1, dw2), na):
            assert torch.equal(a_.view(torch.int16), b_.view(torch.int16))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["float16", "bfloat16"])
def test_dw256_accurate_mode(dt):
    H, B, E, act = 2, 2100, 264, "silu"
    code = _DT[dt]
    x, w1, w2, do = make_inputs(H, B, D, E, dt, 1.0, seed=63)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    dx, dw1, dw2 = _bwd(xd, w1d, w2d, dod, act, code | _lib.FMLP_DW_HILO, dt)
    dx0, dw10, dw20 = _bwd(xd, w1d, w2d, dod, act, code, dt)
    assert torch.equal(dx.view(torch.int16), dx0.view(torch.int16)), "dX must not depend on the dW mode"
    _, _, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    res = {"dw1_bad": _bad(dw1.cpu(), rdw1), "dw2_bad": _bad(dw2.cpu(), rdw2),
           "dw1_rel": _normrel(dw1.cpu(), rdw1), "dw2_rel": _normrel(dw2.cpu(), rdw2),
           "dw1_rel_default": _normrel(dw10.cpu(), rdw1), "dw2_rel_default": _normrel(dw20.cpu(), rdw2)}
    _say(f"[dw256] accurate mode {dt}: {res}")
    bound = 5e-3 if dt == torch.bfloat16 else 1e-3
    assert res["dw1_bad"] == 0 and res["dw2_bad"] == 0, res
    assert res["dw1_rel"] <= bound and res["dw2_rel"] <= bound, res
    assert res["dw1_rel"] <= res["dw1_rel_default"] and res["dw2_rel"] <= res["dw2_rel_default"], res


def test_dw256_few_rows():
    # one row, and no rows (dW must be exactly zero, dX has no elements)
    _check(3, 1, 256, torch.bfloat16, "silu", seed=64)
    H, E = 2, 128
    x = torch.empty(H, 0, D, dtype=torch.float16, device="cuda")
    w1 = torch.randn(H, D, E, device="cuda").half()
    w2 = torch.randn(H, E, D, device="cuda").half()
    do = torch.empty(H, 0, D, dtype=torch.float16, device="cuda")
    _, dw1, dw2 = _bwd(x, w1, w2, do, "silu", _DT[torch.float16], torch.float16)
    assert torch.count_nonzero(dw1.float().nan_to_num(1.0)) == 0
    assert torch.count_nonzero(dw2.float().nan_to_num(1.0)) == 0


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_d256_views_take_the_d256_programs(dt):
    """Through the Python API, views at D = 256 (X transposed from a (B, H, D) tensor, and the
    stride-0 dO that `model(x).sum().backward()` hands to the backward) are copied to dense
    tensors, as the reference's reshape / contiguous does (flashmlp.py:453-459,508), and run on
    the D = 256 programs: outputs bitwise equal to the same values passed densely (the generic
    kernels, which read views in place, sum in another order)."""
    import flashmlp_amd as fm

    H, B, E, act = 3, 1000, 264, "silu"
    x, w1, w2, _ = make_inputs(H, B, D, E, dt, 1.0, seed=65)
    xd, w1d, w2d = (t.cuda() for t in (x, w1, w2))
    xv = xd.transpose(0, 1).contiguous().transpose(0, 1)  # same values, strides (D, H D, 1)
    assert not xv.is_contiguous()
    one = torch.ones((), dtype=dt, device="cuda")
    dov, dod = one.expand(H, B, D), one.expand(H, B, D).contiguous()
    _say(f"[dw256] views through the Python API: H={H} B={B} E={E} {dt}")
    o_v, o_d = fm.flashmlp_fwd(xv, w1d, w2d, act), fm.flashmlp_fwd(xd, w1d, w2d, act)
    g_v, g_d = fm.flashmlp_bwd(xv, w1d, w2d, dov, act), fm.flashmlp_bwd(xd, w1d, w2d, dod, act)
    torch.cuda.synchronize()
    for name, a, b in zip(("o", "dx", "dw1", "dw2"), (o_v, *g_v), (o_d, *g_d)):
        assert torch.isfinite(b).all(), name
        assert torch.equal(a, b), f"{name}: the view's result differs from the dense call's"
