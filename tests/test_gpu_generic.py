"""Parity of the generic kernels (fmlp_gen.hip): the shapes, dtypes and layouts the tuned
kernels do not take, against the CPU oracle.

  * D in {16, 32, 256} (the reference's D is any power of two >= 16, flashmlp.py:66,186),
    E not a multiple of 8, and B tails, at fp16 / bf16 with the bars of test_gpu_parity
    (O and dX elementwise 3e-2 against the fp32 autograd oracle, dW elementwise 3e-2 against
    the cast-point emulation and normwise 1e-2 against fp32);
  * fp32 io (the reference's io dtype is x's, flashmlp.py:87): every output is an fp32 sum,
    held to the north star's 1e-4 relative (normwise) against the fp32 oracle;
  * strided inputs read in place (sliced, transposed and stride-0 views): bit-identical to the
    same values passed densely;
  * the fp32-output flag and the hi/lo dW mode on the generic path.
"""
import ctypes
import sys

import pytest
import torch

import flashmlp_amd as fm
from flashmlp_amd import _lib
from oracle import emulate, reference
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu

ATOL = RTOL = 3e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fail_frac(a, b):
    a, b = a.float(), b.float()
    return ((a - b).abs() > ATOL + RTOL * b.abs()).float().mean().item()


def _normrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _run(H, B, D, E, dtype, act, seed=0, x_std=1.0):
    x, w1, w2, do = make_inputs(H, B, D, E, dtype, x_std, seed)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    o = fm.flashmlp_fwd(xd, w1d, w2d, act)
    dx, dw1, dw2 = fm.flashmlp_bwd(xd, w1d, w2d, dod, act)
    torch.cuda.synchronize()
    return (x, w1, w2, do), (o.cpu(), dx.cpu(), dw1.cpu(), dw2.cpu())


CASES16 = [(D, dt, act) for D in (16, 32, 256) for dt in (torch.float16, torch.bfloat16)
           for act in ("silu", "leaky_relu", "sigmoid", "")]


@pytest.mark.parametrize("D,dt,act", CASES16, ids=[f"D{D}-{str(d).split('.')[-1]}-{a or 'linear'}" for D, d, a in CASES16])
def test_generic_16bit(D, dt, act):
    H, B, E = 2, 77, 45  # B and E tails (E % 8 != 0)
    _say(f"[generic] H={H} B={B} D={D} E={E} {dt} act='{act}'")
    assert not _lib.lib().fmlp_shape_tuned(D, E, _lib.FMLP_DTYPE_BF16)
    (x, w1, w2, do), (o, dx, dw1, dw2) = _run(H, B, D, E, dt, act, seed=D)
    ro, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    eo = emulate.emu_fwd(x, w1, w2, act, dt)
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
    res = {"o": _fail_frac(o, ro), "o_emu": _fail_frac(o, eo), "dx": _fail_frac(dx, rdx),
           "dw1_emu": _fail_frac(dw1, edw1), "dw2_emu": _fail_frac(dw2, edw2),
           "dw1_rel": _normrel(dw1, rdw1), "dw2_rel": _normrel(dw2, rdw2)}
    _say(f"[generic] D={D} {dt} {act}: " + " ".join(f"{k}={v:.3g}" for k, v in res.items()))
    assert res["o"] == 0 and res["o_emu"] == 0 and res["dx"] == 0, res
    assert res["dw1_emu"] == 0 and res["dw2_emu"] == 0, res
    assert res["dw1_rel"] <= 1e-2 and res["dw2_rel"] <= 1e-2, res


def test_generic_tuned_d_with_odd_e():
    # D = 128 bf16 with E % 8 != 0 leaves the tuned kernels for the generic ones
    (x, w1, w2, do), (o, dx, dw1, dw2) = _run(3, 130, 128, 13, torch.bfloat16, "silu", seed=4)
    ro, rdx, _, _ = reference.autograd_grads(x, w1, w2, do, "silu")
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, "silu", torch.bfloat16)
    assert _fail_frac(o, ro) == 0 and _fail_frac(dx, rdx) == 0
    assert _fail_frac(dw1, edw1) == 0 and _fail_frac(dw2, edw2) == 0


FP32 = [(D, act) for D in (16, 64, 128, 256) for act in ("silu", "leaky_relu", "sigmoid", "")]


@pytest.mark.parametrize("D,act", FP32, ids=[f"D{D}-{a or 'linear'}" for D, a in FP32])
def test_fp32_io(D, act):
    H, B, E = 2, 150, 200
    _say(f"[generic] fp32 io H={H} B={B} D={D} E={E} act='{act}'")
    (x, w1, w2, do), outs = _run(H, B, D, E, torch.float32, act, seed=7)
    refs = reference.autograd_grads(x, w1, w2, do, act)
    rel = [_normrel(g, r) for g, r in zip(outs, refs)]
    _say(f"[generic] fp32 io D={D} {act}: normwise O {rel[0]:.2e} dX {rel[1]:.2e} dW1 {rel[2]:.2e} dW2 {rel[3]:.2e}")
    assert max(rel) <= 1e-4, rel  # the north star's fp32 bar


def test_fp32_cfg1_shape():
    # BASELINE.json configs[0] (the reference's CPU case) run on the GPU in fp32
    (x, w1, w2, do), outs = _run(12, 1024, 64, 768, torch.float32, "silu", seed=0)
    refs = reference.autograd_grads(x, w1, w2, do, "silu")
    rel = [_normrel(g, r) for g, r in zip(outs, refs)]
    _say(f"[generic] fp32 cfg1: normwise {['%.2e' % r for r in rel]}")
    assert max(rel) <= 1e-4, rel


@pytest.mark.parametrize("D,dt", [(32, torch.bfloat16), (256, torch.float16), (64, torch.float32)])
def test_strided_views_are_read_in_place(D, dt):
    # both calls on the generic kernels: at D = 256 an E that is no multiple of 8 keeps the dense
    # forward off the tuned kernel (which takes dense D = 256 inputs with E % 8 == 0)
    H, B, E = 3, 70, (44 if D == 256 else 40)
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=8))
    o_ref = fm.flashmlp_fwd(x, w1, w2, "silu")
    g_ref = fm.flashmlp_bwd(x, w1, w2, do, "silu")
    # x as a transposed copy viewed back, w1 inside a wider buffer, w2 with padded rows,
    # dO broadcast along B (stride 0) like the gradient of o.sum()
    xt = x.transpose(0, 1).contiguous().transpose(0, 1)
    w1w = torch.zeros(H, D, E + 24, dtype=dt, device="cuda")
    w1w[:, :, 5:5 + E] = w1
    w1v = w1w[:, :, 5:5 + E]
    w2p = torch.zeros(H, E, D + 16, dtype=dt, device="cuda")
    w2p[:, :, :D] = w2
    w2v = w2p[:, :, :D]
    assert not (xt.is_contiguous() or w1v.is_contiguous() or w2v.is_contiguous())
    o = fm.flashmlp_fwd(xt, w1v, w2v, "silu")
    assert torch.equal(o, o_ref)
    g = fm.flashmlp_bwd(xt, w1v, w2v, do, "silu")
    for a, b in zip(g, g_ref):
        assert torch.equal(a, b)
    row = do[:, :1, :]
    do0 = row.expand(H, B, D)
    assert do0.stride(1) == 0
    g0 = fm.flashmlp_bwd(x, w1, w2, do0, "silu")
    g0_ref = fm.flashmlp_bwd(x, w1, w2, do0.contiguous(), "silu")
    for a, b in zip(g0, g0_ref):
        assert torch.equal(a, b)


def test_fp32_outputs_on_generic_path():
    # FMLP_OUT_F32: the generic kernels' unrounded fp32 sums against the emulation's
    L = _lib.lib()
    H, B, D, E = 2, 90, 32, 72
    x, w1, w2, do = make_inputs(H, B, D, E, torch.bfloat16, seed=12)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    code = _lib.FMLP_DTYPE_BF16 | _lib.FMLP_OUT_F32
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    o = torch.empty(H, B, D, device="cuda")
    dx = torch.empty(H, B, D, device="cuda")
    dw1 = torch.empty(H, D, E, device="cuda")
    dw2 = torch.empty(H, E, D, device="cuda")
    _lib.check(L.fmlp_fwd(p(xd), p(w1d), p(w2d), p(o), H, B, D, E, code, 1, st), "forward")
    _lib.check(L.fmlp_bwd(p(xd), p(w1d), p(w2d), p(dod), p(dx), p(dw1), p(dw2), H, B, D, E, code, 1, None, 0, st),
               "backward")
    torch.cuda.synchronize()
    eo = emulate.emu_fwd(x, w1, w2, "silu", torch.bfloat16, round_out=False)
    edx, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, "silu", torch.bfloat16, round_out=False)
    rel = [_normrel(a.cpu(), b) for a, b in ((o, eo), (dx, edx), (dw1, edw1), (dw2, edw2))]
    _say(f"[generic] fp32 sums D=32: {['%.2e' % r for r in rel]}")
    assert max(rel) <= 1e-4, rel


def test_accurate_dw_on_generic_path():
    H, B, D, E = 2, 3000, 32, 40
    x, w1, w2, do = make_inputs(H, B, D, E, torch.bfloat16, seed=13)
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    dx, dw1, dw2 = fm.flashmlp_bwd(xd, w1d, w2d, dod, "silu", accurate_dw=True)
    dx0, _, _ = fm.flashmlp_bwd(xd, w1d, w2d, dod, "silu")
    torch.cuda.synchronize()
    assert torch.equal(dx, dx0)
    _, _, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, "silu")
    assert _fail_frac(dw1.cpu(), rdw1) == 0 and _fail_frac(dw2.cpu(), rdw2) == 0


def test_module_fp32_and_small_d():
    torch.manual_seed(0)
    m = fm.FlashMLP(4, 32, 96, activation="silu", dtype=torch.float32, device="cuda")
    x = torch.randn(4, 50, 32, device="cuda", requires_grad=True)
    m(x).sum().backward()
    w1 = m.w1.detach().cpu().requires_grad_(True)
    w2 = m.w2.detach().cpu().requires_grad_(True)
    xc = x.detach().cpu().requires_grad_(True)
    reference.torch_fwd(xc, w1, w2, "silu").sum().backward()
    for got, ref in ((x.grad, xc.grad), (m.w1.grad, w1.grad), (m.w2.grad, w2.grad)):
        assert _normrel(got.cpu(), ref) <= 1e-4


def _bwd_strided(x, w1, w2, do, act, ws_bytes):
    """fmlp_bwd_strided on dense tensors with a workspace of ws_bytes (0: none)."""
    L = _lib.lib()
    H, B, D = x.shape
    E = w1.shape[2]
    code = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16,
            torch.float32: _lib.FMLP_DTYPE_F32}[x.dtype]
    outs = (torch.empty_like(x), torch.empty_like(w1), torch.empty_like(w2))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    st = L.fmlp_bwd_strided(p(x), p(w1), p(w2), p(do), *(p(t) for t in outs), H, B, D, E, _lib.strides(x),
                            _lib.strides(w1), _lib.strides(w2), _lib.strides(do), code, _lib.ACT_CODES[act],
                            p(ws), ws_bytes, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, "backward (strided)")
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("D,dt,act", [(32, torch.bfloat16, "silu"), (256, torch.float16, "sigmoid"),
                                      (64, torch.float32, "leaky_relu")], ids=["D32-bf16", "D256-fp16", "D64-fp32"])
def test_generic_dw_b_split(D, dt, act):
    """The generic dW programs split B over workgroups when the workspace allows (fp32 partials,
    then a reduction in split order): with the queried workspace the results match the oracle at
    the usual bars, and the unsplit run (no workspace) within the summation-order difference."""
    H, B, E = 2, 3000, 136
    x, w1, w2, do = make_inputs(H, B, D, E, dt, seed=81)
    L = _lib.lib()
    code = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16,
            torch.float32: _lib.FMLP_DTYPE_F32}[dt]
    assert L.fmlp_shape_tuned(D, E, code) == 0
    n = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
    _say(f"[generic] B split H={H} B={B} D={D} E={E} {dt} act='{act}' workspace={n}")
    assert n > 0, "this shape should split B"
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    split = [t.cpu() for t in _bwd_strided(xd, w1d, w2d, dod, act, n)]
    whole = [t.cpu() for t in _bwd_strided(xd, w1d, w2d, dod, act, 0)]
    _, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    assert torch.equal(split[0], whole[0])  # dX does not depend on the split
    if dt == torch.float32:
        for got, ref in zip(split, (rdx, rdw1, rdw2)):
            assert _normrel(got, ref) <= 1e-4
    else:
        _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
        assert _fail_frac(split[0], rdx) == 0.0
        for got, emu, ref in ((split[1], edw1, rdw1), (split[2], edw2, rdw2)):
            assert _fail_frac(got, emu) == 0.0
            assert _normrel(got, ref) <= 1e-2
    for a, b in zip(split[1:], whole[1:]):
        assert _normrel(a, b) <= (1e-5 if dt == torch.float32 else 5e-3)  # summation order
