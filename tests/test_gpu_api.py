"""GPU behaviour of the Python API (FlashMLPFunction, FlashMLP, low-level functions) through
the C ABI, against the CPU oracle; mirrors the reference's test_autograd / test_module
(flashmlp.py:799-887) with real asserts."""
import sys

import pytest
import torch

import flashmlp_amd as fm
from oracle import emulate, reference
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu
TOL = dict(atol=3e-2, rtol=3e-2)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check_dw(dw1, dw2, x, w1, w2, do, act, rdw1, rdw2):
    """dW bar: elementwise 3e-2 against the cast-point emulation (h and dZ rounded to the io
    dtype before the dW products, flashmlp.py:297-320), normwise 1e-2 against fp32."""
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, x.dtype)
    for got, emu, ref in ((dw1, edw1, rdw1), (dw2, edw2, rdw2)):
        got = got.float().cpu()
        torch.testing.assert_close(got, emu, **TOL)
        assert ((got - ref).norm() / ref.norm()).item() < 1e-2


def test_autograd_matches_oracle():
    # flashmlp.py:799-855 shape and activation, with N(0,1) / N(0,1/D) / N(0,1/E) inputs
    _say("[api] autograd H=8 B=512 D=64 E=512 silu bf16")
    x, w1, w2, do = make_inputs(8, 512, 64, 512, torch.bfloat16, seed=42)
    xd, w1d, w2d = (t.cuda().requires_grad_(True) for t in (x, w1, w2))
    o = fm.FlashMLPFunction.apply(xd, w1d, w2d, "silu")
    o.backward(do.cuda())
    ro, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, "silu")
    torch.testing.assert_close(o.detach().float().cpu(), ro, **TOL)
    torch.testing.assert_close(xd.grad.float().cpu(), rdx, **TOL)
    _check_dw(w1d.grad, w2d.grad, x, w1, w2, do, "silu", rdw1, rdw2)


def test_autograd_sum_loss_stride0_grad():
    # o.sum().backward() hands the backward a stride-0 dO (flashmlp.py:508 makes it contiguous)
    _say("[api] sum loss")
    x, w1, w2, _ = make_inputs(4, 130, 128, 256, torch.bfloat16, seed=1)
    xd, w1d, w2d = (t.cuda().requires_grad_(True) for t in (x, w1, w2))
    fm.FlashMLPFunction.apply(xd, w1d, w2d, "leaky_relu").sum().backward()
    ones = torch.ones(4, 130, 128)
    _, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, ones, "leaky_relu")
    torch.testing.assert_close(xd.grad.float().cpu(), rdx, **TOL)
    _check_dw(w1d.grad, w2d.grad, x, w1, w2, ones.to(x.dtype), "leaky_relu", rdw1, rdw2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_module_3d_and_2d_inputs(dtype):
    # flashmlp.py:858-887 plus the 2-D path (expand to heads, mean over heads, :603-614)
    _say(f"[api] module {dtype}")
    torch.manual_seed(42)
    m = fm.FlashMLP(num_heads=8, hidden_dim=64, intermediate_dim=512, activation="silu", dtype=dtype, device="cuda")
    w1, w2 = m.w1.detach().float().cpu(), m.w2.detach().float().cpu()
    x = torch.randn(8, 512, 64).to(dtype)
    xd = x.cuda().requires_grad_(True)
    o = m(xd)
    assert o.shape == (8, 512, 64)
    o.sum().backward()
    assert xd.grad is not None and m.w1.grad is not None and m.w2.grad is not None
    ro, rdx, _, _ = reference.autograd_grads(x, w1, w2, torch.ones(8, 512, 64), "silu")
    torch.testing.assert_close(o.detach().float().cpu(), ro, **TOL)
    torch.testing.assert_close(xd.grad.float().cpu(), rdx, **TOL)
    # 2-D input
    m.zero_grad()
    x2 = torch.randn(300, 64).to(dtype)
    x2d = x2.cuda().requires_grad_(True)
    o2 = m(x2d)
    assert o2.shape == (300, 64)
    o2.sum().backward()
    xe = x2.float().unsqueeze(0).expand(8, -1, -1).contiguous().requires_grad_(True)
    ref = reference.torch_fwd(xe, w1, w2, "silu").mean(0)
    ref.sum().backward()
    torch.testing.assert_close(o2.detach().float().cpu(), ref.detach(), **TOL)
    torch.testing.assert_close(x2d.grad.float().cpu(), xe.grad.sum(0), **TOL)


def test_unsupported_dtype_and_device_errors():
    x, w1, w2, _ = make_inputs(2, 8, 64, 64, torch.float32)
    with pytest.raises(TypeError, match="float16, bfloat16 and float32"):
        fm.flashmlp_fwd(x.cuda().double(), w1.cuda().double(), w2.cuda().double(), "silu")
    with pytest.raises(TypeError, match="one dtype"):
        fm.flashmlp_fwd(x.cuda().bfloat16(), w1.cuda().half(), w2.cuda().bfloat16(), "silu")
    with pytest.raises(RuntimeError, match="unsupported"):
        xb = torch.zeros(2, 8, 96, dtype=torch.bfloat16, device="cuda")
        fm.flashmlp_fwd(xb, torch.zeros(2, 96, 64, dtype=torch.bfloat16, device="cuda"),
                        torch.zeros(2, 64, 96, dtype=torch.bfloat16, device="cuda"), "silu")


def test_views_streams_and_unknown_activation():
    _say("[api] views/streams")
    x, w1, w2, do = make_inputs(3, 100, 64, 128, torch.bfloat16, seed=5)
    ref_o = fm.flashmlp_fwd(x.cuda(), w1.cuda(), w2.cuda(), "")
    # non-contiguous x: reshape copies, as in the reference
    xt = x.transpose(0, 1).contiguous().cuda().transpose(0, 1)
    assert not xt.is_contiguous()
    torch.testing.assert_close(fm.flashmlp_fwd(xt, w1.cuda(), w2.cuda(), ""), ref_o, atol=0, rtol=0)
    # a view at a 2-byte storage offset (not 16-byte aligned)
    buf = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device="cuda")
    xv = buf[1:].view(x.shape)
    xv.copy_(x.cuda())
    torch.testing.assert_close(fm.flashmlp_fwd(xv, w1.cuda(), w2.cuda(), ""), ref_o, atol=0, rtol=0)
    # unknown activation string means linear (flashmlp.py:146-147)
    torch.testing.assert_close(fm.flashmlp_fwd(x.cuda(), w1.cuda(), w2.cuda(), "gelu"), ref_o, atol=0, rtol=0)
    # a non-default stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        xs, w1s, w2s, dos = x.cuda(), w1.cuda(), w2.cuda(), do.cuda()
        o_s = fm.flashmlp_fwd(xs, w1s, w2s, "")
        g_s = fm.flashmlp_bwd(xs, w1s, w2s, dos, "")
    s.synchronize()
    torch.testing.assert_close(o_s, ref_o, atol=0, rtol=0)
    g = fm.flashmlp_bwd(x.cuda(), w1.cuda(), w2.cuda(), do.cuda(), "")
    for a, b in zip(g_s, g):
        torch.testing.assert_close(a, b, atol=0, rtol=0)


def test_empty_batch():
    x = torch.zeros(2, 0, 64, dtype=torch.bfloat16, device="cuda")
    _, w1, w2, _ = make_inputs(2, 1, 64, 64, torch.bfloat16)
    w1, w2 = w1.cuda(), w2.cuda()
    o = fm.flashmlp_fwd(x, w1, w2, "silu")
    assert o.shape == (2, 0, 64)
    dx, dw1, dw2 = fm.flashmlp_bwd(x, w1, w2, torch.zeros_like(x), "silu")
    assert dx.shape == (2, 0, 64)
    assert torch.count_nonzero(dw1) == 0 and torch.count_nonzero(dw2) == 0


def test_leaky_relu_zero_point_follows_autograd():
    # rows of X that are exactly zero give Z == 0: autograd's slope 0.01 applies there
    # (the reference Triton kernel uses 1, flashmlp.py:33-34); dX differs by 100x
    _say("[api] leaky zero rows")
    x, w1, w2, do = make_inputs(16, 256, 128, 512, torch.bfloat16, seed=3)
    x[:, ::7] = 0
    dx, dw1, dw2 = fm.flashmlp_bwd(x.cuda(), w1.cuda(), w2.cuda(), do.cuda(), "leaky_relu")
    _, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, "leaky_relu")
    torch.testing.assert_close(dx.float().cpu(), rdx, **TOL)
    assert rdx[:, ::7].abs().max() > 0


def test_bwd_falls_back_to_recompute_when_workspace_does_not_fit(monkeypatch):
    """flashmlp_bwd takes the recompute form when the stored-dZ workspace cannot be allocated
    (the reference's backward allocates no workspace): same results as recompute=True."""
    import importlib

    from flashmlp_amd import _lib

    fmm = importlib.import_module("flashmlp_amd.flashmlp")
    # the first of these shapes for which the plan takes the stored-dZ form (the choice is the
    # plan's estimate, so the shape is looked up rather than assumed)
    dt, act = torch.float16, "sigmoid"
    code, act_code = _lib.FMLP_DTYPE_F16, _lib.ACT_CODES[act]
    shapes = [(8, 4097, 64, 2048), (8, 8192, 128, 1024), (16, 8192, 128, 1024), (32, 8192, 128, 1024)]
    found = [s for s in shapes if _lib.lib().fmlp_bwd_stores_dz(*s, code, act_code) == 1
             and _lib.lib().fmlp_bwd_workspace_bytes(*s, code | _lib.FMLP_BWD_RECOMPUTE) < (64 << 20)]
    assert found, "no candidate shape takes the stored-dZ form with a recompute workspace under 64 MiB"
    H, B, D, E = found[0]
    _say(f"[api] workspace fallback H={H} B={B} D={D} E={E} {dt} act='{act}'")
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=61))
    ref = fm.flashmlp_bwd(x, w1, w2, do, act, recompute=True)
    real, sizes = fmm._alloc_ws, []

    def tight(nbytes, device):  # a device with less than 64 MiB free
        sizes.append(nbytes)
        if nbytes > (64 << 20):
            raise torch.OutOfMemoryError("simulated: workspace does not fit")
        return real(nbytes, device)

    monkeypatch.setattr(fmm, "_alloc_ws", tight)
    monkeypatch.setattr(fmm, "_fast", None)  # the general path (the fast path allocates in C++)
    got = fm.flashmlp_bwd(x, w1, w2, do, act)
    torch.cuda.synchronize()
    assert len(sizes) == 2 and sizes[0] > (64 << 20) >= sizes[1]
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_fast_path_falls_back_to_recompute_when_workspace_does_not_fit():
    """The fast path (_fmlp_fast) takes the recompute form when allocating the stored-dZ
    workspace fails, like the general path: a real allocation failure under a per-process memory
    limit that leaves room for the outputs and the recompute form's workspace only."""
    import importlib

    from flashmlp_amd import _lib

    fmm = importlib.import_module("flashmlp_amd.flashmlp")
    assert fmm._fast is not None, "the fast path module is not built"
    dt, act = torch.bfloat16, "silu"
    code, act_code = _lib.FMLP_DTYPE_BF16, _lib.ACT_CODES[act]
    L = _lib.lib()
    found = None
    for H, B, D, E in [(16, 8192, 128, 1024), (32, 8192, 128, 1024), (32, 16384, 128, 1024)]:
        if L.fmlp_bwd_stores_dz(H, B, D, E, code, act_code) != 1:
            continue
        dz_ws = L.fmlp_bwd_workspace_bytes(H, B, D, E, code)
        rec_ws = L.fmlp_bwd_workspace_bytes(H, B, D, E, code | _lib.FMLP_BWD_RECOMPUTE)
        out = 2 * (H * B * D + 2 * H * D * E)
        if dz_ws > rec_ws + out + (96 << 20):
            found = (H, B, D, E, rec_ws, out)
            break
    assert found, "no candidate shape takes the stored-dZ form with room to tell the forms apart"
    H, B, D, E, rec_ws, out = found
    _say(f"[api] fast-path workspace fallback H={H} B={B} D={D} E={E} {dt} act='{act}'")
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=62))
    ref = fm.flashmlp_bwd(x, w1, w2, do, act, recompute=True)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    total = torch.cuda.get_device_properties(0).total_memory
    allowed = torch.cuda.memory_reserved() + rec_ws + out + (64 << 20)
    torch.cuda.set_per_process_memory_fraction(allowed / total)
    try:
        got = fm.flashmlp_bwd(x, w1, w2, do, act)
        torch.cuda.synchronize()
    finally:
        torch.cuda.set_per_process_memory_fraction(1.0)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


FAST_CASES = [
    (4, 1000, 64, 512, torch.float16, "sigmoid"),       # tuned, B tail
    (8, 4097, 64, 2048, torch.float16, "sigmoid"),      # forward split tiles, ragged dX split
    (2, 4096, 128, 512, torch.bfloat16, "silu"),        # B split of the dW programs
    (4, 2048, 128, 1024, torch.bfloat16, "leaky_relu"),
]


@pytest.mark.parametrize("H,B,D,E,dt,act", FAST_CASES, ids=[f"H{c[0]}-B{c[1]}-D{c[2]}-E{c[3]}" for c in FAST_CASES])
def test_fast_path_equals_general_path(monkeypatch, H, B, D, E, dt, act):
    """flashmlp_fwd / flashmlp_bwd through _fmlp_fast and through the ctypes path give bitwise
    equal results (the same C ABI calls), for every backward mode and partial backward."""
    import importlib

    fmm = importlib.import_module("flashmlp_amd.flashmlp")
    assert fmm._fast is not None, "the fast path module is not built"
    _say(f"[api] fast vs general H={H} B={B} D={D} E={E} {dt} act='{act}'")
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=63))
    kws = [dict(), dict(recompute=True), dict(accurate_dw=True), dict(_needs=(True, False)),
           dict(_needs=(False, True))]
    fast_o = fm.flashmlp_fwd(x, w1, w2, act)
    fast_g = [fm.flashmlp_bwd(x, w1, w2, do, act, **kw) for kw in kws]
    monkeypatch.setattr(fmm, "_fast", None)
    gen_o = fm.flashmlp_fwd(x, w1, w2, act)
    gen_g = [fm.flashmlp_bwd(x, w1, w2, do, act, **kw) for kw in kws]
    torch.cuda.synchronize()
    assert torch.equal(fast_o, gen_o)
    for kw, a, b in zip(kws, fast_g, gen_g):
        for u, v in zip(a, b):
            assert (u is None) == (v is None), kw
            if u is not None:
                assert torch.equal(u, v), kw


@pytest.mark.parametrize("H,B,D,E,dt,act", [
    (2, 4096, 128, 512, torch.bfloat16, "silu"),       # tuned kernels, B split of the dW programs
    (8, 4097, 64, 2048, torch.float16, "sigmoid"),     # tuned kernels, B and dX-tile tails
    (3, 300, 32, 45, torch.float16, "leaky_relu"),     # generic kernels
    (1, 4096, 128, 1024, torch.bfloat16, "silu"),      # stored dZ, dW programs split unlike the recompute form's
], ids=["bf16-D128", "fp16-D64-tail", "fp16-D32-generic", "bf16-D128-stored-dz"])
def test_function_computes_only_the_gradients_autograd_needs(H, B, D, E, dt, act):
    """FlashMLPFunction passes autograd's needs_input_grad down (FMLP_BWD_NO_DX / FMLP_BWD_NO_DW):
    an input or weights that need no gradient skip the dX or the dW programs; dW is
    bit-identical to the full backward's (the dW programs of its plan), dX to the recompute
    form's (whose dX programs run)."""
    _say(f"[api] partial backward H={H} B={B} D={D} E={E} {dt} act='{act}'")
    x, w1, w2, do = (t.cuda() for t in make_inputs(H, B, D, E, dt, seed=62))
    dx = fm.flashmlp_bwd(x, w1, w2, do, act, recompute=True)[0]
    _, dw1, dw2 = fm.flashmlp_bwd(x, w1, w2, do, act)
    # the input needs no gradient: dW programs only
    w1g, w2g = w1.clone().requires_grad_(True), w2.clone().requires_grad_(True)
    fm.FlashMLPFunction.apply(x, w1g, w2g, act).backward(do)
    assert torch.equal(w1g.grad, dw1) and torch.equal(w2g.grad, dw2)
    # frozen weights: dX programs only
    xg = x.clone().requires_grad_(True)
    fm.FlashMLPFunction.apply(xg, w1, w2, act).backward(do)
    assert torch.equal(xg.grad, dx)
    # one weight needs a gradient: the dW programs run, only that gradient is returned
    w2h = w2.clone().requires_grad_(True)
    fm.FlashMLPFunction.apply(x, w1, w2h, act).backward(do)
    assert torch.equal(w2h.grad, dw2)
    # the low-level function with nothing needed returns no tensors and launches nothing
    assert fm.flashmlp_bwd(x, w1, w2, do, act, _needs=(False, False)) == (None, None, None)
    torch.cuda.synchronize()
