"""The forward's split tiles (fmlp_fwd_ws): tiles split over E across workgroups, fp32 partials in
the caller's workspace, summed by a second launch.

The split is taken where a last round of tiles would leave most CUs idle: at most a quarter of
the CUs' worth of tiles after full rounds (a ragged B just past a multiple of the CU count, as
cfg5's B = 4097; those tiles split). Each case checks, through the C ABI:
  * that the shape does take the split (fmlp_fwd_workspace_bytes > 0);
  * the fp32 sums (FMLP_OUT_F32) against the oracle's emulation at the north star's 1e-4, and
    against fmlp_fwd's whole tiles (which differ from the split only in summation order);
  * the io output against the oracle's cast-point emulation: no element outside the parity
    bar of test_gpu_parity (3e-2 + 3e-2 |ref|), and the largest error within one io ulp of the
    output's largest magnitude, with NaN-filled output and workspace beforehand (every element
    must be written, no stale partial may be read);
  * bitwise equality of two split calls (a fixed summation order) and, for a workspace one
    byte short, bitwise equality with fmlp_fwd (the split is then not taken).
"""
import ctypes
import sys

import pytest
import torch

from flashmlp_amd import _lib
from oracle import emulate
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu

_DT = {torch.float16: _lib.FMLP_DTYPE_F16, torch.bfloat16: _lib.FMLP_DTYPE_BF16}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _normrel(a, b):
    a = a.double()
    b = b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _cases():
    n = _cus()
    # (name, H, B, D, E, dtype, act, heads checked against the oracle)
    return [
        ("D64-ragged-last-round", 8, (n // 8) * 128 + 1, 64, 2048, torch.float16, "sigmoid", [0, 7]),
        ("D64-ragged-bf16", 4, (n // 4) * 128 + 65, 64, 512, torch.bfloat16, "leaky_relu", [0, 3]),
        ("D64-ragged-E-tail", 2, (n // 2) * 128 + 100, 64, 296, torch.float16, "silu", [0, 1]),
        ("D128-ragged-last-round", 1, n * 256 + 1, 128, 256, torch.bfloat16, "silu", None),
        ("D128-two-rounds-ragged", 3, (n // 3) * 2 * 256 + 256 * (2 * n % 3) + 7, 128, 512, torch.bfloat16, "", [1]),
    ]


def _fwd(L, x, w1, w2, act, code, out_dtype, ws=None, ws_bytes=0, fill_nan=False):
    H, B, D = x.shape
    E = w1.shape[2]
    o = torch.empty(H, B, D, dtype=out_dtype, device=x.device)
    if fill_nan:
        o.fill_(float("nan"))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a = _lib.ACT_CODES[act]
    if ws is None and ws_bytes == 0:
        st = L.fmlp_fwd(_ptr(x), _ptr(w1), _ptr(w2), _ptr(o), H, B, D, E, code, a, stream)
    else:
        st = L.fmlp_fwd_ws(_ptr(x), _ptr(w1), _ptr(w2), _ptr(o), H, B, D, E, code, a, _ptr(ws), ws_bytes, stream)
    _lib.check(st, "forward")
    torch.cuda.synchronize()
    return o


@pytest.mark.parametrize("case", range(5), ids=[c[0] for c in _cases()] if torch.cuda.is_available() else None)
def test_split_forward(case):
    name, H, B, D, E, dt, act, heads = _cases()[case]
    L = _lib.lib()
    code = _DT[dt]
    n = L.fmlp_fwd_workspace_bytes(H, B, D, E, code)
    _say(f"[fwd-split] {name}: H={H} B={B} D={D} E={E} {dt} act='{act}' cus={_cus()} ws={n}")
    assert n > 0, "this shape should take the split"
    assert L.fmlp_fwd_workspace_bytes(H, B, D, E, code | _lib.FMLP_OUT_F32) == n
    x, w1, w2, _ = make_inputs(H, B, D, E, dt, 1.0, seed=7 + case, with_do=False)
    xd, w1d, w2d = (t.cuda() for t in (x, w1, w2))
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    hs = list(range(H)) if heads is None else heads

    # fp32 sums: oracle and whole tiles
    ws.view(torch.float32).fill_(float("nan"))
    s_split = _fwd(L, xd, w1d, w2d, act, code | _lib.FMLP_OUT_F32, torch.float32, ws, n, fill_nan=True)
    s_whole = _fwd(L, xd, w1d, w2d, act, code | _lib.FMLP_OUT_F32, torch.float32)
    assert torch.isfinite(s_split).all()
    eo = emulate.emu_fwd(x[hs], w1[hs], w2[hs], act, dt, round_out=False)
    rel_o = _normrel(s_split[hs].cpu(), eo)
    rel_w = _normrel(s_split, s_whole)
    _say(f"[fwd-split] {name}: fp32 sums rel to oracle {rel_o:.3g}, to whole tiles {rel_w:.3g}")
    assert rel_o <= 1e-4
    assert rel_w <= 1e-5

    # io output: oracle within one io ulp of the output's scale, every element written
    ws.view(torch.float32).fill_(float("nan"))
    o1 = _fwd(L, xd, w1d, w2d, act, code, dt, ws, n, fill_nan=True)
    assert torch.isfinite(o1.float()).all()
    ref = emulate.emu_fwd(x[hs], w1[hs], w2[hs], act, dt, round_out=True).float()
    got = o1[hs].float().cpu()
    # one io ulp at the output's largest magnitude m is at most m 2^-7 (bf16) / m 2^-10 (fp16)
    ulp = 2.0 ** (-7 if dt == torch.bfloat16 else -10)
    tol = ulp * ref.abs().amax().item() + 1e-6
    err = (got - ref).abs().max().item()
    bad = ((got - ref).abs() > 3e-2 + 3e-2 * ref.abs()).sum().item()
    _say(f"[fwd-split] {name}: io max |err| {err:.3g} (bar {tol:.3g}), {bad} outside 3e-2")
    assert bad == 0
    assert err <= tol

    # a fixed summation order; one byte short of the workspace = fmlp_fwd
    o2 = _fwd(L, xd, w1d, w2d, act, code, dt, ws, n)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    o3 = _fwd(L, xd, w1d, w2d, act, code, dt, ws, n - 1)
    o4 = _fwd(L, xd, w1d, w2d, act, code, dt)
    assert torch.equal(o3.view(torch.int16), o4.view(torch.int16))


def test_python_forward_uses_split():
    # flashmlp_fwd allocates the workspace itself: its result equals fmlp_fwd_ws's bitwise
    from flashmlp_amd import flashmlp_fwd

    name, H, B, D, E, dt, act, _ = _cases()[0]
    L = _lib.lib()
    x, w1, w2, _ = make_inputs(H, B, D, E, dt, 1.0, seed=3, with_do=False)
    xd, w1d, w2d = (t.cuda() for t in (x, w1, w2))
    n = L.fmlp_fwd_workspace_bytes(H, B, D, E, _DT[dt])
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    _say(f"[fwd-split] flashmlp_fwd at {name}")
    a = _fwd(L, xd, w1d, w2d, act, _DT[dt], dt, ws, n)
    b = flashmlp_fwd(xd, w1d, w2d, act)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _t64_cases():
    n = _cus()
    # (name, H, B, E, dtype, act): D = 64 grids whose 64-row tiles fit on the CUs at one workgroup
    # each (H ceil(B / 64) <= CUs) with at least 8 E-chunks: the forward's 64-row tiles in four
    # E parts of two waves
    return [
        ("cfg2", 12, 1024, 768, torch.float16, "silu"),
        ("ragged-B-E-tail", 3, 1000, 264, torch.bfloat16, "sigmoid"),  # 9 chunks: the 4th part's are past E
        ("tiny-B", 5, 129, 256, torch.float16, ""),
        ("long-E", 2, 64, 2048, torch.bfloat16, "silu"),
        ("full-round", n // 4, 256 - 17, 512, torch.bfloat16, "leaky_relu"),
    ]


@pytest.mark.parametrize("case", range(5), ids=[c[0] for c in _t64_cases()] if torch.cuda.is_available() else None)
def test_forward_64_row_tiles(case):
    """D = 64 grids small enough for 64-row tiles (fwd_plan: four E parts of two waves, each
    through a 4-slot ring, partial tiles added in part order): fp32 sums against the emulation at
    1e-4 with the output NaN-filled first, io output at the parity bar, bitwise repeats, and no
    workspace (fmlp_fwd_workspace_bytes is 0)."""
    name, H, B, E, dt, act = _t64_cases()[case]
    D = 64
    L = _lib.lib()
    code = _DT[dt]
    assert H * ((B + 63) // 64) <= _cus() and (E + 31) // 32 >= 8, "the case must take the 64-row tiles"
    assert L.fmlp_fwd_workspace_bytes(H, B, D, E, code) == 0
    _say(f"[fwd-t64] {name}: H={H} B={B} D={D} E={E} {dt} act='{act}'")
    x, w1, w2, _ = make_inputs(H, B, D, E, dt, 1.0, seed=40 + case, with_do=False)
    xd, w1d, w2d = (t.cuda() for t in (x, w1, w2))
    s = _fwd(L, xd, w1d, w2d, act, code | _lib.FMLP_OUT_F32, torch.float32, fill_nan=True)
    assert torch.isfinite(s).all()
    rel = _normrel(s.cpu(), emulate.emu_fwd(x, w1, w2, act, dt, round_out=False))
    o1 = _fwd(L, xd, w1d, w2d, act, code, dt, fill_nan=True)
    o2 = _fwd(L, xd, w1d, w2d, act, code, dt)
    ref = emulate.emu_fwd(x, w1, w2, act, dt, round_out=True).float()
    bad = ((o1.float().cpu() - ref).abs() > 3e-2 + 3e-2 * ref.abs()).sum().item()
    _say(f"[fwd-t64] {name}: fp32 sums rel to oracle {rel:.3g}, {bad} io elements outside 3e-2")
    assert rel <= 1e-4
    assert bad == 0
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
