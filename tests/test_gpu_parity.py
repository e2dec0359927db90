"""Parity of the gfx950 kernels (through the Python API and the C ABI) with the oracle.

Bars:
  * O and dX: elementwise |gpu - ref| <= 3e-2 + 3e-2 |ref| against the fp32 autograd oracle
    (oracle.reference) computed on the CPU from the same io-quantised inputs.
  * dW1 and dW2: the same elementwise bar against the cast-point emulation of the reference
    kernels (oracle.emulate: h and dZ rounded to the io dtype before the dW products, as
    flashmlp.py:297-320 does); against the fp32 oracle the normwise relative error must be
    <= 1e-2 (rounding h/dZ to bf16 over B = 16384 terms leaves a few percent of elements
    outside 3e-2 elementwise, for the reference kernel and for torch's own bf16 autograd
    alike; the fraction is printed).
Heads are independent (flashmlp.py:82-85, 360-365): for the large configurations the CPU
oracle checks a subset of heads of the full GPU result.
"""
import math
import sys

import pytest
import torch

from oracle import emulate, reference
from oracle.inputs import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu

ATOL = 3e-2
RTOL = 3e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fail_frac(a, b, atol=ATOL, rtol=RTOL):
    a = a.float()
    b = b.float()
    bad = (a - b).abs() > atol + rtol * b.abs()
    return bad.float().mean().item()


def _normrel(a, b):
    a = a.double()
    b = b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _gpu():
    import flashmlp_amd

    return flashmlp_amd


def run_case(name, H, B, D, E, dtype, act, x_std=1.0, seed=0, heads=None, check_bwd=True, bwd_kw=None):
    fm = _gpu()
    x, w1, w2, do = make_inputs(H, B, D, E, dtype, x_std, seed)
    _say(f"[parity] {name}: H={H} B={B} D={D} E={E} {dtype} act='{act}' seed={seed} bwd={bwd_kw or {}}")
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    o = fm.flashmlp_fwd(xd, w1d, w2d, act)
    if check_bwd:
        dx, dw1, dw2 = fm.flashmlp_bwd(xd, w1d, w2d, dod, act, **(bwd_kw or {}))
    torch.cuda.synchronize()
    hs = list(range(H)) if heads is None else heads
    sel = lambda t: t[hs].cpu()
    xs, w1s, w2s, dos = sel(x), sel(w1), sel(w2), sel(do)
    ro, rdx, rdw1, rdw2 = reference.autograd_grads(xs, w1s, w2s, dos, act)
    res = {}
    res["o_fail"] = _fail_frac(sel(o), ro)
    res["o_rel"] = _normrel(sel(o), ro)
    eo = emulate.emu_fwd(xs, w1s, w2s, act, dtype)
    res["o_emu_fail"] = _fail_frac(sel(o), eo)
    if check_bwd:
        edx, edw1, edw2 = emulate.emu_bwd(xs, w1s, w2s, dos, act, dtype)
        res["dx_fail"] = _fail_frac(sel(dx), rdx)
        res["dx_rel"] = _normrel(sel(dx), rdx)
        res["dw1_emu_fail"] = _fail_frac(sel(dw1), edw1)
        res["dw2_emu_fail"] = _fail_frac(sel(dw2), edw2)
        res["dw1_rel"] = _normrel(sel(dw1), rdw1)
        res["dw2_rel"] = _normrel(sel(dw2), rdw2)
        res["dw1_fail_vs_fp32"] = _fail_frac(sel(dw1), rdw1)
        res["dw2_fail_vs_fp32"] = _fail_frac(sel(dw2), rdw2)
        for t in (dx, dw1, dw2):
            assert torch.isfinite(t.float()).all()
    assert torch.isfinite(o.float()).all()
    _say(f"[parity] {name}: " + " ".join(f"{k}={v:.3g}" for k, v in res.items()))
    assert res["o_fail"] == 0.0, res
    assert res["o_emu_fail"] == 0.0, res
    if check_bwd:
        assert res["dx_fail"] == 0.0, res
        assert res["dw1_emu_fail"] == 0.0, res
        assert res["dw2_emu_fail"] == 0.0, res
        assert res["dw1_rel"] <= 1e-2 and res["dw2_rel"] <= 1e-2, res
    return res


# ---- small cases: every dtype x D x activation, tails in B and E ----
SMALL = []
for dt in (torch.float16, torch.bfloat16):
    for D in (64, 128):
        for act in ("", "silu", "leaky_relu", "sigmoid"):
            SMALL.append((dt, D, act))


@pytest.mark.parametrize("dt,D,act", SMALL, ids=[f"{str(d).split('.')[-1]}-D{D}-{a or 'linear'}" for d, D, a in SMALL])
def test_small(dt, D, act):
    run_case("small", 3, 200, D, 96, dt, act, seed=1)


@pytest.mark.parametrize("B,E", [(1, 8), (33, 40), (127, 136), (129, 264), (300, 520)])
def test_tails(B, E):
    run_case("tail", 2, B, 128, E, torch.bfloat16, "silu", seed=2)
    run_case("tail", 2, B, 64, E, torch.float16, "sigmoid", seed=3)


def test_reference_shapes():
    # flashmlp.py:738 / :807 shapes (bf16), all activations
    for act in ("", "silu", "leaky_relu", "sigmoid"):
        run_case("ref-test-shape", 12, 1024, 64, 768, torch.bfloat16, act, seed=42)
    run_case("ref-autograd-shape", 8, 512, 64, 512, torch.bfloat16, "silu", seed=42)


# Regression guard on dW against the fp32 oracle at the bf16 configurations: rounding h and
# dZ to bf16 (the reference's cast points) leaves this share of dW elements just outside the
# elementwise 3e-2 bar (CPU emulation of the same cast points: cfg3 1.57 % / 2.28 %, cfg4
# 1.48 % / 2.61 %). A kernel change that stays within the normwise 1e-2 but loses accuracy
# elementwise shows up here.
DW_FP32_MISS_BOUND = {"cfg3": (0.019, 0.028), "cfg4": (0.018, 0.031)}


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg5_linear", "cfg5_sigmoid"])
def test_config(name):
    c = CONFIGS[name]
    heads = None if c.H * c.B <= 16 * 4097 else [0, c.H - 1]
    res = run_case(name, c.H, c.B, c.D, c.E, c.dtype, c.activation, c.x_std, heads=heads)
    if name in DW_FP32_MISS_BOUND:
        b1, b2 = DW_FP32_MISS_BOUND[name]
        assert res["dw1_fail_vs_fp32"] <= b1 and res["dw2_fail_vs_fp32"] <= b2, res
    elif c.dtype == torch.float16:
        # fp16 keeps 3 more bits of h and dZ: dW passes the bar against fp32 itself
        assert res["dw1_fail_vs_fp32"] <= 1e-3 and res["dw2_fail_vs_fp32"] <= 1e-3, res


def test_config4_north_star():
    c = CONFIGS["cfg4"]
    res = run_case("cfg4", c.H, c.B, c.D, c.E, c.dtype, c.activation, c.x_std, heads=[0, 17, 31])
    _say(f"[parity] cfg4 dW elementwise-3e-2 fraction vs fp32 oracle: dW1 {res['dw1_fail_vs_fp32']:.4f} "
         f"dW2 {res['dw2_fail_vs_fp32']:.4f}")
    b1, b2 = DW_FP32_MISS_BOUND["cfg4"]
    assert res["dw1_fail_vs_fp32"] <= b1 and res["dw2_fail_vs_fp32"] <= b2, res


def test_config4_recompute_form():
    """cfg4 in the reference's recompute-only backward (flashmlp.py:341-421: the dX programs
    recompute Z and dH, no dZ is stored), the form the north star names; the plan picks the
    stored-dZ form at this shape, so it is forced here. Same heads and bars as above."""
    from flashmlp_amd import _lib

    c = CONFIGS["cfg4"]
    code = _lib.FMLP_DTYPE_BF16 | _lib.FMLP_BWD_RECOMPUTE
    assert _lib.lib().fmlp_bwd_stores_dz(c.H, c.B, c.D, c.E, code, _lib.ACT_CODES[c.activation]) == 0
    res = run_case("cfg4-recompute", c.H, c.B, c.D, c.E, c.dtype, c.activation, c.x_std, heads=[0, 17, 31],
                   bwd_kw=dict(recompute=True))
    b1, b2 = DW_FP32_MISS_BOUND["cfg4"]
    assert res["dw1_fail_vs_fp32"] <= b1 and res["dw2_fail_vs_fp32"] <= b2, res


# More tiles than one round of resident workgroups (over 256 at D = 128, over 512 at D = 64
# on 256 CUs), with a B tail, a partial last E-chunk and an odd number of E-chunks.
MULTI_ROUND = [(8, 8300, 128, 1000, torch.bfloat16, "silu"), (4, 16500, 64, 992, torch.float16, "sigmoid"),
               (9, 7500, 128, 520, torch.bfloat16, "leaky_relu")]


@pytest.mark.parametrize("H,B,D,E,dt,act", MULTI_ROUND, ids=[f"H{c[0]}-B{c[1]}-D{c[2]}-E{c[3]}" for c in MULTI_ROUND])
def test_multi_round_tails(H, B, D, E, dt, act):
    run_case("multi-round", H, B, D, E, dt, act, seed=11, heads=[0, H - 1])


@pytest.mark.parametrize("act", ["", "sigmoid"], ids=["linear", "sigmoid"])
def test_config5s_forward_sweep(act):
    # the fp16 forward-only inference sweep at B = 65536
    # (H=8 D=64 E=2048, X ~ N(0, 4)); heads 0 and 7 against the oracle (heads are independent)
    c = CONFIGS["cfg5s"]
    run_case("cfg5s", c.H, c.B, c.D, c.E, c.dtype, act, c.x_std, heads=[0, c.H - 1], check_bwd=False)
