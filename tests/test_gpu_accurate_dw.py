"""The backward's accuracy mode for dW (accurate_dw=True, C ABI flag FMLP_DW_HILO) against
the fp32 autograd oracle (oracle.reference, flashmlp.py:671-686 restated).

In the default mode h and dZ are rounded to the io dtype before the dW products, as the
reference kernel does (flashmlp.py:297-320); at bf16 and B = 16384 that leaves 1.5-2.6 % of
dW elements just outside the elementwise bar atol = rtol = 3e-2 against fp32. The accuracy
mode takes h and dZ as hi + lo io-dtype terms, so dW1 and dW2 must meet the bar on every
element, at the north-star shape too. dX does not use the mode: it must be bit-identical to
the default mode's.
"""
import sys

import pytest
import torch

from oracle import reference
from oracle.inputs import CONFIGS, make_inputs

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


def _check(name, H, B, D, E, dtype, act, x_std=1.0, seed=0, heads=None, rel_bound=1e-4, recompute=False):
    import flashmlp_amd as fm

    x, w1, w2, do = make_inputs(H, B, D, E, dtype, x_std, seed)
    _say(f"[accurate_dw] {name}: H={H} B={B} D={D} E={E} {dtype} act='{act}' seed={seed} recompute={recompute}")
    xd, w1d, w2d, dod = (t.cuda() for t in (x, w1, w2, do))
    dx, dw1, dw2 = fm.flashmlp_bwd(xd, w1d, w2d, dod, act, accurate_dw=True, recompute=recompute)
    dx0, dw10, dw20 = fm.flashmlp_bwd(xd, w1d, w2d, dod, act, recompute=recompute)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx0), "dX must not depend on the dW mode"
    hs = list(range(H)) if heads is None else heads
    sel = lambda t: t[hs].cpu()
    _, rdx, rdw1, rdw2 = reference.autograd_grads(sel(x), sel(w1), sel(w2), sel(do), act)
    res = {
        "dw1_fail": _fail_frac(sel(dw1), rdw1), "dw2_fail": _fail_frac(sel(dw2), rdw2),
        "dw1_rel": _normrel(sel(dw1), rdw1), "dw2_rel": _normrel(sel(dw2), rdw2),
        "dw1_rel_default": _normrel(sel(dw10), rdw1), "dw2_rel_default": _normrel(sel(dw20), rdw2),
        "dx_fail": _fail_frac(sel(dx), rdx),
    }
    _say(f"[accurate_dw] {name}: " + " ".join(f"{k}={v:.3g}" for k, v in res.items()))
    assert res["dw1_fail"] == 0.0 and res["dw2_fail"] == 0.0, res
    assert res["dx_fail"] == 0.0, res
    # the dW error left is that of the io-dtype output rounding, far below the default mode's
    assert res["dw1_rel"] <= rel_bound and res["dw2_rel"] <= rel_bound, res
    return res


CASES = [(dt, D, act) for dt in (torch.float16, torch.bfloat16) for D in (64, 128)
         for act in ("", "silu", "leaky_relu", "sigmoid")]


@pytest.mark.parametrize("dt,D,act", CASES, ids=[f"{str(d).split('.')[-1]}-D{D}-{a or 'linear'}" for d, D, a in CASES])
def test_small(dt, D, act):
    # B = 700 at D = 64, E = 264: the dW programs split B (fp32 partials + reduction) in this
    # mode for the non-linear activations
    _check("small", 3, 700, D, 264, dt, act, seed=5, rel_bound=5e-3 if dt == torch.bfloat16 else 1e-3)


def test_config3():
    c = CONFIGS["cfg3"]
    _check("cfg3", c.H, c.B, c.D, c.E, c.dtype, c.activation, c.x_std, heads=[0, c.H - 1], rel_bound=5e-3)


@pytest.mark.parametrize("recompute", [False, True], ids=["plan-form", "recompute-form"])
def test_config4_north_star(recompute):
    # the plan's form (stored dZ at this shape) and the reference's recompute-only form
    c = CONFIGS["cfg4"]
    res = _check("cfg4", c.H, c.B, c.D, c.E, c.dtype, c.activation, c.x_std, heads=[0, 17, 31], rel_bound=5e-3,
                 recompute=recompute)
    _say(f"[accurate_dw] cfg4 dW elementwise-3e-2 misses vs fp32: dW1 {res['dw1_fail']:.4f} dW2 {res['dw2_fail']:.4f}"
         f" (default mode normwise {res['dw1_rel_default']:.2e} / {res['dw2_rel_default']:.2e})")


def test_autograd_and_module():
    import flashmlp_amd as fm

    H, B, D, E = 2, 300, 64, 128
    x, w1, w2, do = make_inputs(H, B, D, E, torch.bfloat16, seed=9)
    xd = x.cuda().requires_grad_(True)
    w1d = w1.cuda().requires_grad_(True)
    w2d = w2.cuda().requires_grad_(True)
    o = fm.FlashMLPFunction.apply(xd, w1d, w2d, "silu", True)
    o.backward(do.cuda())
    dx, dw1, dw2 = fm.flashmlp_bwd(x.cuda(), w1.cuda(), w2.cuda(), do.cuda(), "silu", accurate_dw=True)
    torch.cuda.synchronize()
    assert torch.equal(xd.grad, dx) and torch.equal(w1d.grad, dw1) and torch.equal(w2d.grad, dw2)
    m = fm.FlashMLP(H, D, E, activation="silu", dtype=torch.bfloat16, device="cuda", accurate_dw=True)
    m(x.cuda()).float().sum().backward()
    assert m.w1.grad is not None and torch.isfinite(m.w1.grad.float()).all()
