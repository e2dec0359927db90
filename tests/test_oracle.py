"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

The reference ships no golden vectors or known-answer tests for this path (its in-file
tests only print). Each oracle function is pinned here by checks chosen so that a
plausible mistake (dropped term, wrong sign, transposed operand, wrong derivative at a
kink) fails at least one of them:
  * an independent fp64 C brute force (oracle/brute.c) on tiny shapes, all activations;
  * torch.autograd.gradcheck of the restatement in fp64;
  * closed forms of the linear activation: O = X (W1 W2), dX = dO W2^T W1^T,
    dW1 = X^T dO W2^T, dW2 = (X W1)^T dO;
  * derivative values at the kinks (leaky'(0) = 0.01 as autograd, silu'(0) = 1/2,
    sigmoid'(0) = 1/4) and saturation (silu'(+20) = 1, sigmoid(+-30) = 1, 0);
  * invariants: heads independent, rows independent for O and dX, leaky == linear when
    every Z > 0, the manual backward equals autograd except leaky at Z == 0;
  * the cast-point emulation equals the restatement when the io dtype is fp32, and a
    planted missing cast (h not rounded) is detected against it.
"""
import numpy as np
import pytest
import torch

from oracle import emulate, reference
from oracle.build import brute_bwd, brute_fwd
from oracle.inputs import CONFIGS, make_inputs

ACTS = ["", "silu", "leaky_relu", "sigmoid"]


def _f64(*ts):
    return [t.detach().to(torch.float64) for t in ts]


@pytest.mark.parametrize("act", ACTS)
def test_restatement_matches_c_brute_force(act):
    torch.manual_seed(3)
    H, B, D, E = 2, 5, 16, 16
    x, w1, w2, do = (torch.randn(s, dtype=torch.float64) for s in ((H, B, D), (H, D, E), (H, E, D), (H, B, D)))
    o, dx, dw1, dw2 = reference.autograd_grads(x, w1, w2, do, act, dtype=torch.float64)
    bo = brute_fwd(x.numpy(), w1.numpy(), w2.numpy(), act)
    bdx, bdw1, bdw2 = brute_bwd(x.numpy(), w1.numpy(), w2.numpy(), do.numpy(), act)
    for a, b in ((o, bo), (dx, bdx), (dw1, bdw1), (dw2, bdw2)):
        np.testing.assert_allclose(a.numpy(), b, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("act", ACTS)
def test_restatement_gradcheck(act):
    torch.manual_seed(4)
    H, B, D, E = 2, 3, 4, 5
    x = torch.randn(H, B, D, dtype=torch.float64, requires_grad=True)
    w1 = torch.randn(H, D, E, dtype=torch.float64, requires_grad=True)
    w2 = torch.randn(H, E, D, dtype=torch.float64, requires_grad=True)
    # random fp64 inputs do not land on the leaky kink (Z == 0), where the derivative is one-sided
    assert torch.autograd.gradcheck(lambda a, b, c: reference.torch_fwd(a, b, c, act), (x, w1, w2))


def test_linear_closed_forms():
    torch.manual_seed(5)
    H, B, D, E = 3, 7, 8, 12
    x, w1, w2, do = _f64(*(torch.randn(s) for s in ((H, B, D), (H, D, E), (H, E, D), (H, B, D))))
    o, dx, dw1, dw2 = reference.autograd_grads(x, w1, w2, do, "", dtype=torch.float64)
    torch.testing.assert_close(o, x @ (w1 @ w2))
    torch.testing.assert_close(dx, do @ w2.transpose(1, 2) @ w1.transpose(1, 2))
    torch.testing.assert_close(dw1, x.transpose(1, 2) @ (do @ w2.transpose(1, 2)))
    torch.testing.assert_close(dw2, (x @ w1).transpose(1, 2) @ do)


def test_derivatives_at_kinks_and_saturation():
    def grad_at(z, act):
        # one head, D = E = 1, w1 = w2 = 1, do = 1 -> dX = act'(z)
        x = torch.tensor([[[z]]], dtype=torch.float64)
        one = torch.ones(1, 1, 1, dtype=torch.float64)
        _, dx, _, _ = reference.autograd_grads(x, one, one, one, act, dtype=torch.float64)
        return dx.item()

    assert grad_at(0.0, "leaky_relu") == pytest.approx(0.01)
    assert grad_at(-1.0, "leaky_relu") == pytest.approx(0.01)
    assert grad_at(1.0, "leaky_relu") == pytest.approx(1.0)
    assert grad_at(0.0, "silu") == pytest.approx(0.5)
    assert grad_at(20.0, "silu") == pytest.approx(1.0, abs=1e-6)
    assert grad_at(0.0, "sigmoid") == pytest.approx(0.25)
    assert grad_at(30.0, "sigmoid") == pytest.approx(0.0, abs=1e-12)
    x = torch.tensor([[[30.0], [-30.0]]], dtype=torch.float64)
    one = torch.ones(1, 1, 1, dtype=torch.float64)
    o = reference.torch_fwd(x, one, one, "sigmoid")
    assert o[0, 0, 0].item() == pytest.approx(1.0) and o[0, 1, 0].item() == pytest.approx(0.0, abs=1e-12)


@pytest.mark.parametrize("act", ACTS)
def test_heads_and_rows_independent(act):
    x, w1, w2, do = make_inputs(4, 9, 16, 24, torch.float32, seed=6)
    o, dx, dw1, dw2 = reference.autograd_grads(x, w1, w2, do, act)
    perm = torch.tensor([2, 0, 3, 1])
    po, pdx, pdw1, pdw2 = reference.autograd_grads(x[perm], w1[perm], w2[perm], do[perm], act)
    for a, b in ((o[perm], po), (dx[perm], pdx), (dw1[perm], pdw1), (dw2[perm], pdw2)):
        torch.testing.assert_close(a, b)
    # rows: O and dX of a row depend on that row only
    so, sdx, _, _ = reference.autograd_grads(x[:, 3:5], w1, w2, do[:, 3:5], act)
    torch.testing.assert_close(so, o[:, 3:5])
    torch.testing.assert_close(sdx, dx[:, 3:5])


def test_leaky_equals_linear_when_all_positive():
    torch.manual_seed(7)
    H, B, D, E = 2, 6, 8, 10
    x = torch.rand(H, B, D, dtype=torch.float64) + 0.1
    w1 = torch.rand(H, D, E, dtype=torch.float64) + 0.1
    w2 = torch.randn(H, E, D, dtype=torch.float64)
    do = torch.randn(H, B, D, dtype=torch.float64)
    a = reference.autograd_grads(x, w1, w2, do, "leaky_relu", dtype=torch.float64)
    b = reference.autograd_grads(x, w1, w2, do, "", dtype=torch.float64)
    for u, v in zip(a, b):
        torch.testing.assert_close(u, v)


@pytest.mark.parametrize("act", ACTS)
def test_manual_backward_matches_autograd(act):
    x, w1, w2, do = make_inputs(2, 17, 16, 24, torch.float32, seed=8)
    x, w1, w2, do = _f64(x, w1, w2, do)
    _, dx, dw1, dw2 = reference.autograd_grads(x, w1, w2, do, act, dtype=torch.float64)
    mdx, mdw1, mdw2 = reference.manual_bwd(x, w1, w2, do, act)
    for a, b in ((dx, mdx), (dw1, mdw1), (dw2, mdw2)):
        torch.testing.assert_close(a, b)


def test_manual_backward_leaky_kink_differs_from_autograd():
    # X rows of zeros make Z == 0 exactly: the reference's manual backward uses slope 1
    # there (flashmlp.py:710), autograd 0.01; dX differs by a factor of 100
    H, B, D, E = 1, 2, 4, 3
    x = torch.zeros(H, B, D, dtype=torch.float64)
    w1 = torch.randn(H, D, E, dtype=torch.float64)
    w2 = torch.randn(H, E, D, dtype=torch.float64)
    do = torch.randn(H, B, D, dtype=torch.float64)
    _, dx, _, _ = reference.autograd_grads(x, w1, w2, do, "leaky_relu", dtype=torch.float64)
    mdx, _, _ = reference.manual_bwd(x, w1, w2, do, "leaky_relu")
    torch.testing.assert_close(mdx, dx * 100)


@pytest.mark.parametrize("act", ACTS)
def test_emulation_reduces_to_restatement_in_fp32(act):
    x, w1, w2, do = make_inputs(2, 33, 64, 96, torch.float32, seed=9)
    o, dx, dw1, dw2 = reference.autograd_grads(x, w1, w2, do, act)
    eo = emulate.emu_fwd(x, w1, w2, act, torch.float32)
    edx, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, torch.float32)
    for a, b in ((o, eo), (dx, edx), (dw1, edw1), (dw2, edw2)):
        torch.testing.assert_close(a, b, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("act", ACTS)
def test_emu_fwd_matches_blockwise_program(act, dt):
    # emu_fwd against the tile-by-tile restatement of the reference's forward program
    # (flashmlp.py:130-157): same cast points, different summation order
    from oracle import blockwise

    x, w1, w2, _ = make_inputs(2, 200, 64, 320, dt, x_std=2.0 if act == "sigmoid" else 1.0, seed=13, with_do=False)
    e = emulate.emu_fwd(x, w1, w2, act, dt, round_out=False)
    b = blockwise.fwd_blocks(x, w1, w2, act, dt, round_out=False)
    assert _rel(e, b) < 2e-5


@pytest.mark.parametrize("act", ["silu", "sigmoid", "leaky_relu"])
def test_planted_fwd_cast_positions_are_detected(act):
    # the forward rounds h = act(z) to the io dtype, not z before the activation and not only
    # o at the end: each planted position moves o far beyond the fp32 noise that separates
    # emu_fwd from the blockwise program (leaky_relu commutes with the rounding of z, so only
    # the missing cast is observable there)
    from oracle import blockwise

    dt = torch.bfloat16
    x, w1, w2, _ = make_inputs(2, 256, 64, 256, dt, seed=14, with_do=False)
    ref = blockwise.fwd_blocks(x, w1, w2, act, dt, round_out=False)
    assert _rel(emulate.emu_fwd(x, w1, w2, act, dt, round_out=False), ref) < 2e-5
    xs, a, b = (t.float() for t in (x, w1, w2))
    z = torch.bmm(xs, a)
    q = lambda t: t.to(dt).float()
    z_first = torch.bmm(q(emulate._h(q(z), act)), b)   # z rounded before the activation too
    z_only = torch.bmm(emulate._h(q(z), act), b)       # z rounded instead of h
    no_cast = torch.bmm(emulate._h(z, act), b)         # h kept in fp32
    assert _rel(no_cast, ref) > 5e-4
    if act != "leaky_relu":
        assert _rel(z_first, ref) > 5e-4
        assert _rel(z_only, ref) > 5e-4


def test_emulation_cast_point_is_observable():
    # the emulation rounds h to the io dtype before the second product; a planted variant
    # without that cast must differ from it by more than the fp32 summation noise
    x, w1, w2, _ = make_inputs(2, 64, 64, 256, torch.bfloat16, seed=10)
    eo = emulate.emu_fwd(x, w1, w2, "silu", torch.bfloat16, round_out=False)
    xs, a, b = (t.float() for t in (x, w1, w2))
    planted = torch.bmm(torch.nn.functional.silu(torch.bmm(xs, a)), b)  # no cast of h
    rel = ((eo - planted).norm() / planted.norm()).item()
    assert rel > 1e-4


def test_config_table_matches_baseline():
    c = CONFIGS["cfg4"]
    assert (c.H, c.B, c.D, c.E, c.dtype, c.activation) == (32, 16384, 128, 1024, torch.bfloat16, "silu")
    c = CONFIGS["cfg3"]
    assert (c.H, c.B, c.D, c.E, c.dtype, c.activation) == (16, 8192, 128, 512, torch.bfloat16, "leaky_relu")
    c = CONFIGS["cfg5_sigmoid"]
    assert (c.H, c.B, c.D, c.E, c.x_std) == (8, 4097, 64, 2048, 2.0)


def test_inputs_seeded_and_scaled():
    x, w1, w2, do = make_inputs(2, 4096, 128, 512, torch.float32, seed=0)
    x2, _, _, _ = make_inputs(2, 4096, 128, 512, torch.float32, seed=0)
    assert torch.equal(x, x2)
    assert abs(x.std().item() - 1.0) < 0.02
    assert abs(w1.std().item() - 128 ** -0.5) < 0.005
    assert abs(w2.std().item() - 512 ** -0.5) < 0.002
    assert abs(do.std().item() - 1.0) < 0.02


# ---- emu_bwd's cast points, pinned against the blockwise restatement of the reference's
# backward programs (oracle/blockwise.py follows flashmlp.py:165-329 tile by tile) ----

def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("act", ACTS)
def test_emu_bwd_matches_blockwise_programs(act, dt):
    # same cast points, different tiling and summation order: only fp32 rounding noise
    from oracle import blockwise

    x, w1, w2, do = make_inputs(2, 256, 64, 256, dt, seed=11)
    e = emulate.emu_bwd(x, w1, w2, do, act, dt, round_out=False)
    b = blockwise.bwd_blocks(x, w1, w2, do, act, dt, deriv="fp32", round_out=False)
    for u, v in zip(e, b):
        assert _rel(u, v) < 2e-5
    # rounded outputs: a summation-order difference can flip an output's last io bit
    ulp = 2.0 ** -7 if dt == torch.bfloat16 else 2.0 ** -10
    e = emulate.emu_bwd(x, w1, w2, do, act, dt)
    b = blockwise.bwd_blocks(x, w1, w2, do, act, dt, deriv="fp32")
    for u, v in zip(e, b):
        diff = (u - v).abs()
        assert (diff > 0).float().mean().item() < 0.01
        # small outputs are sums with cancellation, where fp32 order noise can reach two io ulps
        rms = v.pow(2).mean().sqrt()
        assert (diff <= 2 * ulp * v.abs() + 1e-4 * rms).all()


def _planted(x, w1, w2, do, act, dt, variant):
    """emu_bwd with one cast point planted wrong (each is a plausible emulation mistake)."""
    xs, a, b, g = (t.float() for t in (x, w1, w2, do))
    z = torch.bmm(xs, a)
    dh = torch.bmm(g, b.transpose(1, 2))
    q = lambda t: t.to(dt).float()
    h = emulate._h(z, act)
    dz = emulate._dz(z, dh, act)
    if variant == "no_h_cast":
        dz = q(dz)
    elif variant == "no_dz_cast":
        h = q(h)
    elif variant == "dh_cast_not_dz":
        h, dz = q(h), emulate._dz(z, q(dh), act)
    return torch.bmm(dz, a.transpose(1, 2)), torch.bmm(xs.transpose(1, 2), dz), torch.bmm(h.transpose(1, 2), g)


@pytest.mark.parametrize("act", ["silu", "sigmoid"])
@pytest.mark.parametrize("variant,moved", [("no_h_cast", (2,)), ("no_dz_cast", (0, 1)), ("dh_cast_not_dz", (0, 1))])
def test_planted_bwd_cast_mistakes_are_detected(act, variant, moved):
    # each planted variant moves the outputs its cast feeds by far more than the 1e-4 bar of
    # the fp32-sum tests, while emu_bwd stays within fp32 noise of the blockwise programs
    from oracle import blockwise

    dt = torch.bfloat16
    x, w1, w2, do = make_inputs(2, 256, 64, 256, dt, seed=12)
    ref = blockwise.bwd_blocks(x, w1, w2, do, act, dt, deriv="fp32", round_out=False)
    good = emulate.emu_bwd(x, w1, w2, do, act, dt, round_out=False)
    bad = _planted(x, w1, w2, do, act, dt, variant)
    for i in range(3):
        assert _rel(good[i], ref[i]) < 2e-5
        if i in moved:
            assert _rel(bad[i], ref[i]) > 5e-4, (variant, i)
        else:
            assert _rel(bad[i], ref[i]) < 2e-5, (variant, i)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("act", ["silu", "sigmoid"])
def test_fp32_derivative_is_closer_to_autograd_than_rounded_h(act, dt):
    # the kernels (and emu_bwd) evaluate SiLU's and sigmoid's derivative from the fp32
    # sigmoid; the reference kernel uses the io-rounded h (flashmlp.py:230-233, :315-318).
    # Both round dZ to the io dtype; against the fp32 autograd oracle the fp32 form is the
    # closer of the two, and they differ by ~1e-3 (bf16) normwise in dX and dW1.
    from oracle import blockwise

    x, w1, w2, do = make_inputs(2, 256, 64, 256, dt, seed=11)
    _, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    f = blockwise.bwd_blocks(x, w1, w2, do, act, dt, deriv="fp32", round_out=False)
    r = blockwise.bwd_blocks(x, w1, w2, do, act, dt, deriv="reference", round_out=False)
    assert _rel(f[0], rdx) < _rel(r[0], rdx)
    assert _rel(f[1], rdw1) < _rel(r[1], rdw1)
    assert torch.equal(f[2], r[2])  # dW2 does not involve the derivative


def test_blockwise_reference_derivative_leaky_kink():
    # literal reference derivative: slope 1 at z == 0 (flashmlp.py:33-34); the fp32 form
    # follows autograd (0.01). Zero X rows make every z == 0.
    from oracle import blockwise

    x = torch.zeros(1, 4, 16)
    w1 = torch.randn(1, 16, 8)
    w2 = torch.randn(1, 8, 16)
    do = torch.randn(1, 4, 16)
    r = blockwise.bwd_blocks(x, w1, w2, do, "leaky_relu", torch.float32, deriv="reference", round_out=False)
    f = blockwise.bwd_blocks(x, w1, w2, do, "leaky_relu", torch.float32, deriv="fp32", round_out=False)
    torch.testing.assert_close(r[0], f[0] * 100)
