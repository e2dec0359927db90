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
