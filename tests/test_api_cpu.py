"""Python API behaviour that needs no GPU: the reference's assertion messages, loud failure
off the GPU (no CPU fallback), module parameters, and the unfused baseline API."""
import pytest
import torch

import flashmlp_amd as fm
from oracle import reference
from oracle.inputs import make_inputs


def _t(*shape):
    return torch.zeros(*shape, dtype=torch.bfloat16)


@pytest.mark.parametrize(
    "x,w1,w2,msg",
    [
        (_t(2, 4, 8), _t(3, 8, 16), _t(2, 16, 8), "Number of heads must match"),
        (_t(2, 4, 8), _t(2, 8, 16), _t(3, 16, 8), "Number of heads must match"),
        (_t(2, 4, 8), _t(2, 6, 16), _t(2, 16, 8), "Hidden dimension mismatch"),
        (_t(2, 4, 8), _t(2, 8, 16), _t(2, 12, 8), "Intermediate dimension mismatch"),
        (_t(2, 4, 8), _t(2, 8, 16), _t(2, 16, 6), "Output dimension mismatch"),
    ],
)
def test_forward_shape_asserts(x, w1, w2, msg):
    # flashmlp.py:443-447
    with pytest.raises(AssertionError, match=msg):
        fm.flashmlp_fwd(x, w1, w2, "silu")


def test_backward_shape_asserts():
    # flashmlp.py:496-499, plus the head-count check the reference omits
    x, w1, w2 = _t(2, 4, 8), _t(2, 8, 16), _t(2, 16, 8)
    with pytest.raises(AssertionError, match="Gradient shape mismatch"):
        fm.flashmlp_bwd(x, w1, w2, _t(2, 5, 8), "silu")
    with pytest.raises(AssertionError, match="Number of heads must match"):
        fm.flashmlp_bwd(x, _t(3, 8, 16), w2, _t(2, 4, 8), "silu")


def test_no_cpu_fallback():
    x, w1, w2, do = make_inputs(2, 16, 64, 64, torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        fm.flashmlp_fwd(x, w1, w2, "silu")
    with pytest.raises(RuntimeError, match="GPU"):
        fm.flashmlp_bwd(x, w1, w2, do, "silu")
    with pytest.raises(RuntimeError, match="GPU"):
        fm.FlashMLPFunction.apply(x, w1, w2, "silu")


def test_fast_path_declines_what_it_does_not_take():
    """The wrappers' fast path (_fmlp_fast, built with the library) returns None for anything but
    16-bit GPU tensors of a tuned shape, so the general path validates and raises."""
    import importlib

    fmm = importlib.import_module("flashmlp_amd.flashmlp")
    assert fmm._fast is not None, "_fmlp_fast.so is not built"
    x, w1, w2, do = make_inputs(2, 16, 64, 64, torch.bfloat16)
    assert fmm._fast.fwd(x, w1, w2, 1) is None
    assert fmm._fast.bwd(x, w1, w2, do, 1, 0) is None
    assert fmm._fast.fwd(x.float(), w1.float(), w2.float(), 1) is None
    assert fmm._fast.fwd(x, w1, "not a tensor", 1) is None
    with pytest.raises(TypeError):
        fmm._fast.fwd(x, w1, w2)


def test_module_parameters_match_reference_layout():
    # flashmlp.py:577-591: parameter names, shapes, dtype and init scales
    torch.manual_seed(0)
    m = fm.FlashMLP(num_heads=4, hidden_dim=64, intermediate_dim=256, activation="silu", dtype=torch.float32,
                    device="cpu")
    sd = m.state_dict()
    assert list(sd) == ["w1", "w2"]
    assert sd["w1"].shape == (4, 64, 256) and sd["w2"].shape == (4, 256, 64)
    assert abs(sd["w1"].std().item() - 256 ** -0.5) < 0.01
    assert abs(sd["w2"].std().item() - 64 ** -0.5) < 0.01
    assert m.activation == "silu" and m.num_heads == 4
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(4, 8, 64))


def test_module_default_dtype_is_fp16():
    m = fm.FlashMLP(2, 64, 64, device="cpu")
    assert m.w1.dtype == torch.float16 and m.activation == "silu"


@pytest.mark.parametrize("act", ["", "silu", "leaky_relu", "sigmoid"])
def test_unfused_baseline_api(act):
    x, w1, w2, do = make_inputs(2, 24, 64, 96, torch.float32, seed=11)
    o = fm.flashmlp_torch_fwd(x, w1, w2, act)
    ro, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    torch.testing.assert_close(o, ro)
    dx, dw1, dw2 = fm.flashmlp_torch_bwd(x, w1, w2, do, act)
    for a, b in ((dx, rdx), (dw1, rdw1), (dw2, rdw2)):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5)
    m = fm.PyTorchMLP(2, 64, 96, activation=act, dtype=torch.float32, device="cpu")
    with torch.no_grad():
        m.w1.copy_(w1)
        m.w2.copy_(w2)
    torch.testing.assert_close(m(x), ro)
    # 2-D input: expanded to every head, mean over heads (flashmlp.py:642-663)
    x2 = x[0]
    torch.testing.assert_close(m(x2), reference.torch_fwd(x2.expand(2, -1, -1), w1, w2, act).mean(0))
