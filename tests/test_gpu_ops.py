"""The registered operators on the GPU: torch.library.opcheck (schema, fake kernel against
the real one, autograd registration, AOT dispatch), torch.compile through AOTAutograd
(backend "aot_eager", so the compiled graph runs the same HIP kernels) against eager, and
the compiled operator path against the CPU oracle at the parity bars of test_gpu_parity."""
import sys

import pytest
import torch

import flashmlp_amd as fm
from oracle import emulate, reference
from oracle.inputs import make_inputs

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("act", ["", "silu"])
def test_opcheck(act):
    _say(f"[ops] opcheck act='{act}'")
    x, w1, w2, do = (t.cuda() for t in make_inputs(2, 70, 64, 96, torch.bfloat16, seed=5))
    torch.library.opcheck(torch.ops.flashmlp_amd.fwd.default, (x, w1, w2, act))
    torch.library.opcheck(torch.ops.flashmlp_amd.bwd.default, (x, w1, w2, do, act))
    xg, w1g, w2g = (t.clone().requires_grad_(True) for t in (x, w1, w2))
    torch.library.opcheck(torch.ops.flashmlp_amd.fwd.default, (xg, w1g, w2g, act),
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


def _loss_and_grads(fn, x, w1, w2, do):
    xg, w1g, w2g = (t.clone().requires_grad_(True) for t in (x, w1, w2))
    o = fn(xg, w1g, w2g)
    o.backward(do)
    return o.detach(), xg.grad, w1g.grad, w2g.grad


@pytest.mark.parametrize("act", ["silu", "leaky_relu"])
def test_compile_matches_eager(act):
    _say(f"[ops] torch.compile aot_eager act='{act}'")
    x, w1, w2, do = (t.cuda() for t in make_inputs(3, 300, 128, 256, torch.bfloat16, seed=6))

    def f(a, b, c):
        return fm.flashmlp(a, b, c, act)

    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)
    got = _loss_and_grads(compiled, x, w1, w2, do)
    ref = _loss_and_grads(lambda a, b, c: fm.FlashMLPFunction.apply(a, b, c, act), x, w1, w2, do)
    torch.cuda.synchronize()
    for g, r in zip(got, ref):
        assert torch.equal(g, r)  # same kernels, same inputs: bit-identical


def test_compiled_module_matches_eager():
    _say("[ops] torch.compile FlashMLP module")
    torch.manual_seed(0)
    m = fm.FlashMLP(4, 64, 192, activation="silu", dtype=torch.bfloat16, device="cuda")
    x = torch.randn(4, 257, 64, dtype=torch.bfloat16, device="cuda")
    cm = torch.compile(m, backend="aot_eager", fullgraph=True)
    o_c = cm(x)
    o_c.float().pow(2).sum().backward()
    g_c = (m.w1.grad.clone(), m.w2.grad.clone())
    m.zero_grad()
    o_e = m(x)
    o_e.float().pow(2).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(o_c, o_e)
    assert torch.equal(g_c[0], m.w1.grad) and torch.equal(g_c[1], m.w2.grad)


@pytest.mark.parametrize("dt,act", [(torch.bfloat16, "silu"), (torch.float16, "sigmoid"), (torch.bfloat16, "leaky_relu")],
                         ids=["bf16-silu", "f16-sigmoid", "bf16-leaky"])
def test_compiled_op_matches_oracle(dt, act):
    # O and dX elementwise against fp32 autograd; dW1, dW2 elementwise against the
    # cast-point emulation and normwise (1e-2) against fp32, through the traced operator
    _say(f"[ops] compiled operator vs oracle {dt} act='{act}'")
    x, w1, w2, do = make_inputs(3, 333, 128, 264, dt, seed=13)
    compiled = torch.compile(lambda a, b, c: fm.flashmlp(a, b, c, act), backend="aot_eager", fullgraph=True)
    o, dx, dw1, dw2 = (t.float().cpu() for t in _loss_and_grads(compiled, *(t.cuda() for t in (x, w1, w2, do))))
    ro, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
    _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
    close = lambda a, b: bool(((a - b).abs() <= 3e-2 + 3e-2 * b.abs()).all())
    rel = lambda a, b: ((a - b).norm() / b.norm()).item()
    assert close(o, ro) and close(dx, rdx)
    assert close(dw1, edw1) and close(dw2, edw2)
    assert rel(dw1, rdw1) <= 1e-2 and rel(dw2, rdw2) <= 1e-2
