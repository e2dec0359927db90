"""torch.library registration of the FlashMLP operators, checked without a GPU: schemas,
fake (meta) kernels under FakeTensorMode, the reference's shape messages from the fake
kernels, and no CPU kernel (CPU tensors raise instead of falling back)."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import flashmlp_amd  # noqa: F401  (registers torch.ops.flashmlp_amd)


def test_schemas():
    assert str(torch.ops.flashmlp_amd.fwd.default._schema) == (
        'flashmlp_amd::fwd(Tensor x, Tensor w1, Tensor w2, str activation="", bool accurate_dw=False) -> Tensor')
    assert str(torch.ops.flashmlp_amd.bwd.default._schema) == (
        'flashmlp_amd::bwd(Tensor x, Tensor w1, Tensor w2, Tensor do, str activation="", bool accurate_dw=False) '
        '-> (Tensor, Tensor, Tensor)')


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fake_shapes(dtype):
    with FakeTensorMode():
        x = torch.empty(3, 200, 128, dtype=dtype, device="cuda")
        w1 = torch.empty(3, 128, 96, dtype=dtype, device="cuda")
        w2 = torch.empty(3, 96, 128, dtype=dtype, device="cuda")
        o = torch.ops.flashmlp_amd.fwd(x, w1, w2, "silu")
        dx, dw1, dw2 = torch.ops.flashmlp_amd.bwd(x, w1, w2, o, "silu")
    assert o.shape == x.shape and o.dtype == dtype and o.device.type == "cuda"
    assert (dx.shape, dw1.shape, dw2.shape) == (x.shape, w1.shape, w2.shape)
    assert dx.dtype == dw1.dtype == dw2.dtype == dtype


@pytest.mark.parametrize(
    "w1s,w2s,dos,msg",
    [
        ((2, 64, 96), (3, 96, 64), (3, 10, 64), "Number of heads must match"),
        ((3, 32, 96), (3, 96, 64), (3, 10, 64), "Hidden dimension mismatch"),
        ((3, 64, 96), (3, 80, 64), (3, 10, 64), "Intermediate dimension mismatch"),
        ((3, 64, 96), (3, 96, 32), (3, 10, 64), "Output dimension mismatch"),
        ((3, 64, 96), (3, 96, 64), (3, 11, 64), "Gradient shape mismatch"),
    ],
)
def test_fake_shape_checks(w1s, w2s, dos, msg):
    with FakeTensorMode():
        x = torch.empty(3, 10, 64, dtype=torch.bfloat16, device="cuda")
        w1 = torch.empty(*w1s, dtype=torch.bfloat16, device="cuda")
        w2 = torch.empty(*w2s, dtype=torch.bfloat16, device="cuda")
        do = torch.empty(*dos, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(RuntimeError, match=msg):
            if msg == "Gradient shape mismatch":
                torch.ops.flashmlp_amd.bwd(x, w1, w2, do, "")
            else:
                torch.ops.flashmlp_amd.fwd(x, w1, w2, "")


def test_no_cpu_kernel():
    x = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    w1 = torch.zeros(2, 64, 16, dtype=torch.bfloat16)
    w2 = torch.zeros(2, 16, 64, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        torch.ops.flashmlp_amd.fwd(x, w1, w2, "silu")
