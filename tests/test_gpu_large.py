"""Maximum sizes: (H, B, D) tensors past 2^32 bytes (more than 2^31 elements), through the tuned
kernels and the C ABI, so that every address the kernels form for the last rows of the last
head lies beyond what 32-bit element or byte offsets can reach.

Inputs are drawn on the GPU (seeded). dO is zero except on a set S of rows per head (the first
rows, rows around 2^23, the last rows): rows with dO = 0 have dH = 0 and dZ = 0, so they add
exactly nothing to dW1 = X^T dZ and dW2 = h^T dO and their dX rows are exactly zero. That makes
the full-size dW equal to the oracle's dW over the rows in S alone, which the CPU oracle computes
in seconds (rows are independent: flashmlp.py:82-85, 360-365). Checks, at the bars of
test_gpu_parity.py:
  * O on the rows of S (first, middle, last) against the fp32 oracle and the cast-point emulation;
  * dX on S against the fp32 oracle, and every other dX row exactly zero;
  * dW1, dW2 elementwise against the emulation over S, normwise against fp32.
Cases: D = 64 fp16 sigmoid and D = 128 bf16 SiLU with B past 2^24 (recompute form: one head's
dZ image would exceed 2 GB, so the plan cannot store it); a four-head D = 128 shape forced into
the stored-dZ form (FMLP_BWD_STORE_DZ), whose dZ workspace also passes 2^32 bytes; fp32 io on the
generic kernels (normwise 1e-4 against fp32, the north star's bar for fp32 sums); and X as a
transposed view of a (B, H, D) tensor through fmlp_fwd_strided / fmlp_bwd_strided (generic
kernels reading the view in place, row stride H D).
"""
import ctypes
import sys

import pytest
import torch

from oracle import emulate, reference

pytestmark = pytest.mark.gpu

ATOL = 3e-2
RTOL = 3e-2
ACT = {"": 0, "silu": 1, "leaky_relu": 2, "sigmoid": 3}

# name, H, B, D, E, dtype, activation, kind: "api" (the Python API), "stored_dz" (C ABI with
# FMLP_BWD_STORE_DZ), "strided" (C ABI *_strided with X a transposed view)
CASES = [
    ("d64_fp16_sigmoid", 2, (1 << 24) + 129, 64, 128, torch.float16, "sigmoid", "api"),
    ("d128_bf16_silu", 2, (1 << 24) + 129, 128, 256, torch.bfloat16, "silu", "api"),
    ("d128_bf16_silu_stored_dz", 4, (1 << 22) + 65, 128, 128, torch.bfloat16, "silu", "stored_dz"),
    ("d32_fp32_leaky_generic", 2, (1 << 25) + 33, 32, 64, torch.float32, "leaky_relu", "api"),
    ("d64_fp16_silu_strided_x", 2, (1 << 24) + 129, 64, 64, torch.float16, "silu", "strided"),
]
CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fail_frac(a, b):
    a, b = a.float(), b.float()
    return ((a - b).abs() > ATOL + RTOL * b.abs()).float().mean().item()


def _normrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _rows(B):
    mid = 1 << 23 if B > (1 << 23) + 64 else B // 2
    return sorted(set(range(64)) | set(range(mid - 32, mid + 32)) | set(range(B - 200, B)))


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_past_32bit_offsets(case):
    import flashmlp_amd as fm
    from flashmlp_amd import _lib

    name, H, B, D, E, dt, act, kind = CASES[case]
    elems, esz = H * B * D, torch.finfo(dt).bits // 8
    assert elems * esz > (1 << 32), "the case must reach past 2^32 bytes"
    _say(f"[large] {name}: H={H} B={B} D={D} E={E} {dt} act='{act}' {kind} "
         f"({elems * esz / 2**30:.2f} GiB per (H, B, D) tensor)")
    gen = torch.Generator(device="cuda").manual_seed(1234 + case)
    if kind == "strided":  # (H, B, D) view of a (B, H, D) tensor: strides (D, H D, 1)
        x = torch.randn(B, H, D, generator=gen, device="cuda", dtype=dt).transpose(0, 1)
        assert not x.is_contiguous()
    else:
        x = torch.randn(H, B, D, generator=gen, device="cuda", dtype=dt)
    w1 = (torch.randn(H, D, E, generator=gen, device="cuda", dtype=torch.float32) / D ** 0.5).to(dt)
    w2 = (torch.randn(H, E, D, generator=gen, device="cuda", dtype=torch.float32) / E ** 0.5).to(dt)
    S = _rows(B)
    s_idx = torch.tensor(S, device="cuda")
    do = torch.zeros(H, B, D, device="cuda", dtype=dt)
    do[:, s_idx] = torch.randn(H, len(S), D, generator=gen, device="cuda", dtype=dt)

    L = _lib.lib()
    code = CODES[dt]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if kind == "strided":
        o = torch.empty(H, B, D, device="cuda", dtype=dt)
        _lib.check(L.fmlp_fwd_strided(_p(x), _p(w1), _p(w2), _p(o), H, B, D, E, _lib.strides(x), _lib.strides(w1),
                                      _lib.strides(w2), code, ACT[act], stream), "forward (strided)")
    else:
        o = fm.flashmlp_fwd(x, w1, w2, act)
    torch.cuda.synchronize()
    _say(f"[large] {name}: forward done")
    if kind == "strided":
        dx, dw1, dw2 = torch.empty(H, B, D, device="cuda", dtype=dt), torch.empty_like(w1), torch.empty_like(w2)
        nbytes = 64 << 20  # the generic dW programs split B as far as it allows
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        st = L.fmlp_bwd_strided(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E,
                                _lib.strides(x), _lib.strides(w1), _lib.strides(w2), _lib.strides(do), code,
                                ACT[act], _p(ws), nbytes, stream)
        _lib.check(st, "backward (strided)")
        del ws
    elif kind == "stored_dz":
        flags = code | _lib.FMLP_BWD_STORE_DZ
        assert L.fmlp_bwd_stores_dz(H, B, D, E, flags, ACT[act]) == 1
        nbytes = L.fmlp_bwd_workspace_bytes(H, B, D, E, flags)
        assert nbytes > (1 << 32), "the dZ workspace must reach past 2^32 bytes"
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        dx, dw1, dw2 = torch.empty_like(x), torch.empty_like(w1), torch.empty_like(w2)
        st = L.fmlp_bwd(_p(x), _p(w1), _p(w2), _p(do), _p(dx), _p(dw1), _p(dw2), H, B, D, E, flags, ACT[act],
                        _p(ws), nbytes, stream)
        _lib.check(st, "backward")
        del ws
    else:
        dx, dw1, dw2 = fm.flashmlp_bwd(x, w1, w2, do, act)
    torch.cuda.synchronize()
    _say(f"[large] {name}: backward done")

    # dX rows outside S are exactly zero (their dO, hence dZ, is zero)
    row_max = torch.maximum(dx.amax(dim=2).float().abs(), dx.amin(dim=2).float().abs())
    row_max[:, s_idx] = 0
    assert row_max.max().item() == 0.0, "dX rows whose dO is zero must be zero"
    del row_max

    xs, dos = x[:, s_idx].cpu(), do[:, s_idx].cpu()
    w1c, w2c = w1.cpu(), w2.cpu()
    os_, dxs = o[:, s_idx].cpu(), dx[:, s_idx].cpu()
    dw1c, dw2c = dw1.cpu(), dw2.cpu()
    del x, do, o, dx
    torch.cuda.empty_cache()

    ro, rdx, rdw1, rdw2 = reference.autograd_grads(xs, w1c, w2c, dos, act)
    if dt == torch.float32:  # fp32 io: no io rounding anywhere, normwise 1e-4 against fp32
        res = {"o_rel": _normrel(os_, ro), "dx_rel": _normrel(dxs, rdx), "dw1_rel": _normrel(dw1c, rdw1),
               "dw2_rel": _normrel(dw2c, rdw2), "o_last_rows_rel": _normrel(os_[:, -200:], ro[:, -200:])}
        _say(f"[large] {name}: " + " ".join(f"{k}={v:.3g}" for k, v in res.items()))
        assert all(v < 1e-4 for v in res.values()), res
        return
    eo = emulate.emu_fwd(xs, w1c, w2c, act, dt)
    _, edw1, edw2 = emulate.emu_bwd(xs, w1c, w2c, dos, act, dt)
    res = {
        "o_fail": _fail_frac(os_, ro), "o_emu_fail": _fail_frac(os_, eo), "dx_fail": _fail_frac(dxs, rdx),
        "dw1_emu_fail": _fail_frac(dw1c, edw1), "dw2_emu_fail": _fail_frac(dw2c, edw2),
        "dw1_rel": _normrel(dw1c, rdw1), "dw2_rel": _normrel(dw2c, rdw2),
        "o_last_rows_rel": _normrel(os_[:, -200:], ro[:, -200:]),
    }
    _say(f"[large] {name}: " + " ".join(f"{k}={v:.3g}" for k, v in res.items()))
    assert res["o_fail"] == 0.0 and res["o_emu_fail"] == 0.0 and res["dx_fail"] == 0.0
    assert res["dw1_emu_fail"] == 0.0 and res["dw2_emu_fail"] == 0.0
    assert res["dw1_rel"] < 1e-2 and res["dw2_rel"] < 1e-2 and res["o_last_rows_rel"] < 1e-2
