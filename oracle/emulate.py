"""Cast-point emulation of the reference FlashMLP kernels (test infrastructure only).

All contractions accumulate in fp32 (flashmlp.py:137,150,212,224,238,294,306,309,323 use
out_dtype=float32). Values are rounded to the io dtype exactly where the reference kernels
round them:
  forward  h = act(z).to(io)                 flashmlp.py:141-147;  O.to(io)  :157
  dX path  dz = (dh * act'(z, h)).to(io)     flashmlp.py:227-235;  dX.to(io) :393
  dW path  h.to(io), dz.to(io)               flashmlp.py:297-320;  dW.to(io) :420-421
Derivatives follow autograd (Leaky ReLU slope 0.01 at z == 0) and use the fp32 h for
SiLU's derivative, as the gfx950 kernels do (flashmlp.py:230 uses the rounded h; the
difference is far inside tolerance).

Inputs are io-dtype tensors; outputs are fp32 tensors holding io-dtype-representable
values (the `round_out=False` variants keep the fp32 sums unrounded).
"""
from __future__ import annotations

import torch


def _sig(z):
    return torch.sigmoid(z)


def _h(z, activation):
    if activation == "leaky_relu":
        return torch.where(z > 0, z, 0.01 * z)
    if activation == "silu":
        return z * _sig(z)
    if activation == "sigmoid":
        return _sig(z)
    return z


def _dz(z, dh, activation):
    if activation == "leaky_relu":
        return torch.where(z > 0, dh, 0.01 * dh)
    if activation == "silu":
        s = _sig(z)
        h = z * s
        return dh * (s + h * (1 - s))
    if activation == "sigmoid":
        s = _sig(z)
        return dh * (s - s * s)
    return dh


def _q(t, io_dtype):
    return t.to(io_dtype).to(torch.float32)


def emu_fwd(x, w1, w2, activation="", io_dtype=torch.bfloat16, round_out=True):
    x, w1, w2 = (t.detach().to("cpu", torch.float32) for t in (x, w1, w2))
    z = torch.bmm(x, w1)
    h = _q(_h(z, activation), io_dtype)
    o = torch.bmm(h, w2)
    return _q(o, io_dtype) if round_out else o


def emu_bwd(x, w1, w2, do, activation="", io_dtype=torch.bfloat16, round_out=True):
    x, w1, w2, do = (t.detach().to("cpu", torch.float32) for t in (x, w1, w2, do))
    z = torch.bmm(x, w1)
    dh = torch.bmm(do, w2.transpose(1, 2))
    h = _q(_h(z, activation), io_dtype)
    dz = _q(_dz(z, dh, activation), io_dtype)
    dx = torch.bmm(dz, w1.transpose(1, 2))
    dw1 = torch.bmm(x.transpose(1, 2), dz)
    dw2 = torch.bmm(h.transpose(1, 2), do)
    if round_out:
        dx, dw1, dw2 = _q(dx, io_dtype), _q(dw1, io_dtype), _q(dw2, io_dtype)
    return dx, dw1, dw2
