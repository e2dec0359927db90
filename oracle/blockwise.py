"""Blockwise restatement of the reference kernels (test infrastructure only).

Follows the loop structure of the reference's forward program and its two backward roles
literally, one tile at a time, with fp32 accumulation and `.to(io)` exactly where the
reference casts:

  forward  flashmlp.py:63-158    per B-block, loop over E-blocks:
           z = x @ w1 (fp32) :137; h = act(z).to(io) :140-147; o += h @ w2 (fp32) :150;
           o.to(io) at the store :157
  dX role  flashmlp.py:165-244   per B-block, loop over E-blocks:
           z = x @ w1 (fp32) :212; h = act(z).to(io) :214-221; dh = do @ w2^T (fp32) :224;
           dz = (dh * act'(z, h)).to(io) :227-235; dx += dz @ w1^T (fp32) :238
  dW role  flashmlp.py:247-329   per E-block, loop over B-blocks:
           z, h, dh as above :294-306; dw2 += h^T @ do (fp32) :309;
           dz = (dh * act'(z, h)).to(io) :312-320; dw1 += x^T @ dz (fp32) :323

`deriv="reference"` evaluates the derivative as the reference kernel does: SiLU's from the
io-rounded h (d_silu(z, h), flashmlp.py:42-46, :230, :315) and sigmoid's as h (1 - h) with
the rounded h (:231-233, :316-318); Leaky ReLU's slope at z == 0 is 1 (:33-34).
`deriv="fp32"` uses the unrounded fp32 sigmoid (and autograd's Leaky ReLU slope 0.01 at
z == 0), which is what the gfx950 kernels and oracle.emulate do.

Nothing here shares code with oracle.emulate: it is the independent check of where emulate
rounds (tests/test_oracle.py).
"""
from __future__ import annotations

import torch


def _act(z, activation):
    if activation == "leaky_relu":
        return torch.where(z >= 0, z, 0.01 * z)  # flashmlp.py:28-30
    if activation == "silu":
        return z * torch.sigmoid(z)  # flashmlp.py:37-40
    if activation == "sigmoid":
        return torch.sigmoid(z)
    return z


def _dz(z, h_io, dh, activation, deriv):
    """dh * act'(z), before the cast (flashmlp.py:227-235)."""
    if activation == "leaky_relu":
        if deriv == "reference":
            slope = torch.where(z >= 0, 1.0, 0.01)  # flashmlp.py:33-34
        else:
            slope = torch.where(z > 0, 1.0, 0.01)   # autograd at z == 0
        return dh * slope
    if activation == "silu":
        sig = torch.sigmoid(z)
        h = h_io if deriv == "reference" else z * sig
        return dh * (sig + h * (1 - sig))  # flashmlp.py:43-46
    if activation == "sigmoid":
        sig = h_io if deriv == "reference" else torch.sigmoid(z)
        return dh * sig * (1 - sig)  # flashmlp.py:231-233
    return dh


def fwd_blocks(x, w1, w2, activation="", io_dtype=torch.bfloat16, block_b=64, block_e=64, round_out=True):
    """o as an fp32 tensor, computed tile by tile like the reference's forward program."""
    x, w1, w2 = (t.detach().to("cpu", torch.float32) for t in (x, w1, w2))
    H, B, D = x.shape
    E = w1.shape[2]
    o = torch.zeros(H, B, D)
    for h in range(H):
        for b0 in range(0, B, block_b):  # one program per B-block (flashmlp.py:82-85)
            xb = x[h, b0:b0 + block_b]
            acc = torch.zeros(xb.shape[0], D)
            for e0 in range(0, E, block_e):  # flashmlp.py:130-154
                z = xb @ w1[h, :, e0:e0 + block_e]
                h_io = _act(z, activation).to(io_dtype).to(torch.float32)
                acc += h_io @ w2[h, e0:e0 + block_e]
            o[h, b0:b0 + block_b] = acc
    return o.to(io_dtype).to(torch.float32) if round_out else o


def bwd_blocks(x, w1, w2, do, activation="", io_dtype=torch.bfloat16, block_b=64, block_e=64,
               deriv="fp32", round_out=True):
    """(dx, dw1, dw2) as fp32 tensors, computed tile by tile like the reference programs."""
    x, w1, w2, do = (t.detach().to("cpu", torch.float32) for t in (x, w1, w2, do))
    H, B, D = x.shape
    E = w1.shape[2]

    def q(t):
        return t.to(io_dtype).to(torch.float32)

    dx = torch.zeros(H, B, D)
    dw1 = torch.zeros(H, D, E)
    dw2 = torch.zeros(H, E, D)
    for h in range(H):
        # dX programs: one B-block each, looping over E (flashmlp.py:165-244)
        for b0 in range(0, B, block_b):
            xb, dob = x[h, b0:b0 + block_b], do[h, b0:b0 + block_b]
            acc = torch.zeros(xb.shape[0], D)
            for e0 in range(0, E, block_e):
                w1e, w2e = w1[h, :, e0:e0 + block_e], w2[h, e0:e0 + block_e]
                z = xb @ w1e
                h_io = q(_act(z, activation))
                dh = dob @ w2e.T
                dz = q(_dz(z, h_io, dh, activation, deriv))
                acc += dz @ w1e.T
            dx[h, b0:b0 + block_b] = acc
        # dW programs: one E-block each, looping over B (flashmlp.py:247-329)
        for e0 in range(0, E, block_e):
            w1e, w2e = w1[h, :, e0:e0 + block_e], w2[h, e0:e0 + block_e]
            a1 = torch.zeros(D, w1e.shape[1])
            a2 = torch.zeros(w1e.shape[1], D)
            for b0 in range(0, B, block_b):
                xb, dob = x[h, b0:b0 + block_b], do[h, b0:b0 + block_b]
                z = xb @ w1e
                h_io = q(_act(z, activation))
                dh = dob @ w2e.T
                a2 += h_io.T @ dob
                dz = q(_dz(z, h_io, dh, activation, deriv))
                a1 += xb.T @ dz
            dw1[h, :, e0:e0 + block_e] = a1
            dw2[h, e0:e0 + block_e] = a2
    if round_out:
        dx, dw1, dw2 = q(dx), q(dw1), q(dw2)
    return dx, dw1, dw2
