"""CPU oracle for FlashMLP — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or, for the CPU baseline, as the thing timed on the
host). The FlashMLP product path (flashmlp_amd) never imports it and has no CPU fallback.

Contents
  reference.py  torch fp32 restatement of the reference path (flashmlp.py:671-686) and its
                autograd gradients; the reference's manual backward (flashmlp.py:689-723).
  emulate.py    cast-point emulation of the reference kernels: fp32 accumulation with
                act(Z) and dZ rounded to the io dtype where flashmlp.py:141-150, :215-235
                and :297-320 round them.
  blockwise.py  the reference's two backward programs (flashmlp.py:165-329) restated tile by
                tile with the reference's cast points; pins where emulate.emu_bwd rounds.
  inputs.py     seeded inputs for the BASELINE.json configurations.
  brute.c       independent fp64 loop implementation (C) of forward and backward, built
                by build.py into oracle/_build/; pins reference.py on tiny shapes.

How each function is pinned (tests/test_oracle.py):
  reference.torch_fwd / autograd_grads: fp64 C brute force on tiny shapes (all four
      activations), torch.autograd.gradcheck, closed forms for the linear activation
      (O = X (W1 W2), dX = dO W2^T W1^T, ...), derivative values at the kinks, head and
      row independence, leaky == linear when every Z > 0.
  reference.manual_bwd: equals autograd except for Leaky ReLU at Z == 0 (slope 1 vs 0.01).
  emulate.*: with fp32 io it reduces to reference.* exactly-up-to-summation-order;
      emu_fwd's rounding point is checked by planting a missing cast (the test expects a
      miss); emu_bwd equals blockwise.bwd_blocks (the reference programs tile by tile) to
      fp32 noise, and planted variants (no h cast, no dZ cast, dH cast instead of dZ) each
      move the outputs they feed by > 5e-4 relative against it.
  blockwise.*: its literal-reference derivative (SiLU/sigmoid from the rounded h, Leaky
      ReLU slope 1 at z == 0) is checked against the fp32 form: farther from autograd, and
      exactly 100x at the leaky kink.
The reference ships no golden vectors or known-answer tests for this path.
"""
