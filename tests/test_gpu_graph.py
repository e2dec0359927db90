"""HIP graph capture of flashmlp_fwd + flashmlp_bwd (torch.cuda.graph): the library launches
kernels on the caller's stream and never allocates, synchronises or clears memory itself (the
Python wrappers allocate outputs and workspaces with torch, which a capture serves from the
graph's pool), so a captured step replays the same kernels with the same plans.

Each case captures one forward + backward on static input tensors (after eager warm-up calls),
then replays the graph several times. Before each replay new values are copied into the static
inputs and the same call is run eagerly on separate tensors, with synchronisations between:
every replay's outputs must be bitwise equal to the eager call's (the kernels are deterministic).
Cases: D = 64 fp16 with a B-split workspace (recompute form), a ragged D = 64 forward whose
split tiles use the forward's workspace (cfg5's shape), the stored-dZ backward at cfg4's shape,
and the generic kernels (D = 32). The reference has no graph support to compare with.
"""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

# name, H, B, D, E, dtype, activation, backward keyword arguments
CASES = [
    ("d64_fp16_bsplit", 12, 1024, 64, 768, torch.float16, "silu", {}),
    ("d64_fp16_ragged_split_fwd", 8, 4097, 64, 2048, torch.float16, "sigmoid", {}),
    ("d128_bf16_stored_dz", 32, 16384, 128, 1024, torch.bfloat16, "silu", {}),
    ("d128_bf16_recompute_accurate", 4, 2048, 128, 512, torch.bfloat16, "leaky_relu",
     {"recompute": True, "accurate_dw": True}),
    ("d32_generic", 3, 300, 32, 72, torch.bfloat16, "sigmoid", {}),
]
REPLAYS = 4


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(H, B, D, E, dt, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(H, B, D, generator=g, device=dev, dtype=torch.float32).to(dt)
    w1 = (torch.randn(H, D, E, generator=g, device=dev, dtype=torch.float32) / D ** 0.5).to(dt)
    w2 = (torch.randn(H, E, D, generator=g, device=dev, dtype=torch.float32) / E ** 0.5).to(dt)
    do = torch.randn(H, B, D, generator=g, device=dev, dtype=torch.float32).to(dt)
    return x, w1, w2, do


@pytest.mark.parametrize("case", range(len(CASES)), ids=[c[0] for c in CASES])
def test_captured_step_replays_bitwise(case):
    import flashmlp_amd as fm
    from flashmlp_amd import _lib

    name, H, B, D, E, dt, act, kw = CASES[case]
    dev = torch.device("cuda", 0)
    _say(f"[graph] {name}: H={H} B={B} D={D} E={E} {dt} act='{act}' {kw}")
    if name == "d64_fp16_ragged_split_fwd":
        assert _lib.lib().fmlp_fwd_workspace_bytes(H, B, D, E, _lib.FMLP_DTYPE_F16) > 0, "the forward must split"
    if name == "d128_bf16_stored_dz":
        assert _lib.lib().fmlp_bwd_stores_dz(H, B, D, E, _lib.FMLP_DTYPE_BF16, 1) == 1, "the plan must store dZ"
    sx, sw1, sw2, sdo = (t.clone() for t in _inputs(H, B, D, E, dt, 100, dev))

    def step():
        o = fm.flashmlp_fwd(sx, sw1, sw2, act)
        return (o, *fm.flashmlp_bwd(sx, sw1, sw2, sdo, act, **kw))

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up: plans, kernel attributes and allocator pools
            step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    torch.cuda.synchronize(dev)
    _say(f"[graph] {name}: captured")
    for r in range(REPLAYS):
        x, w1, w2, do = _inputs(H, B, D, E, dt, 200 + r, dev)
        for s, t in ((sx, x), (sw1, w1), (sw2, w2), (sdo, do)):
            s.copy_(t)
        torch.cuda.synchronize(dev)
        graph.replay()
        eo = fm.flashmlp_fwd(x, w1, w2, act)  # eager work between the replays
        edx, edw1, edw2 = fm.flashmlp_bwd(x, w1, w2, do, act, **kw)
        torch.cuda.synchronize(dev)
        for nm, got, ref in zip(("o", "dx", "dw1", "dw2"), outs, (eo, edx, edw1, edw2)):
            assert torch.isfinite(ref).all(), f"{name}: eager {nm} not finite"
            assert torch.equal(got, ref), f"{name}: replay {r}: {nm} differs from the eager call"
        _say(f"[graph] {name}: replay {r} bitwise equal to eager")
    del graph
