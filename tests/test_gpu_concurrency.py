"""Concurrent calls: the C ABI is reentrant except fmlp_bwd_noalloc (its only shared state is
caches of per-device CU counts and backward plans behind locks, and kernel attributes set once
atomically), and ctypes releases the GIL during a call, so threads on their own streams run the
library at the same time. No kernel waits on another workgroup, so kernels of different
streams may overlap on the device in any way.

Four threads, each on its own stream, run forward + backward on a shape of their own (the
tuned D = 128 and D = 64 kernels, the generic kernels in fp32, the D = 256 programs) several
times, starting on shapes no other test plans, so the plans are computed concurrently too.
Afterwards each shape runs once more serially on the default stream: every output of every
thread must be bitwise equal to it (same plan, deterministic kernels).
"""
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest
import torch

pytestmark = pytest.mark.gpu

# H, B, D, E, dtype, activation
CASES = [
    (4, 2311, 128, 384, torch.bfloat16, "silu"),
    (6, 1517, 64, 520, torch.float16, "sigmoid"),
    (3, 777, 32, 200, torch.float32, "leaky_relu"),
    (2, 1203, 256, 264, torch.bfloat16, "silu"),
]
ITERS = 5


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(i):
    H, B, D, E, dt, _ = CASES[i]
    g = torch.Generator(device="cuda").manual_seed(500 + i)
    x = torch.randn(H, B, D, generator=g, device="cuda", dtype=torch.float32).to(dt)
    w1 = (torch.randn(H, D, E, generator=g, device="cuda", dtype=torch.float32) / D ** 0.5).to(dt)
    w2 = (torch.randn(H, E, D, generator=g, device="cuda", dtype=torch.float32) / E ** 0.5).to(dt)
    do = torch.randn(H, B, D, generator=g, device="cuda", dtype=torch.float32).to(dt)
    return x, w1, w2, do


def test_threads_on_their_own_streams():
    import flashmlp_amd as fm

    inputs = [_inputs(i) for i in range(len(CASES))]
    torch.cuda.synchronize()

    def work(i):
        x, w1, w2, do = inputs[i]
        act = CASES[i][5]
        stream = torch.cuda.Stream()
        outs = []
        with torch.cuda.stream(stream):
            for _ in range(ITERS):
                o = fm.flashmlp_fwd(x, w1, w2, act)
                outs.append((o, *fm.flashmlp_bwd(x, w1, w2, do, act)))
        stream.synchronize()
        return outs

    _say(f"[concurrency] {len(CASES)} threads x {ITERS} fwd + bwd: " + ", ".join(
        f"H={c[0]} B={c[1]} D={c[2]} E={c[3]} {c[4]} {c[5]}" for c in CASES))
    with ThreadPoolExecutor(max_workers=len(CASES)) as ex:
        results = list(ex.map(work, range(len(CASES))))
    torch.cuda.synchronize()
    for i, outs in enumerate(results):
        x, w1, w2, do = inputs[i]
        act = CASES[i][5]
        ref = (fm.flashmlp_fwd(x, w1, w2, act), *fm.flashmlp_bwd(x, w1, w2, do, act))
        torch.cuda.synchronize()
        for it, out in enumerate(outs):
            for name, a, b in zip(("o", "dx", "dw1", "dw2"), out, ref):
                assert torch.isfinite(b).all(), f"case {i}: {name} not finite"
                assert torch.equal(a, b), f"case {i}, iteration {it}: {name} differs from the serial call"
        _say(f"[concurrency] case {i}: {ITERS} concurrent results bitwise equal to the serial call")
