"""Child process of tests/test_gpu_plan_overrides.py: forward + backward of a fixed set of shapes
under whatever FMLP_* plan overrides its environment holds (each is read once per process),
checked against the CPU oracle at the bars of tests/test_gpu_random_shapes.py. Prints one line
per case and exits 1 if any case misses its bar."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

import flashmlp_amd as fm  # noqa: E402
from oracle import emulate, reference  # noqa: E402
from oracle.inputs import make_inputs  # noqa: E402

# H, B, D, E, dtype, activation, backward keywords
CASES = [
    (3, 2100, 64, 1000, torch.float16, "sigmoid", {}),
    (4, 4097, 64, 520, torch.bfloat16, "silu", {}),
    (2, 8192, 128, 256, torch.bfloat16, "silu", {}),
    (5, 700, 128, 40, torch.bfloat16, "leaky_relu", {"recompute": True}),
    (2, 2049, 128, 1024, torch.float16, "silu", {"accurate_dw": True}),
    (2, 1203, 256, 264, torch.bfloat16, "silu", {}),
    (3, 300, 32, 45, torch.float32, "sigmoid", {}),
]


def _fail(a, b, tol=3e-2):
    a, b = a.float(), b.float()
    return ((a - b).abs() > tol + tol * b.abs()).float().mean().item()


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def main():
    env = " ".join(f"{k}={v}" for k, v in sorted(os.environ.items()) if k.startswith("FMLP_"))
    bad = 0
    for i, (H, B, D, E, dt, act, kw) in enumerate(CASES):
        x, w1, w2, do = make_inputs(H, B, D, E, dt, seed=300 + i)
        xg, w1g, w2g, dog = (t.cuda() for t in (x, w1, w2, do))
        o = fm.flashmlp_fwd(xg, w1g, w2g, act)
        dx, dw1, dw2 = fm.flashmlp_bwd(xg, w1g, w2g, dog, act, **kw)
        torch.cuda.synchronize()
        ro, rdx, rdw1, rdw2 = reference.autograd_grads(x, w1, w2, do, act)
        msgs = []
        if dt == torch.float32:
            for n, g, r in (("o", o, ro), ("dx", dx, rdx), ("dw1", dw1, rdw1), ("dw2", dw2, rdw2)):
                if not _rel(g.cpu(), r) <= 1e-4:
                    msgs.append(f"{n} normwise {_rel(g.cpu(), r):.2e}")
        else:
            for n, g, r in (("o", o, ro), ("dx", dx, rdx)):
                if _fail(g.cpu(), r) > 1e-4:
                    msgs.append(f"{n} miss fraction {_fail(g.cpu(), r):.2e}")
            _, edw1, edw2 = emulate.emu_bwd(x, w1, w2, do, act, dt)
            for n, g, e, r in (("dw1", dw1, edw1, rdw1), ("dw2", dw2, edw2, rdw2)):
                g = g.cpu()
                f = _fail(g, r) if kw.get("accurate_dw") else _fail(g, e)
                if f > 1e-5 or _rel(g, r) > 1e-2:
                    msgs.append(f"{n} miss fraction {f:.2e}, normwise {_rel(g, r):.2e}")
        for n, g in (("o", o), ("dx", dx), ("dw1", dw1), ("dw2", dw2)):
            if not torch.isfinite(g).all():
                msgs.append(f"{n} not finite")
        bad += bool(msgs)
        print(f"[{env}] H={H} B={B} D={D} E={E} {dt} act='{act}' {kw}: {'; '.join(msgs) or 'ok'}", flush=True)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
