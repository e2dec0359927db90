"""FlashMLP benchmark on one MI355X: fwd+bwd TFLOP/s at the north-star shape.

    python bench.py [--steps K] [--warmup W] [--workload cfg4]

A step is one flashmlp_fwd + flashmlp_bwd over the workload's synthetic inputs, all
resident in HBM before the timed region. Prints ONE JSON line (rank 0 of one process).

FLOP accounting: u = H*B*D*E; forward 4u, backward 8u, step 12u.
`value` = 12u / wall-clock ms_per_step. `roofline` describes the dominant launch, the
backward entry point fmlp_bwd (its dW and dX kernels, 8u algorithmic FLOPs per call),
with its duration from HIP events recorded on the stream the kernels run on; the
per-kernel split is in the committed rocprofv3 summary. `cpu_baseline` times the CPU
oracle (torch fp32 autograd of the restated reference path) on a bounded sample of the
same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd TFLOP/s and % of MFMA peak (bf16/fp16), H=32 B=16384 D=128 E=1024"
PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6}  # MI355X dense MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_GBS = 8000.0

WORKLOADS = {
    # name: (H, B, D, E, dtype, activation, x_std)
    "cfg4": (32, 16384, 128, 1024, "bf16", "silu", 1.0),
    "cfg3": (16, 8192, 128, 512, "bf16", "leaky_relu", 1.0),
    "cfg2": (12, 1024, 64, 768, "f16", "silu", 1.0),
    "cfg5": (8, 4097, 64, 2048, "f16", "sigmoid", 2.0),
}


def _torch_dtype(name):
    import torch

    return {"bf16": torch.bfloat16, "f16": torch.float16}[name]


def make_gpu_inputs(H, B, D, E, dtype, x_std, seed=0):
    """Synthetic inputs drawn on the GPU (BASELINE.json init: X~N(0,x_std^2), W1~N(0,1/D),
    W2~N(0,1/E), dO~N(0,1)), rounded to the io dtype."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    f = dict(device="cuda", dtype=torch.float32, generator=g)
    x = (torch.randn(H, B, D, **f) * x_std).to(dtype)
    w1 = (torch.randn(H, D, E, **f) / D ** 0.5).to(dtype)
    w2 = (torch.randn(H, E, D, **f) / E ** 0.5).to(dtype)
    do = torch.randn(H, B, D, **f).to(dtype)
    return x, w1, w2, do


def traffic_from_profile(workload):
    """HBM bytes per backward call (dW + dX kernels) from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE runs, each scaled by the same counter's reading for
    a device copy of known size), or None when no summary exists for this workload."""
    path = os.path.join(ROOT, "profiles", f"bwd_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            key, _, val = line.partition("=")
            if key.strip() == "hbm_bytes_per_call_bwd":
                return int(float(val))
    return None


def cpu_baseline(H, B, D, E, activation, x_std, budget_s=10.0):
    """Torch fp32 autograd of the restated reference path on the host cores, on a sample of
    the workload: 2 of the H heads (heads are independent), full B, D, E."""
    import torch

    from oracle import reference
    from oracle.inputs import make_inputs

    hs = min(2, H)
    x, w1, w2, do = make_inputs(hs, B, D, E, torch.float32, x_std, seed=0)
    threads = torch.get_num_threads()
    reference.autograd_grads(x, w1, w2, do, activation)  # warm-up
    n = 0
    t0 = time.perf_counter()
    while True:
        reference.autograd_grads(x, w1, w2, do, activation)
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = (time.perf_counter() - t0) / n
    flops = 12.0 * hs * B * D * E
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{hs} of {H} heads (H={hs},B={B},D={D},E={E}, fp32, {activation}), "
                  f"fwd + autograd bwd, {n} iterations, {dt * 1e3:.1f} ms each",
    }


def peak_memory(x, w1, w2, do, activation):
    """Peak allocated MB of one fwd+bwd (example.py:142-200 method) for FlashMLP and for the
    unfused PyTorch path that keeps Z and h from the forward (contiguous bmm operands)."""
    import torch

    import flashmlp_amd as fm

    def flash():
        o = fm.flashmlp_fwd(x, w1, w2, activation)
        return o, (lambda: fm.flashmlp_bwd(x, w1, w2, do, activation))

    def unfused():
        z = torch.bmm(x, w1)
        h = {"silu": torch.nn.functional.silu, "sigmoid": torch.sigmoid,
             "leaky_relu": lambda t: torch.nn.functional.leaky_relu(t, 0.01)}.get(activation, lambda t: t)(z)
        o = torch.bmm(h, w2)

        def bwd():
            dh = torch.bmm(do, w2.transpose(1, 2).contiguous())
            dw2 = torch.bmm(h.transpose(1, 2).contiguous(), do)
            if activation == "silu":
                s = torch.sigmoid(z)
                dz = dh * (s + z * s * (1 - s))
            elif activation == "sigmoid":
                dz = dh * h * (1 - h)
            elif activation == "leaky_relu":
                dz = dh * torch.where(z > 0, 1.0, 0.01).to(dh.dtype)
            else:
                dz = dh
            dx = torch.bmm(dz, w1.transpose(1, 2).contiguous())
            dw1 = torch.bmm(x.transpose(1, 2).contiguous(), dz)
            return dx, dw1, dw2

        return o, bwd

    out = {}
    for name, fn in (("flashmlp", flash), ("pytorch_unfused", unfused)):
        o, b = fn()
        b()
        del o, b
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        o, b = fn()
        fwd_mb = (torch.cuda.memory_allocated() - base) / 2 ** 20
        g = b()
        torch.cuda.synchronize()
        peak_mb = (torch.cuda.max_memory_allocated() - base) / 2 ** 20
        del o, b, g
        torch.cuda.empty_cache()
        out[name] = {"fwd_alloc_mb": round(fwd_mb, 1), "peak_mb": round(peak_mb, 1)}
    out["peak_savings"] = round(1 - out["flashmlp"]["peak_mb"] / out["pytorch_unfused"]["peak_mb"], 4)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg4", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-memory", action="store_true", help="skip the peak-memory comparison")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="after timing, run device copies of this size (HBM counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU; the fused MLP shards by head with no "
                                   "communication (see DESIGN.md), multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    import torch

    import flashmlp_amd as fm

    H, B, D, E, dt_name, act, x_std = WORKLOADS[args.workload]
    dtype = _torch_dtype(dt_name)
    torch.cuda.set_device(0)
    x, w1, w2, do = make_gpu_inputs(H, B, D, E, dtype, x_std)
    torch.cuda.synchronize()

    def step():
        o = fm.flashmlp_fwd(x, w1, w2, act)
        g = fm.flashmlp_bwd(x, w1, w2, do, act)
        return o, g

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(K)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        ev[k][0].record()
        o = fm.flashmlp_fwd(x, w1, w2, act)
        ev[k][1].record()
        g = fm.flashmlp_bwd(x, w1, w2, do, act)
        ev[k][2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / K
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / K
    assert torch.isfinite(o.float()).all() and all(torch.isfinite(t.float()).all() for t in g)

    u = float(H) * B * D * E
    ms_per_step = wall * 1e3 / K
    value = 12 * u / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_TFLOPS[dt_name]
    bwd_tf = 8 * u / (bwd_ms * 1e-3) / 1e12
    fwd_tf = 4 * u / (fwd_ms * 1e-3) / 1e12

    if args.calib_copy_mb > 0:
        n = args.calib_copy_mb * 2 ** 20 // 4
        src = torch.ones(n, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt_name,
        "data": "synthetic (seeded N(0,1) X and dO, N(0,1/D) W1, N(0,1/E) W2, drawn on the GPU)",
        "config": {"workload": f"{args.workload}: fused MLP fwd+bwd H={H} B={B} D={D} E={E} act={act or 'linear'}",
                   "H": H, "B": B, "D": D, "E": E, "activation": act, "flops_per_step": 12 * u},
        "pct_of_peak": round(100 * value / peak, 2),
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "fwd_tflops": round(fwd_tf, 2),
        "bwd_tflops": round(bwd_tf, 2),
        "roofline": {
            "kernel": "fmlp_bwd call: fmlp::dw2_kernel + fmlp::dx2_kernel",
            "bound": "mfma",
            "achieved": round(bwd_tf, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / peak, 4),
            "traffic": traffic_from_profile(args.workload),
            "algorithmic_flops_per_launch": 8 * u,
            "avg_launch_ms": round(bwd_ms, 4),
        },
    }
    if not args.no_memory:
        line["memory"] = peak_memory(x, w1, w2, do, act)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(H, B, D, E, act, x_std)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
