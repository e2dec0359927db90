"""FlashMLP benchmark on one MI355X: fwd+bwd TFLOP/s at the north-star shape.

    python bench.py [--steps K] [--warmup W] [--workload cfg4]

A step is one flashmlp_fwd + flashmlp_bwd over the workload's synthetic inputs, all
resident in HBM before the timed region (cfg5s: one flashmlp_fwd, the forward-only sweep).
Prints ONE JSON line (one process, one GPU).

FLOP accounting: u = H*B*D*E; forward 4u, backward 8u, step 12u.
`value` = 12u / wall-clock ms_per_step (4u for cfg5s). `roofline` describes the dominant
launch, the backward entry point fmlp_bwd (8u algorithmic FLOPs per call; the forward for
cfg5s), with its duration from HIP events recorded on the stream the kernels run on.
Algorithmic HBM bytes at s bytes per element: forward (2 HBD + 2 HDE) s, backward
(3 HBD + 4 HDE) s. `autograd_ms_per_step` times the module-level step the reference's
example.py:120-128 times (FlashMLPFunction forward, then .backward). `cpu_baseline` times
the CPU oracle (torch fp32 autograd of the restated reference path) on a bounded sample of
the same workload, plus the reference's CPU configuration (cfg1) in full.

Other workloads: cfg2, cfg3, cfg5, cfg5_linear (fwd+bwd), cfg5s
(forward-only, reports HBM GB/s), example (the four shapes of the reference's
performance.md through the FlashMLP module, timed as example.py times them), mfma_ceiling
(the sustained bf16 MFMA rate of the device: register-fed v_mfma_f32_32x32x16_bf16 chains, two
waves per SIMD, random and all-zero operands; libfmlp_ceiling.so).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd TFLOP/s and % of MFMA peak (bf16/fp16), H=32 B=16384 D=128 E=1024"
PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6}  # MI355X dense MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_GBS = 8000.0

WORKLOADS = {
    # name: (H, B, D, E, dtype, activation, x_std, forward_only)
    "cfg4": (32, 16384, 128, 1024, "bf16", "silu", 1.0, False),
    "cfg3": (16, 8192, 128, 512, "bf16", "leaky_relu", 1.0, False),
    "cfg2": (12, 1024, 64, 768, "f16", "silu", 1.0, False),
    "cfg5": (8, 4097, 64, 2048, "f16", "sigmoid", 2.0, False),
    "cfg5_linear": (8, 4097, 64, 2048, "f16", "", 2.0, False),
    "cfg5s": (8, 65536, 64, 2048, "f16", "sigmoid", 2.0, True),
}
# performance.md:9-12 (example.py:86-91): bf16, SiLU, timed through the FlashMLP module
EXAMPLE_SHAPES = [(8, 512, 64, 512), (12, 1024, 64, 768), (16, 2048, 64, 1024), (32, 4096, 64, 512)]
EXAMPLE_PUBLISHED_MS = {  # (fwd, fwd+bwd) of the reference on its (unstated) hardware
    (8, 512, 64, 512): (0.036, 0.217), (12, 1024, 64, 768): (0.035, 0.222),
    (16, 2048, 64, 1024): (0.036, 0.219), (32, 4096, 64, 512): (0.060, 0.380),
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


def traffic_from_profile(kind, workload):
    """HBM bytes per call of the `kind` entry point ("bwd" or "fwd") from the committed
    rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE runs, each scaled by the same counter's
    reading for a device copy of known size), or None when no summary exists."""
    path = os.path.join(ROOT, "profiles", f"{kind}_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            key, _, val = line.partition("=")
            if key.strip() == f"hbm_bytes_per_call_{kind}":
                return int(float(val))
    return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(H, B, D, E, activation, x_std, budget_s=10.0):
    """Torch fp32 autograd of the restated reference path on the host cores this process may
    run on: a bounded sample of the workload (2 of the H heads, heads being independent,
    full B, D, E; about `budget_s` of work), and the reference's CPU configuration cfg1
    (H=12 B=1024 D=64 E=768 SiLU) in full, median of 20 iterations."""
    import torch

    from oracle import reference
    from oracle.inputs import CONFIGS, make_inputs

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def timed(args, act, min_iter, budget):
        reference.autograd_grads(*args, act)  # warm-up
        ts = []
        t_end = time.perf_counter() + budget
        while len(ts) < min_iter or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            reference.autograd_grads(*args, act)
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), len(ts)

    hs = min(2, H)
    dt, n = timed(make_inputs(hs, B, D, E, torch.float32, x_std, seed=0), activation, 3, budget_s)
    c1 = CONFIGS["cfg1"]
    dt1, n1 = timed(make_inputs(c1.H, c1.B, c1.D, c1.E, torch.float32, c1.x_std, seed=0), c1.activation, 20, 0.0)
    u1 = float(c1.H) * c1.B * c1.D * c1.E
    return {
        "value": 12.0 * hs * B * D * E / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "sample": f"{hs} of {H} heads (H={hs},B={B},D={D},E={E}, fp32, {activation or 'linear'}), "
                  f"fwd + autograd bwd, median of {n} iterations, {dt * 1e3:.1f} ms each",
        "cfg1_ms": round(dt1 * 1e3, 3),
        "cfg1_gflops": round(12 * u1 / dt1 / 1e9, 1),
        "cfg1": f"H={c1.H} B={c1.B} D={c1.D} E={c1.E} fp32 {c1.activation}, median of {n1} iterations",
    }


def peak_memory(x, w1, w2, do, activation):
    """Peak allocated MB of one fwd+bwd (example.py:142-200 method) for FlashMLP and for the
    unfused PyTorch path that keeps Z and h from the forward (contiguous bmm operands)."""
    import torch

    import flashmlp_amd as fm

    def flash():
        o = fm.flashmlp_fwd(x, w1, w2, activation)
        return o, (lambda: fm.flashmlp_bwd(x, w1, w2, do, activation))

    def flash_recompute():  # the recompute-only backward (no stored dZ)
        o = fm.flashmlp_fwd(x, w1, w2, activation)
        return o, (lambda: fm.flashmlp_bwd(x, w1, w2, do, activation, recompute=True))

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
    for name, fn in (("flashmlp", flash), ("flashmlp_recompute", flash_recompute), ("pytorch_unfused", unfused)):
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
    out["peak_savings_recompute"] = round(1 - out["flashmlp_recompute"]["peak_mb"] / out["pytorch_unfused"]["peak_mb"], 4)
    return out


def _wall_ms(fn, iters):
    """example.py:65-75: perf_counter around `iters` calls, synchronised at both ends."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / iters * 1e3


def host_us_per_call(fn, n=200):
    """CPU time to issue one call (Python wrapper + C ABI + launch), measured with the GPU
    idle so the launch queue never blocks: mean over n issues, then synchronise."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        fn()
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    return (t1 - t0) / n * 1e6


def autograd_step_ms(x, w1, w2, do, act, warmup=3, iters=20):
    """Module-level training step as example.py:120-128 times it: FlashMLPFunction forward
    on a leaf that requires grad, then backward (here with dO, the bench's gradient)."""
    import flashmlp_amd as fm

    xg = x.detach().requires_grad_(True)
    w1g = w1.detach().requires_grad_(True)
    w2g = w2.detach().requires_grad_(True)

    def step():
        o = fm.FlashMLPFunction.apply(xg, w1g, w2g, act)
        o.backward(do)
        xg.grad = w1g.grad = w2g.grad = None

    for _ in range(warmup):
        step()
    return _wall_ms(step, iters)


def run_example(args):
    """performance.md's four shapes through the FlashMLP module, timed like example.py
    (10 warmup + 100 iterations, wall clock, fwd = model(x), fwd+bwd = model(x).sum().backward())."""
    import numpy as np
    import torch

    import flashmlp_amd as fm

    rows = []
    for H, B, D, E in EXAMPLE_SHAPES:
        torch.manual_seed(0)
        model = fm.FlashMLP(H, D, E, activation="silu", dtype=torch.bfloat16, device="cuda")
        x = torch.randn(H, B, D, device="cuda", dtype=torch.bfloat16) / np.sqrt(D)

        def fwd():
            return model(x)

        def fwd_bwd():
            x_in = x.detach().requires_grad_(True)
            model(x_in).sum().backward()

        for f in (fwd, fwd_bwd):
            for _ in range(10):
                f()
        t_f = _wall_ms(fwd, 100)
        t_fb = _wall_ms(fwd_bwd, 100)
        u = float(H) * B * D * E
        pub = EXAMPLE_PUBLISHED_MS[(H, B, D, E)]
        rows.append({"H": H, "B": B, "D": D, "E": E, "fwd_ms": round(t_f, 4), "fwd_bwd_ms": round(t_fb, 4),
                     "fwd_tflops": round(4 * u / t_f / 1e9, 2), "fwd_bwd_tflops": round(12 * u / t_fb / 1e9, 2),
                     "reference_published_ms": {"fwd": pub[0], "fwd_bwd": pub[1], "hardware": "unstated"}})
        model.zero_grad()
    line = {"metric": METRIC, "workload": "example", "unit": "ms", "dtype": "bf16",
            "note": "performance.md shapes through FlashMLP (module, autograd), wall clock incl. Python",
            "rows": rows}
    print(json.dumps(line), flush=True)


def run_mfma_ceiling(args):
    """Sustained executed bf16 MFMA rate with operands in registers (no memory traffic), random
    and all-zero operand bits: the power-limited ceiling the FlashMLP kernels are compared with."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "flashmlp_amd", "libfmlp_ceiling.so"))
    lib.fmlp_ceiling_mfma.restype = ctypes.c_int
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    grid, iters = 2 * ncu, 4000  # two waves per SIMD
    out = torch.empty(grid * 256, device="cuda", dtype=torch.float32)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    flops = float(grid) * 4 * iters * 4 * 32768
    res = {}
    for name, zero in (("random", 0), ("zero", 1)):
        def call():
            r = lib.fmlp_ceiling_mfma(ctypes.c_void_p(out.data_ptr()), iters, zero, grid, st)
            if r != 0:
                raise RuntimeError(f"fmlp_ceiling_mfma: hip error {r}")
        for _ in range(args.warmup + 20):
            call()
        torch.cuda.synchronize()
        ms = _wall_ms(call, max(args.steps, 50))
        res[name] = {"tflops": round(flops / (ms * 1e-3) / 1e12, 1), "ms_per_launch": round(ms, 4)}
    # the same loop with a kernel's other per-MFMA work added (random operands): LDS reads
    # feeding the A operand (1 KB per wave per MFMA) and sigmoid-like VALU chains
    lib.fmlp_ceiling_mix.restype = ctypes.c_int
    mix_iters = 1000
    mix_flops = float(grid) * 4 * mix_iters * 16 * 32768
    mix = {}
    for lds_reads in (0, 1):
        for chains in (0, 1, 2):
            def call_mix():
                r = lib.fmlp_ceiling_mix(ctypes.c_void_p(out.data_ptr()), mix_iters, lds_reads, chains, grid, st)
                if r != 0:
                    raise RuntimeError(f"fmlp_ceiling_mix: hip error {r}")
            for _ in range(args.warmup + 20):
                call_mix()
            torch.cuda.synchronize()
            ms = _wall_ms(call_mix, max(args.steps, 50))
            mix[f"lds{lds_reads}_chains{chains}"] = round(mix_flops / (ms * 1e-3) / 1e12, 1)
    peak = PEAK_TFLOPS["bf16"]
    line = {"metric": "sustained bf16 MFMA rate (v_mfma_f32_32x32x16_bf16, register operands)", "workload": "mfma_ceiling",
            "unit": "TFLOP/s", "peak": peak, "random": res["random"], "zero": res["zero"],
            "random_frac_of_peak": round(res["random"]["tflops"] / peak, 4),
            "with_per_mfma_work": {"unit": "TFLOP/s", "lds": "1 KB LDS read per wave per MFMA (A operand)",
                                   "chains": "sigmoid-like VALU chains (mul, exp, add, rcp) per MFMA", **mix},
            "config": {"grid": grid, "waves_per_simd": 2, "mfma_per_wave": iters * 4, "chains_per_wave": 4}}
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg4", choices=sorted(WORKLOADS) + ["example", "mfma_ceiling"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-memory", action="store_true", help="skip the peak-memory comparison")
    ap.add_argument("--no-extra", action="store_true", help="skip the autograd-step and host-overhead timings")
    ap.add_argument("--accurate-dw", action="store_true",
                    help="time the backward in its dW accuracy mode (h and dZ as hi + lo terms)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="after timing, run device copies of this size (HBM counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU: the fused MLP shards by head with no "
                                   "communication (each GPU runs its heads' share as one GPU does here), "
                                   "so multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    import torch

    import flashmlp_amd as fm

    torch.cuda.set_device(0)
    if args.workload == "example":
        run_example(args)
        return
    if args.workload == "mfma_ceiling":
        run_mfma_ceiling(args)
        return

    H, B, D, E, dt_name, act, x_std, fwd_only = WORKLOADS[args.workload]
    dtype = _torch_dtype(dt_name)
    x, w1, w2, do = make_gpu_inputs(H, B, D, E, dtype, x_std)
    torch.cuda.synchronize()
    s = 2  # bytes per io element

    for _ in range(args.warmup):
        fm.flashmlp_fwd(x, w1, w2, act)
        if not fwd_only:
            fm.flashmlp_bwd(x, w1, w2, do, act, accurate_dw=args.accurate_dw)
    torch.cuda.synchronize()

    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(K)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        ev[k][0].record()
        o = fm.flashmlp_fwd(x, w1, w2, act)
        ev[k][1].record()
        if not fwd_only:
            g = fm.flashmlp_bwd(x, w1, w2, do, act, accurate_dw=args.accurate_dw)
        ev[k][2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / K
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / K if not fwd_only else 0.0
    assert torch.isfinite(o.float()).all()
    if not fwd_only:
        assert all(torch.isfinite(t.float()).all() for t in g)

    u = float(H) * B * D * E
    flops = (4 if fwd_only else 12) * u
    ms_per_step = wall * 1e3 / K
    value = flops / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_TFLOPS[dt_name]
    fwd_tf = 4 * u / (fwd_ms * 1e-3) / 1e12
    fwd_bytes = (2 * H * B * D + 2 * H * D * E) * s
    bwd_bytes = (3 * H * B * D + 4 * H * D * E) * s

    if args.calib_copy_mb > 0:
        n = args.calib_copy_mb * 2 ** 20 // 4
        src = torch.ones(n, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    step_name = "fused MLP forward (inference sweep)" if fwd_only else "fused MLP fwd+bwd"
    if args.accurate_dw:
        step_name += " (dW accuracy mode)"
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
        "data": f"synthetic (seeded N(0,{x_std:g}^2) X, N(0,1) dO, N(0,1/D) W1, N(0,1/E) W2, drawn on the GPU)",
        "config": {"workload": f"{args.workload}: {step_name} H={H} B={B} D={D} E={E} act={act or 'linear'}",
                   "H": H, "B": B, "D": D, "E": E, "activation": act, "flops_per_step": flops},
        "pct_of_peak": round(100 * value / peak, 2),
        "fwd_ms": round(fwd_ms, 4),
        "fwd_tflops": round(fwd_tf, 2),
        "fwd_hbm_gbs": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9, 1),
    }
    if fwd_only:
        line["roofline"] = {
            "kernel": "fmlp_fwd call: fmlp::fwd_kernel",
            "bound": "mfma",
            "achieved": round(fwd_tf, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(fwd_tf / peak, 4),
            "traffic": traffic_from_profile("fwd", args.workload),
            "algorithmic_flops_per_launch": 4 * u,
            "algorithmic_bytes_per_launch": fwd_bytes,
            "avg_launch_ms": round(fwd_ms, 4),
            "hbm_gbs": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9 / HBM_GBS, 4),
        }
    else:
        bwd_tf = 8 * u / (bwd_ms * 1e-3) / 1e12
        line["bwd_ms"] = round(bwd_ms, 4)
        line["bwd_tflops"] = round(bwd_tf, 2)
        line["bwd_hbm_gbs"] = round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1)
        from flashmlp_amd import _lib
        code = (_lib.FMLP_DTYPE_BF16 if dt_name == "bf16" else _lib.FMLP_DTYPE_F16) | \
            (_lib.FMLP_DW_HILO if args.accurate_dw else 0)
        stores_dz = bool(_lib.lib().fmlp_bwd_stores_dz(H, B, D, E, code, _lib.ACT_CODES[act]))
        line["bwd_form"] = "stored-dZ" if stores_dz else "recompute"
        line["roofline"] = {
            "kernel": ("fmlp_bwd call, stored-dZ form: fmlp::dw2_kernel (dW programs, also writing dZ), "
                       "fmlp::dw_reduce_kernel when they split B, then fmlp::dxg_kernel (dX = dZ W1^T)"
                       if stores_dz else
                       "fmlp_bwd call, recompute form: fmlp::bwd_kernel (dW and dX programs in one launch; "
                       "then fmlp::dw_reduce_kernel when the dW programs split B)"),
            "bound": "mfma",
            "achieved": round(bwd_tf, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / peak, 4),
            "traffic": traffic_from_profile("bwd", args.workload),
            "algorithmic_flops_per_launch": 8 * u,
            "algorithmic_bytes_per_launch": bwd_bytes,
            "avg_launch_ms": round(bwd_ms, 4),
        }
    if not args.no_extra:
        line["host_us_per_call"] = {"fwd": round(host_us_per_call(lambda: fm.flashmlp_fwd(x, w1, w2, act)), 2)}
        if not fwd_only:
            line["host_us_per_call"]["bwd"] = round(host_us_per_call(lambda: fm.flashmlp_bwd(x, w1, w2, do, act)), 2)
            line["autograd_ms_per_step"] = round(autograd_step_ms(x, w1, w2, do, act), 4)
    if not args.no_memory and not fwd_only:
        line["memory"] = peak_memory(x, w1, w2, do, act)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(H, B, D, E, act, x_std)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
