"""FlashMLP benchmark on one MI355X: fwd+bwd TFLOP/s at the north-star shape.

    python bench.py [--steps K] [--warmup W] [--workload cfg4]

A step is one flashmlp_fwd + flashmlp_bwd over the workload's synthetic inputs, all
resident in HBM before the timed region (cfg5s: one flashmlp_fwd, the forward-only sweep).
Prints ONE JSON line (one process, one GPU).

FLOP accounting: u = H*B*D*E; forward 4u, backward 8u, step 12u.
`value` = 12u / wall-clock ms_per_step (4u for cfg5s) over K steps issued back to back
(`gpu_ms_per_step`: the same region timed by two HIP events at its ends). `roofline` describes
the dominant launch, the backward entry point fmlp_bwd (8u algorithmic FLOPs per call; the
forward for cfg5s), with its mean duration from HIP events recorded around each call, on the
stream the kernels run on, over K further steps right after the timed ones (events between
kernels idle the GPU for several microseconds each, so they stay out of the timed steps).
Algorithmic HBM bytes at s bytes per element: forward (2 HBD + 2 HDE) s, backward
(3 HBD + 4 HDE) s.

The default (cfg4) line also carries, measured in the same process after the headline:
  * `cfg4_forms`: the same step with the reference's recompute-only backward (recompute=True,
    the form the north star names), with the dW accuracy mode (accurate_dw=True: dW within the
    elementwise tolerance of fp32), and with both;
  * `configs`: every other BASELINE.json configuration (cfg2, cfg3, cfg5 sigmoid and linear,
    the forward-only cfg5s sweep) on the tuned kernels, and two shapes outside the tuned
    kernels' main range: the reference's CPU configuration cfg1 in fp32 (generic kernels) and
    D = 256 (its own tuned forward, dX and dW programs); per configuration also its peak
    memory against the unfused path and the CPU oracle's time per step;
  * `vs_pytorch_unfused`: the unfused PyTorch path (bmm -> activation -> bmm, the (H, B, E)
    intermediates kept, manual backward) on the same GPU against FlashMLP, at cfg4 and at the
    four shapes of the reference's performance.md (example.py:98-135 compares the two);
  * `memory`: peak allocated MB of one fwd+bwd for both backward forms and the unfused path
    (example.py:142-200), plus the device memory the library's code objects hold, and
    example.py's own module comparison at the five shapes of performance.md's memory table;
  * `autograd_ms_per_step` (FlashMLPFunction forward + backward, as example.py:120-128 times
    the module), host microseconds per call;
  * `cpu_baseline`: the CPU oracle (torch fp32 autograd of the restated reference path) on a
    bounded sample of the workload, plus the reference's CPU configuration (cfg1) in full.

Other workloads: cfg2, cfg3, cfg5, cfg5_linear (fwd+bwd), cfg5s
(forward-only, reports HBM GB/s), example (the four shapes of the reference's
performance.md through the FlashMLP module, timed as example.py times them), mfma_ceiling
(the sustained bf16 MFMA rate of the device: register-fed v_mfma_f32_32x32x16_bf16 chains, two
waves per SIMD, random and all-zero operands; libfmlp_ceiling.so).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd TFLOP/s and % of MFMA peak (bf16/fp16), H=32 B=16384 D=128 E=1024"
# MI355X dense MFMA peaks (256 CU x 2.4 GHz): bf16 / fp16 4096 FLOP/clk/CU, fp32 256
PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}
HBM_GBS = 8000.0

WORKLOADS = {
    # name: (H, B, D, E, dtype, activation, x_std, forward_only)
    "cfg4": (32, 16384, 128, 1024, "bf16", "silu", 1.0, False),
    "cfg3": (16, 8192, 128, 512, "bf16", "leaky_relu", 1.0, False),
    "cfg2": (12, 1024, 64, 768, "f16", "silu", 1.0, False),
    "cfg5": (8, 4097, 64, 2048, "f16", "sigmoid", 2.0, False),
    "cfg5_linear": (8, 4097, 64, 2048, "f16", "", 2.0, False),
    "cfg5s": (8, 65536, 64, 2048, "f16", "sigmoid", 2.0, True),
    # the reference's CPU configuration in fp32 (generic kernels), and
    # D = 256 (its own tuned forward, dX and dW programs)
    "cfg1_fp32": (12, 1024, 64, 768, "f32", "silu", 1.0, False),
    "d256": (8, 4096, 256, 1024, "bf16", "silu", 1.0, False),
}
# the `configs` pass of the default line, in this order
CONFIG_PASS = ["cfg2", "cfg3", "cfg5", "cfg5_linear", "cfg5s", "cfg1_fp32", "d256"]
# performance.md:9-12 (example.py:86-91): bf16, SiLU, timed through the FlashMLP module
EXAMPLE_SHAPES = [(8, 512, 64, 512), (12, 1024, 64, 768), (16, 2048, 64, 1024), (32, 4096, 64, 512)]
# performance.md:24-30 (example.py:142-200): peak and forward-allocated MB of one module forward +
# backward, PyTorch vs the reference's FlashMLP, bf16 SiLU
MEMORY_SHAPES = [(8, 512, 64, 512), (12, 1024, 64, 768), (16, 2048, 64, 1024), (32, 4096, 64, 512),
                 (12, 4096, 64, 768)]
MEMORY_PUBLISHED_MB = {  # (PyTorch peak, FlashMLP peak, PyTorch fwd, FlashMLP fwd)
    (8, 512, 64, 512): (13.5, 2.5, 8.5, 0.5), (12, 1024, 64, 768): (58.1, 7.5, 37.5, 1.5),
    (16, 2048, 64, 1024): (202.0, 16.0, 132.0, 4.0), (32, 4096, 64, 512): (418.0, 52.0, 272.0, 16.0),
    (12, 4096, 64, 768): (229.1, 21.0, 150.0, 6.0),
}
EXAMPLE_PUBLISHED_MS = {  # (fwd, fwd+bwd) of the reference on its (unstated) hardware
    (8, 512, 64, 512): (0.036, 0.217), (12, 1024, 64, 768): (0.035, 0.222),
    (16, 2048, 64, 1024): (0.036, 0.219), (32, 4096, 64, 512): (0.060, 0.380),
}


def _torch_dtype(name):
    import torch

    return {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[name]


def _es(name):
    return 4 if name == "f32" else 2


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


# ---------------------------------------------------------------------------------------
# The unfused PyTorch path (the reference's PyTorchMLP / flashmlp_torch_bwd computation,
# flashmlp.py:619-723): Z and h kept from the forward, the backward's products as bmm calls on
# contiguous operands (transposed views are copied first; with the transposes placed so that
# only weight-sized and X/dO-sized copies are made, never a copy of the (H, B, E) plane).
# ---------------------------------------------------------------------------------------
def _torch_act(t, activation):
    import torch

    return {"silu": torch.nn.functional.silu, "sigmoid": torch.sigmoid,
            "leaky_relu": lambda v: torch.nn.functional.leaky_relu(v, 0.01)}.get(activation, lambda v: v)(t)


def unfused_fwd(x, w1, w2, activation):
    import torch

    z = torch.bmm(x, w1)
    h = _torch_act(z, activation)
    return torch.bmm(h, w2), z, h


def unfused_bwd(x, w1, w2, do, z, h, activation):
    import torch

    dh = torch.bmm(do, w2.transpose(1, 2).contiguous())
    dw2 = torch.bmm(do.transpose(1, 2).contiguous(), h).transpose(1, 2).contiguous()
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


def _device_used():
    import torch

    free, total = torch.cuda.mem_get_info()
    return total - free


def module_memory():
    """example.py:142-200's comparison, as it runs it: per shape, a PyTorchMLP and a FlashMLP module
    (bf16, SiLU), one warm-up forward + `.sum().backward()`, then peak allocated MB of one more
    (max_memory_allocated minus the memory allocated before the forward) and the MB the forward
    leaves allocated; the reference's published rows beside them (performance.md:24-30)."""
    import numpy as np
    import torch

    import flashmlp_amd as fm

    rows = []
    for H, B, D, E in MEMORY_SHAPES:
        r = {"H": H, "B": B, "D": D, "E": E}
        for name, cls in (("pytorch", fm.PyTorchMLP), ("flashmlp", fm.FlashMLP)):
            torch.cuda.empty_cache()
            model = cls(H, D, E, activation="silu", dtype=torch.bfloat16, device="cuda")
            xw = (torch.randn(H, B, D, device="cuda", dtype=torch.bfloat16) / np.sqrt(D)).requires_grad_(True)
            model(xw).sum().backward()
            del xw
            model.zero_grad()
            torch.cuda.empty_cache()
            torch.cuda.reset_peak_memory_stats()
            x = (torch.randn(H, B, D, device="cuda", dtype=torch.bfloat16) / np.sqrt(D)).requires_grad_(True)
            before = torch.cuda.memory_allocated()
            o = model(x)
            fwd_mb = (torch.cuda.memory_allocated() - before) / 2 ** 20
            o.sum().backward()
            torch.cuda.synchronize()
            r[f"{name}_peak_mb"] = round((torch.cuda.max_memory_allocated() - before) / 2 ** 20, 1)
            r[f"{name}_fwd_mb"] = round(fwd_mb, 1)
            del model, x, o
            torch.cuda.empty_cache()
        r["peak_savings"] = round(1 - r["flashmlp_peak_mb"] / r["pytorch_peak_mb"], 4)
        r["fwd_savings"] = round(1 - r["flashmlp_fwd_mb"] / r["pytorch_fwd_mb"], 4)
        pub = MEMORY_PUBLISHED_MB[(H, B, D, E)]
        r["reference_published_mb"] = {"pytorch_peak": pub[0], "triton_peak": pub[1], "pytorch_fwd": pub[2],
                                       "triton_fwd": pub[3]}
        rows.append(r)
    return rows


def peak_memory(x, w1, w2, do, activation):
    """Peak allocated MB of one fwd+bwd (example.py:142-200 method) for FlashMLP (both backward
    forms) and for the unfused PyTorch path, plus the device memory held outside torch's
    allocator by the library (its code objects; fmlp_bwd_noalloc's static scratch is a code
    object of its own, loaded at the first no-alloc call, measured last)."""
    import torch

    import flashmlp_amd as fm
    from flashmlp_amd import _lib

    def flash():
        o = fm.flashmlp_fwd(x, w1, w2, activation)
        return o, (lambda: fm.flashmlp_bwd(x, w1, w2, do, activation))

    def flash_recompute():  # the recompute-only backward (no stored dZ)
        o = fm.flashmlp_fwd(x, w1, w2, activation)
        return o, (lambda: fm.flashmlp_bwd(x, w1, w2, do, activation, recompute=True))

    def unfused():
        o, z, h = unfused_fwd(x, w1, w2, activation)
        return o, (lambda: unfused_bwd(x, w1, w2, do, z, h, activation))

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

    # fmlp_bwd_noalloc's static scratch: device memory taken by the first no-alloc call (no
    # torch allocation happens in it), i.e. what a process using that entry point holds beyond
    # the peaks above, which were measured before it was loaded
    H, B, D = x.shape
    E = w1.shape[2]
    hs, bs = 1, min(B, 512)
    xs, dos = x[:hs, :bs].contiguous(), do[:hs, :bs].contiguous()
    w1s, w2s = w1[:hs].contiguous(), w2[:hs].contiguous()
    gs = (torch.empty_like(xs), torch.empty_like(w1s), torch.empty_like(w2s))
    code = {torch.bfloat16: _lib.FMLP_DTYPE_BF16, torch.float16: _lib.FMLP_DTYPE_F16}.get(x.dtype, _lib.FMLP_DTYPE_F32)
    torch.cuda.synchronize()
    used0 = _device_used()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    st = _lib.lib().fmlp_bwd_noalloc(p(xs), p(w1s), p(w2s), p(dos), *(p(t) for t in gs), hs, bs, D, E, code,
                                     _lib.ACT_CODES[activation], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, "backward (no allocation)")
    torch.cuda.synchronize()
    out["noalloc_scratch_device_mb"] = round((_device_used() - used0) / 2 ** 20, 1)
    out["noalloc_scratch_note"] = ("held per device only by processes that call fmlp_bwd_noalloc (loaded at "
                                   "its first call); not part of the peaks above")
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


def autograd_step_ms(x, w1, w2, do, act, warmup=5, iters=50):
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


def time_steps(fwd, bwd, steps, warmup):
    """W untimed steps, then K timed steps of fwd() then bwd() (bwd may be None) issued back to
    back with nothing between them: wall-clock ms per step, synchronised at both ends (two HIP
    events bracket the region, for its GPU-side duration). Then K more steps with a HIP event
    recorded around each call, on the stream the kernels run on: the mean fwd / bwd durations.
    The per-call events stay out of the timed steps: each one recorded between two kernels
    leaves the GPU idle for several microseconds (measured on MI355X: 5-10 us per event)."""
    import torch

    for _ in range(warmup):
        fwd()
        if bwd is not None:
            bwd()
    torch.cuda.synchronize()
    outs = None
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_start.record()
    for _ in range(steps):
        o = fwd()
        g = bwd() if bwd is not None else None
        outs = (o, g)
    e_end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    gpu = e_start.elapsed_time(e_end) / steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for k in range(steps):
        ev[k][0].record()
        fwd()
        ev[k][1].record()
        if bwd is not None:
            bwd()
        ev[k][2].record()
    torch.cuda.synchronize()
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / steps if bwd is not None else 0.0
    time_steps.gpu_ms_per_step = gpu
    return wall, fwd_ms, bwd_ms, outs


def _finite(outs):
    import torch

    o, g = outs
    ok = bool(torch.isfinite(o.float()).all())
    if g is not None:
        ok = ok and all(bool(torch.isfinite(t.float()).all()) for t in g if t is not None)
    return ok


def _bwd_form(H, B, D, E, dt_name, act, accurate_dw=False, recompute=False):
    from flashmlp_amd import _lib

    code = {"bf16": _lib.FMLP_DTYPE_BF16, "f16": _lib.FMLP_DTYPE_F16, "f32": _lib.FMLP_DTYPE_F32}[dt_name]
    if not _lib.lib().fmlp_shape_tuned(D, E, code):
        # dense 16-bit D = 256 (E % 8 == 0): the D = 256 dX and dW programs
        return "dx256+dw256" if D == 256 and dt_name != "f32" and E % 8 == 0 else "generic"
    code |= (_lib.FMLP_DW_HILO if accurate_dw else 0) | (_lib.FMLP_BWD_RECOMPUTE if recompute else 0)
    return "stored-dZ" if _lib.lib().fmlp_bwd_stores_dz(H, B, D, E, code, _lib.ACT_CODES[act]) else "recompute"


def _summary(H, B, D, E, dt_name, act, fwd_only, wall, fwd_ms, bwd_ms, bwd_form):
    """Per-configuration figures: times, TFLOP/s (12u per step, 4u forward, 8u backward), % of
    the dtype's dense MFMA peak, and algorithmic HBM GB/s of each call."""
    u = float(H) * B * D * E
    s = _es(dt_name)
    peak = PEAK_TFLOPS[dt_name]
    step_flops = (4 if fwd_only else 12) * u
    r = {"H": H, "B": B, "D": D, "E": E, "dtype": dt_name, "activation": act or "linear",
         "ms_per_step": round(wall, 4), "tflops": round(step_flops / (wall * 1e-3) / 1e12, 2),
         "pct_of_peak": round(100 * step_flops / (wall * 1e-3) / 1e12 / peak, 2), "peak_tflops": peak,
         "fwd_ms": round(fwd_ms, 4), "fwd_tflops": round(4 * u / (fwd_ms * 1e-3) / 1e12, 2),
         "fwd_hbm_gbs": round((2 * H * B * D + 2 * H * D * E) * s / (fwd_ms * 1e-3) / 1e9, 1)}
    if not fwd_only:
        r.update({"bwd_ms": round(bwd_ms, 4), "bwd_tflops": round(8 * u / (bwd_ms * 1e-3) / 1e12, 2),
                  "bwd_hbm_gbs": round((3 * H * B * D + 4 * H * D * E) * s / (bwd_ms * 1e-3) / 1e9, 1),
                  "bwd_form": bwd_form})
    return r


def _peak_mb(run):
    """Peak allocated MB of run() over the memory allocated before it (example.py:142-200's
    method), after one unmeasured run."""
    import torch

    run()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out = run()
    torch.cuda.synchronize()
    peak = (torch.cuda.max_memory_allocated() - base) / 2 ** 20
    del out
    torch.cuda.empty_cache()
    return round(peak, 1)


def _cpu_config_ms(H, B, D, E, act, x_std, fwd_only):
    """The CPU oracle (torch fp32 autograd of the restated reference path, the forward alone for
    a forward-only workload) on one head of the workload, median of 3 after a warm-up, scaled to
    all H heads (heads are independent): milliseconds per full step."""
    import torch

    from oracle import reference
    from oracle.inputs import make_inputs

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    x, w1, w2, do = make_inputs(1, B, D, E, torch.float32, x_std, seed=0)
    if fwd_only:
        f = lambda: reference.torch_fwd(x, w1, w2, act)
    else:
        f = lambda: reference.autograd_grads(x, w1, w2, do, act)
    f()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        f()
        ts.append(time.perf_counter() - t0)
    return round(statistics.median(ts) * 1e3 * H, 2)


def run_config(name, steps, warmup, **bwd_kw):
    """One workload's step timed on freshly drawn inputs (the `configs` pass)."""
    import torch

    import flashmlp_amd as fm

    H, B, D, E, dt_name, act, x_std, fwd_only = WORKLOADS[name]
    x, w1, w2, do = make_gpu_inputs(H, B, D, E, _torch_dtype(dt_name), x_std)
    fwd = lambda: fm.flashmlp_fwd(x, w1, w2, act)
    bwd = None if fwd_only else (lambda: fm.flashmlp_bwd(x, w1, w2, do, act, **bwd_kw))
    wall, f_ms, b_ms, outs = time_steps(fwd, bwd, steps, warmup)
    r = _summary(H, B, D, E, dt_name, act, fwd_only, wall, f_ms, b_ms,
                 None if fwd_only else _bwd_form(H, B, D, E, dt_name, act, **bwd_kw))
    r["finite"] = _finite(outs)
    if fwd_only:
        r["note"] = "forward only (inference sweep)"
    del x, w1, w2, do, outs
    torch.cuda.empty_cache()
    return r


def config_extras(name):
    """A workload's peak allocated MB of one step against the unfused PyTorch path, and the CPU
    oracle's time per step on the host's cores (one head, scaled to all). Run after every
    configuration is timed: the oracle's host threads keep spinning for a while after it, which
    would slow the launches of the next timed steps."""
    import torch

    import flashmlp_amd as fm

    H, B, D, E, dt_name, act, x_std, fwd_only = WORKLOADS[name]
    x, w1, w2, do = make_gpu_inputs(H, B, D, E, _torch_dtype(dt_name), x_std)
    fwd = lambda: fm.flashmlp_fwd(x, w1, w2, act)
    bwd = lambda: fm.flashmlp_bwd(x, w1, w2, do, act)
    r = {}
    if fwd_only:
        r["peak_mb"] = _peak_mb(fwd)
        r["unfused_peak_mb"] = _peak_mb(lambda: unfused_fwd(x, w1, w2, act))
    else:
        r["peak_mb"] = _peak_mb(lambda: (fwd(), bwd()))

        def unfused():
            o, z, h = unfused_fwd(x, w1, w2, act)
            return o, unfused_bwd(x, w1, w2, do, z, h, act)

        r["unfused_peak_mb"] = _peak_mb(unfused)
    r["peak_savings"] = round(1 - r["peak_mb"] / r["unfused_peak_mb"], 4)
    del x, w1, w2, do
    torch.cuda.empty_cache()
    r["cpu_ms"] = _cpu_config_ms(H, B, D, E, act, x_std, fwd_only)
    r["cpu_note"] = ("CPU oracle (torch fp32 autograd), one head timed and scaled to all, "
                     f"{len(os.sched_getaffinity(0))} cores")
    return r


def vs_unfused(x4, w14, w24, do4, act4, steps, warmup):
    """FlashMLP against the unfused PyTorch path on the same GPU and inputs: forward, and
    forward + backward (direct calls for both, no autograd), at cfg4 and at performance.md's
    shapes (bf16 SiLU, X~N(0,1/D) as example.py draws it, module init scales)."""
    import torch

    import flashmlp_amd as fm

    def pair(x, w1, w2, do, act, k, w):
        H, B, D = x.shape
        E = w1.shape[2]
        u = float(H) * B * D * E
        f_fwd = lambda: fm.flashmlp_fwd(x, w1, w2, act)
        f_bwd = lambda: fm.flashmlp_bwd(x, w1, w2, do, act)

        def t_step():
            o, z, h = unfused_fwd(x, w1, w2, act)
            return unfused_bwd(x, w1, w2, do, z, h, act)

        ff = time_steps(f_fwd, None, k, w)[0]
        fb = time_steps(f_fwd, f_bwd, k, w)[0]
        tf = time_steps(lambda: unfused_fwd(x, w1, w2, act)[0], None, k, w)[0]
        for _ in range(w):
            t_step()
        tb = _wall_ms(t_step, k)
        return {"H": H, "B": B, "D": D, "E": E, "flashmlp_fwd_ms": round(ff, 4),
                "flashmlp_fwd_bwd_ms": round(fb, 4), "pytorch_fwd_ms": round(tf, 4),
                "pytorch_fwd_bwd_ms": round(tb, 4), "speedup_fwd": round(tf / ff, 2),
                "speedup_fwd_bwd": round(tb / fb, 2),
                "flashmlp_fwd_bwd_tflops": round(12 * u / (fb * 1e-3) / 1e12, 1),
                "pytorch_fwd_bwd_tflops": round(12 * u / (tb * 1e-3) / 1e12, 1)}

    res = {"method": "wall clock of direct calls, W warmup then K steps, synchronised at both ends; unfused = "
                     "bmm -> activation -> bmm keeping Z and h, backward as five bmm on contiguous operands "
                     "(flashmlp.py:689-723)",
           "cfg4": pair(x4, w14, w24, do4, act4, steps, warmup)}
    rows = []
    for H, B, D, E in EXAMPLE_SHAPES:
        g = torch.Generator(device="cuda").manual_seed(0)
        f = dict(device="cuda", dtype=torch.float32, generator=g)
        x = (torch.randn(H, B, D, **f) / D ** 0.5).bfloat16()
        w1 = (torch.randn(H, D, E, **f) / E ** 0.5).bfloat16()  # FlashMLP's init (flashmlp.py:586-591)
        w2 = (torch.randn(H, E, D, **f) / D ** 0.5).bfloat16()
        do = torch.randn(H, B, D, **f).bfloat16()
        r = pair(x, w1, w2, do, "silu", 100, 10)
        pub = EXAMPLE_PUBLISHED_MS[(H, B, D, E)]
        r["reference_published_ms"] = {"triton_fwd": pub[0], "triton_fwd_bwd": pub[1], "hardware": "unstated"}
        rows.append(r)
    res["performance_md_shapes"] = rows
    return res


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
    # the dW role's mix: LDS bytes and SiLU-backward elements per MFMA, at one or two waves per
    # SIMD (the grid holds that many workgroups of four waves per CU)
    lib.fmlp_ceiling_act_mix.restype = ctypes.c_int
    act_mix = {}
    for lds8, el2, wps in ((0, 1, 2), (0, 1, 1), (2, 1, 2), (2, 1, 1), (3, 1, 2), (3, 1, 1),
                           (0, 2, 2), (0, 2, 1), (2, 2, 2), (2, 2, 1)):
        g = wps * ncu

        def call_act():
            r = lib.fmlp_ceiling_act_mix(ctypes.c_void_p(out.data_ptr()), mix_iters, lds8, el2, wps, g, st)
            if r != 0:
                raise RuntimeError(f"fmlp_ceiling_act_mix: hip error {r}")
        for _ in range(args.warmup + 20):
            call_act()
        torch.cuda.synchronize()
        ms = _wall_ms(call_act, max(args.steps, 50))
        act_mix[f"lds{lds8 * 512}_elem{el2 / 2:g}_wps{wps}"] = round(g * 4 * mix_iters * 16 * 32768.0 / (ms * 1e-3) / 1e12, 1)
    peak = PEAK_TFLOPS["bf16"]
    line = {"metric": "sustained bf16 MFMA rate (v_mfma_f32_32x32x16_bf16, register operands)", "workload": "mfma_ceiling",
            "unit": "TFLOP/s", "peak": peak, "random": res["random"], "zero": res["zero"],
            "random_frac_of_peak": round(res["random"]["tflops"] / peak, 4),
            "with_per_mfma_work": {"unit": "TFLOP/s", "lds": "1 KB LDS read per wave per MFMA (A operand)",
                                   "chains": "sigmoid-like VALU chains (mul, exp, add, rcp) per MFMA", **mix},
            "dw_role_mix": {"unit": "TFLOP/s", "lds": "LDS bytes per wave per MFMA",
                            "elem": "SiLU-backward elements (h and dZ, packed to bf16) per lane per MFMA",
                            "wps": "waves per SIMD", **act_mix},
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
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the autograd-step and host-overhead timings, the cfg4 forms, the configs pass "
                         "and the unfused comparison (headline timing only)")
    ap.add_argument("--accurate-dw", action="store_true",
                    help="time the backward in its dW accuracy mode (h and dZ as hi + lo terms)")
    ap.add_argument("--recompute", action="store_true", help="time the backward in its recompute-only form")
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
    s = _es(dt_name)
    bwd_kw = dict(accurate_dw=args.accurate_dw, recompute=args.recompute)

    fwd = lambda: fm.flashmlp_fwd(x, w1, w2, act)
    bwd = None if fwd_only else (lambda: fm.flashmlp_bwd(x, w1, w2, do, act, **bwd_kw))
    ms_per_step, fwd_ms, bwd_ms, outs = time_steps(fwd, bwd, args.steps, args.warmup)
    gpu_ms = time_steps.gpu_ms_per_step
    assert _finite(outs), "non-finite outputs"
    del outs

    K = args.steps
    u = float(H) * B * D * E
    flops = (4 if fwd_only else 12) * u
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
    if args.recompute:
        step_name += " (recompute-only backward)"
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "gpu_ms_per_step": round(gpu_ms, 4),
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
            "kernel": "fmlp_fwd: fmlp::fwd_kernel",
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
        form = _bwd_form(H, B, D, E, dt_name, act, **bwd_kw)
        line["bwd_form"] = form
        kernels = {"stored-dZ": "fmlp::dw2_kernel (storing dZ), fmlp::dxg_kernel",
                   "recompute": "fmlp::bwd_kernel (dW and dX programs)",
                   "generic": "fmlp::gen_dw_kernel, fmlp::gen_dx_kernel",
                   "dx256+dw256": "fmlp::dx256_kernel, fmlp::dw256_kernel"}[form]
        line["roofline"] = {
            "kernel": f"fmlp_bwd ({form}): {kernels}",
            "bound": "mfma",
            "achieved": round(bwd_tf, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / peak, 4),
            "traffic": traffic_from_profile("bwd", args.workload) if not (args.accurate_dw or args.recompute) else None,
            "algorithmic_flops_per_launch": 8 * u,
            "algorithmic_bytes_per_launch": bwd_bytes,
            "avg_launch_ms": round(bwd_ms, 4),
        }
    if not args.no_extra:
        line["host_us_per_call"] = {"fwd": round(host_us_per_call(fwd), 2)}
        if not fwd_only:
            line["host_us_per_call"]["bwd"] = round(host_us_per_call(bwd), 2)
            line["autograd_ms_per_step"] = round(autograd_step_ms(x, w1, w2, do, act), 4)
        if args.workload == "cfg4" and not (args.accurate_dw or args.recompute):
            # the same step in the north star's recompute-only form and in the dW accuracy mode
            forms = {}
            for name, kw in (("recompute", dict(recompute=True)), ("accurate_dw", dict(accurate_dw=True)),
                             ("recompute_accurate_dw", dict(recompute=True, accurate_dw=True))):
                wall, f_ms, b_ms, o = time_steps(fwd, lambda: fm.flashmlp_bwd(x, w1, w2, do, act, **kw),
                                                 K, max(3, min(args.warmup, 5)))
                r = _summary(H, B, D, E, dt_name, act, False, wall, f_ms, b_ms, _bwd_form(H, B, D, E, dt_name, act, **kw))
                forms[name] = {k: r[k] for k in ("ms_per_step", "tflops", "pct_of_peak", "fwd_ms", "bwd_ms",
                                                 "bwd_tflops", "bwd_form")}
                forms[name]["finite"] = _finite(o)
                del o
            line["cfg4_forms"] = forms
            # short configurations get more steps (each is well under a millisecond)
            line["configs"] = {name: run_config(name, 10 if name in ("cfg1_fp32", "d256") else 50,
                                                3 if name in ("cfg1_fp32", "d256") else 10)
                               for name in CONFIG_PASS}
            line["vs_pytorch_unfused"] = vs_unfused(x, w1, w2, do, act, 10, 3)
    if not args.no_memory and not fwd_only:
        line["memory"] = peak_memory(x, w1, w2, do, act)
        if args.workload == "cfg4" and not args.no_extra:
            line["memory"]["performance_md_shapes"] = module_memory()
    if "configs" in line and not (args.no_memory or args.no_cpu):
        for name in CONFIG_PASS:
            line["configs"][name].update(config_extras(name))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(H, B, D, E, act, x_std)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
