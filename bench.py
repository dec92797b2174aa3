"""Benchmark of mtorch's SD-UNet hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload resnet|linear_gelu|unet|copy_calibration|suite|vendor]
                    [--no-cpu] [--no-extras]

Default workload (fp16 leg): the SD ResNet sub-block on a 64x64
latent at batch 2 -- x[2,320,64,64] -> GroupNorm(32, eps 1e-5, affine) -> SiLU ->
conv2d 3x3 s1 p1 320->320 (+bias) -> + x -- with inputs and parameters drawn from mtorch's
generator (seed 0): x ~ N(0,1), gamma = 1 + 0.1 N(0,1), beta = 0.1 N(0,1), conv weight
kaiming_uniform_(a=sqrt 5), bias U(+-1/sqrt(2880)); all drawn in fp32 and cast to fp16.

The same line carries the rest of the headline metric: the configs[4] SD-1.5 UNet step at
batch 2 (unet_ms_per_step, graph-replayed) and the configs[0]/[2]/[3] contractions (TFLOP/s and
MFMA fraction per op, under "configs").

One step = one pass of the block over the resident batch.  The timed region is K steps
bracketed by device synchronisation; HIP events on the device stream time the whole step and,
separately, the conv GEMM launch (the dominant kernel) for the roofline object.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"fp16_mfma_tflops": 2516.6, "fp32_tflops": 157.3, "hbm_gbs": 8000.0}
CPU_CHANNELS = 128  # output channels of the CPU-baseline conv sample


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _time_events(fn, reps):
    import mtorch_amd as mt

    start, end = mt.cuda.Event(), mt.cuda.Event()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    mt.cuda.synchronize()
    return start.elapsed_time(end) / reps


# ------------------------------------------------------------------------------ workloads


def resnet_inputs(mt):
    mt.manual_seed(0)
    x = mt.randn(2, 320, 64, 64)
    gamma = mt.randn(320)
    beta = mt.randn(320)
    w = mt.empty(320, 320, 3, 3)
    mt.nn.init.kaiming_uniform_(w, a=math.sqrt(5))
    bound = 1.0 / math.sqrt(320 * 9)
    b = mt.empty(320).uniform_(-bound, bound)
    return x, gamma, beta, w, b


def _traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc summaries under
    profiles/ (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the copy-kernel
    calibration recorded in the same file), or None when no summary is present."""
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel_key}.md")
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def run_resnet(args):
    """One step = GroupNorm(32)+SiLU written channels-last, then the implicit-GEMM conv with bias
    and residual, through the C ABI exactly as F.group_norm_silu_conv2d issues it.  HIP events
    on the library's stream time `steps` steps captured into one HIP graph and replayed (and,
    for comparison, the same steps launched eagerly), and the conv launches alone the same way."""
    import ctypes

    import mtorch_amd as mt
    from mtorch_amd import _lib, _ops
    from mtorch_amd import _tensor as T

    x, gamma, beta, w, b = resnet_inputs(mt)
    # gamma = 1 + 0.1 N(0,1), beta = 0.1 N(0,1): formed on the device in fp32, then cast.
    xd = x.to("cuda").half()
    gd = (gamma.to("cuda") * 0.1 + 1.0).half()
    bd = (beta.to("cuda") * 0.1).half()
    wd = w.to("cuda").half()
    bbd = b.to("cuda").half()
    L = _lib.lib()
    B, C, H, W, O = 2, 320, 64, 64, 320
    wp = _ops._conv_packed_weight(wd, 0, O, C, 3, 3)
    xn = T._DeviceBuffer(B * H * W * C * 2, 0)
    y = mt.empty(B, O, H, W, dtype=mt.float16, device="cuda")
    ev = [(mt.cuda.Event(), mt.cuda.Event()) for _ in range(args.steps)]

    def step(marks=None):
        _lib.check(L.mthip_group_norm_nhwc(0, _lib.F16, xd.data_ptr(), gd.data_ptr(), bd.data_ptr(), xn.ptr, B, C,
                                           H * W, 32, 1e-5, 1, _lib.F16))
        if marks:
            marks[0].record()
        _lib.check(L.mthip_conv2d_nhwc(0, _lib.F16, xn.ptr, wp, bbd.data_ptr(), y.data_ptr(), B, C, H, W, O, 3, 3,
                                       1, 1, 1, 1, 1, 1, xd.data_ptr(), None, 0))
        if marks:
            marks[1].record()

    def conv():
        _lib.check(L.mthip_conv2d_nhwc(0, _lib.F16, xn.ptr, wp, bbd.data_ptr(), y.data_ptr(), B, C, H, W, O, 3, 3,
                                       1, 1, 1, 1, 1, 1, xd.data_ptr(), None, 0))

    def replayed(fn):
        """(ms of one replay, wall ms) of a HIP graph of `steps` back-to-back fn() calls, after
        one untimed replay: the device runs the calls back to back whatever the host's launch
        rate."""
        g = mt.cuda.CUDAGraph()
        with mt.cuda.graph(g):
            for _ in range(args.steps):
                fn()
        g.replay()
        mt.cuda.synchronize()
        e0, e1 = mt.cuda.Event(), mt.cuda.Event()
        t0 = time.perf_counter()
        e0.record()
        g.replay()
        e1.record()
        mt.cuda.synchronize()
        return e0.elapsed_time(e1), (time.perf_counter() - t0) * 1e3

    for _ in range(args.warmup):
        step()
    mt.cuda.synchronize()
    # The timed region: `steps` steps captured into one graph and replayed once.
    ms, wall = replayed(step)
    ms_step, wall_ms = ms / args.steps, wall / args.steps
    # The same steps launched eagerly from the host, for comparison.
    start, end = mt.cuda.Event(), mt.cuda.Event()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    mt.cuda.synchronize()
    eager_ms_step = start.elapsed_time(end) / args.steps
    # An untimed eager run with an event pair around each conv launch: in a step that pair also
    # spans the conv's dispatch after the GroupNorm (the event between them waits for the
    # GroupNorm to finish), and the event records themselves separate the launches, so they stay
    # out of the timed steps above.  The roofline uses `steps` back-to-back conv launches
    # replayed as one graph, which is the kernel's own duration as rocprofv3's kernel trace
    # reports it.
    for i in range(args.steps):
        step(ev[i])
    mt.cuda.synchronize()
    conv_in_step_ms = sum(a.elapsed_time(b_) for a, b_ in ev) / args.steps
    conv_ms = replayed(conv)[0] / args.steps
    flops = 2.0 * B * H * W * O * C * 9  # 15.10 GFLOP per step (the conv; GN/SiLU/add are not counted)
    value = flops / (ms_step * 1e-3) / 1e12
    conv_tflops = flops / (conv_ms * 1e-3) / 1e12
    out = {
        "metric": "SD ResNet sub-block (GN32+SiLU+conv3x3 320->320+residual) fp16 TFLOP/s, batch 2, 64x64",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "wall_ms_per_step": round(wall_ms, 4),
        "eager_ms_per_step": round(eager_ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (mtorch generator, seed 0)",
        "config": {"workload": "configs[1] ResNet sub-block fp16: x[2,320,64,64], GN(32), SiLU, conv3x3 320->320, residual",
                   "batch": 2, "channels": 320, "hw": [64, 64]},
        "roofline": {
            "kernel": "conv3x3 launch: conv3x3_halo_kernel<80 channels x 2 rows x 64, 6-stage weight ring, "
                      "4 compute + 2 producer waves> (input halo staged once per 64-channel block and reused "
                      "by the 9 taps; bias and residual fused in the epilogue)",
            "bound": "mfma",
            "achieved": round(conv_tflops, 3),
            "peak": PEAK["fp16_mfma_tflops"],
            "unit": "TFLOP/s",
            "frac": round(conv_tflops / PEAK["fp16_mfma_tflops"], 4),
            "traffic": _traffic("conv_halo_resnet_fp16"),
            "kernel_ms": round(conv_ms, 5),
            "kernel_ms_in_step": round(conv_in_step_ms, 5),
        },
    }
    if args.cpu:
        out["cpu_baseline"] = cpu_baseline_resnet(x, gamma, beta, w, b)
    if args.extras:
        out.update(headline_extras(args))
        if args.cpu:
            out["cpu_baselines"] = cpu_baselines_extra(out["cpu_baseline"])
    return out


def headline_extras(args):
    """The rest of BASELINE.json's metric on the same line: the configs[4] UNet step (ms at
    batch 2, graph-replayed) and the configs[0], [2], [3] contractions (TFLOP/s and fraction of
    the MFMA peak that bounds each), every op graph-replayed x20 at its SD shape."""
    import mtorch_amd as mt
    from mtorch_amd import sd_unet

    unet = run_unet(argparse.Namespace(steps=max(args.steps // 2, 5), warmup=max(args.warmup, 2)))
    extras = {"unet_ms_per_step": unet["ms_per_step"], "unet_tflops": unet["tflops"],
              "unet_mfma_frac": unet["mfma_frac"], "unet_tflop_per_step": unet["unet_tflop_per_step"]}
    del unet
    F = mt.nn.functional
    mt.manual_seed(0)
    rows = {}

    def rnd(*shape, dt=mt.float16, scale=1.0):
        t = mt.randn(*shape).to("cuda")
        return (t * scale if scale != 1.0 else t).to(dt)

    def put(key, r):
        rows[key] = {"us": r["us"], "tflops": r["tflops"], "frac": r["frac"]}

    bound = 1.0 / math.sqrt(320)
    x = mt.randn(8192, 320).to("cuda")
    w = mt.empty(1280, 320).uniform_(-bound, bound).to("cuda")
    b = mt.empty(1280).uniform_(-bound, bound).to("cuda")
    put("c0_linear_gelu_fp32", _suite_row("c0", lambda: F.linear_gelu(x, w, b), 20, flops=2.0 * 8192 * 1280 * 320,
                                          peak=PEAK["fp32_tflops"], quiet=True))
    for L, E in ((4096, 40), (1024, 80), (256, 160)):
        q, k, v = rnd(2, 8, L, E, scale=1.0 / math.sqrt(E)), rnd(2, 8, L, E), rnd(2, 8, L, E)
        put(f"c2_self_{L}x{E}", _suite_row("c2", lambda: F.scaled_dot_product_attention(q, k, v), 20,
                                           flops=4.0 * 2 * 8 * L * L * E, quiet=True))
    st = sd_unet.SpatialTransformer(sd_unet._Init("cuda"), 640)
    xt, ctx = rnd(2, 640, 32, 32), rnd(2, 77, 768)
    put("c3_spatial_transformer", _suite_row("c3", lambda: st(xt, ctx), 5, flops=39.63e9, quiet=True))
    del st, xt, ctx
    # configs[1], fp32 leg: the same sub-block in fp32 (GN+SiLU written channels-last, conv3x3 on
    # the fp32 MFMA GEMM with bias and residual fused), priced against the fp32 peak.
    x32, g32, b32 = rnd(2, 320, 64, 64, dt=mt.float32), rnd(320, dt=mt.float32), rnd(320, dt=mt.float32)
    w32, bb32 = rnd(320, 320, 3, 3, dt=mt.float32, scale=0.02), rnd(320, dt=mt.float32, scale=0.02)
    conv_flops = 2.0 * 2 * 4096 * 320 * 2880
    put("c1_resnet_fp32", _suite_row("c1", lambda: F.group_norm_silu_conv2d(x32, 32, g32, b32, 1e-5, w32, bb32,
                                                                          padding=1, residual=x32), 10,
                                     flops=conv_flops, peak=PEAK["fp32_tflops"], quiet=True))
    put("c1_conv3x3_fp32", _suite_row("c1", lambda: F.conv2d(x32, w32, bb32, padding=1), 10, flops=conv_flops,
                                      peak=PEAK["fp32_tflops"], quiet=True))
    extras["configs"] = rows
    return extras


def cpu_baselines_extra(resnet_cpu):
    """CPU baselines of the other configs on the same line, 1 core, the oracle's restatement of
    mtorch's Linux path (kind "port"):
      * fp32 linear + erf-GELU on 2048 of the 8192 rows (the rate scales: rows are
        independent);
      * a per-op-family estimate of one UNet step, labelled as such -- each family's
        FLOP (sd_unet.unet_flops) divided by the oracle's measured 1-core rate for it: 3x3 convs
        at the rate of the main sample (cpu_baseline), 1x1 convs, linears and attention on
        bounded fp16 samples; GroupNorm / LayerNorm / softmax / elementwise ops (linear in the
        data, no contraction) are left out."""
    import numpy as np

    import oracle
    from mtorch_amd import sd_unet

    os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    r = oracle.Rng(0)

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    out = {}
    x = r.randn((2048, 320), "float32", 0.0, 1.0)
    bound = 1.0 / math.sqrt(320)
    w = r.uniform((1280, 320), -bound, bound, "float32")
    b = r.uniform((1280,), -bound, bound, "float32")
    dt = timed(lambda: oracle.gelu(oracle.linear(x, w, b)))
    fl = 2.0 * 2048 * 1280 * 320
    out["c0_linear_gelu_fp32"] = {"value": round(fl / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                                  "sample": f"fp32 linear+GELU on 2048/8192 rows of X[8192,320].W[1280,320]^T+b; "
                                            f"{dt:.2f} s on 1 core", "seconds": round(dt, 3)}
    rates = {"conv3x3": resnet_cpu["value"] * 1e12}
    xh, wh = r.randn((512, 640), "float16", 0.0, 1.0), r.randn((640, 640), "float16", 0.0, 0.05)
    rates["linear"] = 2.0 * 512 * 640 * 640 / timed(lambda: oracle.linear(xh, wh))
    xc, wc = r.randn((1, 640, 16, 16), "float16", 0.0, 1.0), r.randn((640, 640, 1, 1), "float16", 0.0, 0.05)
    rates["conv1x1"] = 2.0 * 256 * 640 * 640 / timed(lambda: oracle.conv2d(xc, wc))
    q = r.randn((1, 1, 512, 80), "float16", 0.0, 1.0)
    k, v = r.randn((1, 1, 1024, 80), "float16", 0.0, 1.0), r.randn((1, 1, 1024, 80), "float16", 0.0, 1.0)
    rates["attention"] = 4.0 * 512 * 1024 * 80 / timed(lambda: oracle.sdpa(q, k, v))
    parts = {}
    total = sd_unet.unet_flops(parts=parts)
    est = {f: parts[f] / rates[f] for f in parts}
    secs = sum(est.values())
    out["c4_unet_step_estimate"] = {
        "value": round(secs, 1), "unit": "s per UNet step (estimate)", "cores": 1, "kind": "port",
        "sample": "per-op-family sum: each family's FLOP of the step / the oracle's 1-core rate on a bounded fp16 "
                  "sample (3x3 conv: the main cpu_baseline sample; linear [512,640]x[640,640]; 1x1 conv "
                  "[1,640,16,16]; attention [512 queries x 1024 keys x 80]); norm/softmax/elementwise excluded",
        "family_gflop": {f: round(parts[f] / 1e9, 1) for f in parts},
        "family_gflops_rate": {f: round(rates[f] / 1e9, 3) for f in rates},
        "family_seconds": {f: round(est[f], 1) for f in est},
        "tflop_per_step": round(total / 1e12, 4),
    }
    return out


def run_copy_calibration(args):
    """A plain streaming kernel of known size (fp32 negation over 256 MiB: 256 MiB read and
    256 MiB written per launch) for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import mtorch_amd as mt
    from mtorch_amd import _lib

    n = 64 << 20
    x = mt.zeros(n, device="cuda")
    y = mt.empty(n, device="cuda")
    L = _lib.lib()
    for _ in range(args.warmup + args.steps):
        _lib.check(L.mthip_unary(0, 6, _lib.F32, x.data_ptr(), y.data_ptr(), n))
    mt.cuda.synchronize()
    return {"metric": "copy calibration", "bytes_read_per_launch": n * 4, "bytes_written_per_launch": n * 4,
            "launches": args.warmup + args.steps}


def cpu_baseline_resnet(x, gamma, beta, w, b):
    """The oracle's restatement of mtorch's Linux fp16 path, one core, on a bounded sample:
    GroupNorm+SiLU on the full input and the conv for CPU_CHANNELS of the 320 output channels
    (about 10 s of CPU work); the rate is the sample's conv FLOP over its time."""
    import numpy as np

    import oracle

    xh = oracle.f2h(x.numpy())
    g = oracle.f2h((gamma.numpy().astype(np.float64) * 0.1 + 1.0).astype(np.float32))
    be = oracle.f2h((beta.numpy().astype(np.float64) * 0.1).astype(np.float32))
    wh = oracle.f2h(w.numpy())[:CPU_CHANNELS]
    bh = oracle.f2h(b.numpy())[:CPU_CHANNELS]
    os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    t0 = time.perf_counter()
    h = oracle.silu(oracle.group_norm(xh, 32, g, be, 1e-5))
    y = oracle.conv2d(h, wh, bh, padding=1)
    oracle.binary(y, np.ascontiguousarray(xh[:, :CPU_CHANNELS]), "add")
    dt = time.perf_counter() - t0
    flops = 2.0 * 2 * CPU_CHANNELS * 64 * 64 * 320 * 9
    return {
        "value": round(flops / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": f"fp16 GN32+SiLU on the full [2,320,64,64] input + conv3x3 for {CPU_CHANNELS}/320 output channels "
                  f"+ residual; {dt:.2f} s on 1 core of {_cpu_model()} (nproc {os.cpu_count()})",
        "seconds": round(dt, 3),
    }


def run_linear_gelu(args):
    """fp32 linear + GELU, X[8192,320] . W[1280,320]^T + b (erf GELU)."""
    import mtorch_amd as mt

    F = mt.nn.functional
    mt.manual_seed(0)
    x = mt.randn(8192, 320)
    bound = 1.0 / math.sqrt(320)
    w = mt.empty(1280, 320).uniform_(-bound, bound)
    b = mt.empty(1280).uniform_(-bound, bound)
    xd, wd, bd = x.to("cuda"), w.to("cuda"), b.to("cuda")

    def step():
        return F.linear_gelu(xd, wd, bd)

    for _ in range(args.warmup):
        step()
    mt.cuda.synchronize()
    ms = _time_events(step, args.steps)
    flops = 2.0 * 8192 * 1280 * 320
    value = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "fp32 linear+GELU TFLOP/s, X[8192,320].W[1280,320]^T+b",
        "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (mtorch generator, seed 0)",
        "config": {"workload": "configs[0] fp32 linear+GELU [8192,320]x[1280,320]^T"},
        "roofline": {"kernel": "gemm_kernel MODE_NT EPI_LINEAR (GELU fused)", "bound": "mfma",
                     "achieved": round(value, 3), "peak": PEAK["fp32_tflops"], "unit": "TFLOP/s",
                     "frac": round(value / PEAK["fp32_tflops"], 4), "traffic": None},
    }


def run_unet(args):
    """one SD-1.5-shaped UNet denoising step at batch 2 (latent [2,4,64,64], t = 500,
    context [2,77,768]; ~860 M parameters N(0, 0.02) in fp16, norms fp32 with upcast), captured
    once into a HIP graph and replayed; each replay is one full forward."""
    import mtorch_amd as mt
    from mtorch_amd import sd_unet

    t0 = time.perf_counter()
    model = sd_unet.UNet(seed=0, device="cuda")
    build_s = time.perf_counter() - t0
    mt.manual_seed(1)
    latent = mt.randn(2, 4, 64, 64).half().to("cuda")
    ctx = mt.randn(2, 77, 768).half().to("cuda")
    t = mt.tensor([500.0, 500.0]).to("cuda")
    model(latent, t, ctx)  # eager pass: packs the conv weights outside the graph
    mt.cuda.synchronize()
    t1 = time.perf_counter()
    model(latent, t, ctx)
    mt.cuda.synchronize()
    eager_ms = (time.perf_counter() - t1) * 1e3
    g = mt.cuda.CUDAGraph()
    with mt.cuda.graph(g):
        model(latent, t, ctx)
    for _ in range(args.warmup):
        g.replay()
    mt.cuda.synchronize()
    start, end = mt.cuda.Event(), mt.cuda.Event()
    start.record()
    for _ in range(args.steps):
        g.replay()
    end.record()
    mt.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    flops = sd_unet.unet_flops()
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "SD-1.5 UNet step ms, batch 2, 64x64 latent, fp16 (graph-replayed)",
        "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (mtorch generator: weights seed 0, inputs seed 1)",
        "config": {"workload": "configs[4] SD-1.5 UNet, batch 2, latent [2,4,64,64], context [2,77,768], t=500",
                   "params": sum(p.numel() for p in model.parameters())},
        "tflops": round(tflops, 2), "unet_tflop_per_step": round(flops / 1e12, 4),
        "mfma_frac": round(tflops / PEAK["fp16_mfma_tflops"], 4),
        "eager_ms_per_step": round(eager_ms, 2), "model_build_s": round(build_s, 1),
    }


def _suite_row(name, fn, reps, flops=None, nbytes=None, bound="mfma", peak=None, graph=True, quiet=False):
    """Time one op: a HIP graph of `reps` back-to-back calls replayed once (so launch gaps do
    not count against short kernels), averaged per call; then price it against its roofline."""
    import mtorch_amd as mt

    fn()
    mt.cuda.synchronize()
    if graph:
        g = mt.cuda.CUDAGraph()
        with mt.cuda.graph(g):
            for _ in range(reps):
                fn()
        g.replay()
        ms = _time_events(g.replay, 5) / reps
    else:
        ms = _time_events(fn, reps)
    row = {"op": name, "us": round(ms * 1e3, 2), "bound": bound}
    if flops is not None:
        row["tflops"] = round(flops / (ms * 1e-3) / 1e12, 2)
    if nbytes is not None:
        row["gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    if bound == "mfma":
        row["frac"] = round(row["tflops"] / (peak or PEAK["fp16_mfma_tflops"]), 4)
    else:
        row["frac"] = round(row["gbs"] / PEAK["hbm_gbs"], 4)
    if not quiet:
        print(json.dumps(row), file=sys.stderr, flush=True)
    return row


def run_suite(args):
    """Every op row of the hot path at its SD-1.5 shape (BASELINE.json configs[0]-[3]), each
    priced against the roofline that bounds it: contractions in TFLOP/s against MFMA peak,
    normalisation / softmax / elementwise in GB/s of algorithmic bytes (read once, written once)
    against HBM peak.  The HBM-bound ops are also timed on a 64x larger batch, where the
    working set no longer fits the 256 MB Infinity Cache and a launch lasts long enough for
    its ramp-up not to dominate."""
    import mtorch_amd as mt
    from mtorch_amd import sd_unet

    F = mt.nn.functional
    mt.manual_seed(0)
    reps = 20
    rows = []

    def rnd(*shape, dt=mt.float16, scale=1.0):
        t = mt.randn(*shape).to("cuda")
        if scale != 1.0:
            t = t * scale
        return t.to(dt)

    # linear + GELU, fp32 and fp16.
    for dt, peak, tag in ((mt.float32, PEAK["fp32_tflops"], "fp32"), (mt.float16, None, "fp16")):
        x, w, b = rnd(8192, 320, dt=dt), rnd(1280, 320, dt=dt, scale=0.05), rnd(1280, dt=dt, scale=0.05)
        rows.append(_suite_row(f"linear+gelu {tag} [8192,320]x[1280,320]^T", lambda: F.linear_gelu(x, w, b),
                               reps, flops=2.0 * 8192 * 1280 * 320, peak=peak))
    # the ResNet sub-block pieces.
    for dt, esz, tag in ((mt.float32, 4, "fp32"), (mt.float16, 2, "fp16")):
        for nb in (2, 128):
            x = rnd(nb, 320, 64, 64, dt=dt)
            g, bb = rnd(320, dt=dt), rnd(320, dt=dt)
            n = nb * 320 * 64 * 64
            rows.append(_suite_row(f"group_norm(32) {tag} [{nb},320,64,64]", lambda: F.group_norm(x, 32, g, bb, 1e-5),
                                   reps if nb == 2 else 3, nbytes=2 * n * esz, bound="hbm"))
            rows.append(_suite_row(f"group_norm(32)+silu {tag} [{nb},320,64,64]",
                                   lambda: F.group_norm_silu(x, 32, g, bb, 1e-5),
                                   reps if nb == 2 else 3, nbytes=2 * n * esz, bound="hbm"))
            y = rnd(nb, 320, 64, 64, dt=dt)
            rows.append(_suite_row(f"add {tag} [{nb},320,64,64]", lambda: x + y, reps if nb == 2 else 3,
                                   nbytes=3 * n * esz, bound="hbm"))
            rows.append(_suite_row(f"silu {tag} [{nb},320,64,64]", lambda: F.silu(x), reps if nb == 2 else 3,
                                   nbytes=2 * n * esz, bound="hbm"))
            rows.append(_suite_row(f"gelu {tag} [{nb},320,64,64]", lambda: F.gelu(x), reps if nb == 2 else 3,
                                   nbytes=2 * n * esz, bound="hbm"))
            del x, y
    xs = rnd(2, 320, 64, 64)
    ws, bs = rnd(320, 320, 3, 3, scale=0.02), rnd(320, scale=0.02)
    rows.append(_suite_row("conv2d 3x3 fp16 [2,320,64,64] 320->320", lambda: F.conv2d(xs, ws, bs, padding=1),
                           reps, flops=2.0 * 2 * 4096 * 320 * 2880))
    for C, hw in ((640, 32), (1280, 16), (1280, 8)):
        xc = rnd(2, C, hw, hw)
        wc, bc = rnd(C, C, 3, 3, scale=0.02), rnd(C, scale=0.02)
        rows.append(_suite_row(f"conv2d 3x3 fp16 [2,{C},{hw},{hw}] {C}->{C}",
                               lambda: F.conv2d(xc, wc, bc, padding=1), reps, flops=2.0 * 2 * hw * hw * C * C * 9))
    # attention, self and cross, at the three latent sizes.
    for L, C, E in ((4096, 320, 40), (1024, 640, 80), (256, 1280, 160)):
        q, k, v = rnd(2, 8, L, E), rnd(2, 8, L, E), rnd(2, 8, L, E)
        rows.append(_suite_row(f"sdpa self fp16 [2,8,{L},{E}]",
                               lambda: F.scaled_dot_product_attention(q, k, v), reps,
                               flops=4.0 * 2 * 8 * L * L * E))
        kc, vc = rnd(2, 8, 77, E), rnd(2, 8, 77, E)
        nbytes = 2 * (2 * 2 * 8 * L * E + 2 * 2 * 8 * 77 * E)
        rows.append(_suite_row(f"sdpa cross fp16 [2,8,{L},{E}] x 77 keys",
                               lambda: F.scaled_dot_product_attention(q, kc, vc), reps,
                               flops=4.0 * 2 * 8 * L * 77 * E, nbytes=nbytes, bound="hbm"))
    # softmax / layer_norm rows (attention scores of the legacy path, transformer tokens).
    for rws, N in ((2 * 8 * 4096, 77), (2 * 8 * 1024, 1024), (2 * 8 * 4096 * 8, 1024)):
        s = rnd(rws, N)
        rows.append(_suite_row(f"softmax fp16 [{rws},{N}]", lambda: F.softmax(s, dim=-1), reps,
                               nbytes=2 * rws * N * 2, bound="hbm"))
        del s
    for rws, C in ((8192, 320), (2048, 640), (512, 1280), (8192 * 64, 320)):
        t = rnd(rws, C)
        lw, lb = rnd(C), rnd(C)
        rows.append(_suite_row(f"layer_norm fp16 [{rws},{C}]", lambda: F.layer_norm(t, (C,), lw, lb, 1e-5), reps,
                               nbytes=2 * rws * C * 2, bound="hbm"))
        del t
    # the SpatialTransformer block at 32x32.
    mt.manual_seed(0)
    st = sd_unet.SpatialTransformer(sd_unet._Init("cuda"), 640)
    xt, ctx = rnd(2, 640, 32, 32), rnd(2, 77, 768)
    rows.append(_suite_row("SpatialTransformer fp16 [2,640,32,32] ctx [2,77,768]", lambda: st(xt, ctx), 5,
                           flops=39.63e9))
    mfma = [r for r in rows if r["bound"] == "mfma"]
    return {
        "metric": "per-op TFLOP/s (vs fp16/fp32 MFMA peak) and GB/s (vs HBM peak) at the SD-1.5 shapes",
        "value": round(sum(r["frac"] for r in mfma) / len(mfma), 4), "unit": "mean MFMA fraction",
        "n_gpus": 1, "steps": reps, "warmup": 1, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic (mtorch generator, seed 0)",
        "config": {"workload": "configs[0]-[3] op rows, each graph-replayed x20"}, "rows": rows,
    }


VENDOR_CONV = ((320, 64), (640, 32), (1280, 16), (1280, 8))
VENDOR_LINEAR = ((8192, 320, 320), (2048, 640, 640), (512, 1280, 1280), (2048, 640, 2560), (8192, 1280, 320))


def _vendor_torch_rows(reps):
    """torch's F.conv2d (MIOpen, NCHW and channels-last) and F.linear (hipBLASLt) in fp16 on the
    vendor comparison shapes.  Runs in a child process that never loads libmthip (torch brings its
    own HIP runtime)."""
    import torch
    import torch.nn.functional as TF

    def timed(fn):
        """(µs per call, how): a CUDA graph of 20 calls replayed `reps` times, or eager calls
        when the library call cannot be captured."""
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(20):
                    fn()
            g.replay()
            torch.cuda.synchronize()
            s.record()
            for _ in range(reps):
                g.replay()
            e.record()
            torch.cuda.synchronize()
            return s.elapsed_time(e) * 1e3 / (reps * 20), "graph"
        except Exception:  # capture refused: time eager back-to-back calls instead
            torch.cuda.synchronize()
            s.record()
            for _ in range(reps):
                fn()
            e.record()
            torch.cuda.synchronize()
            return s.elapsed_time(e) * 1e3 / reps, "eager"

    torch.manual_seed(0)
    out = {"torch": torch.__version__, "conv": [], "linear": []}
    for C, hw in VENDOR_CONV:
        tx = torch.randn(2, C, hw, hw, device="cuda", dtype=torch.float16)
        tw = torch.randn(C, C, 3, 3, device="cuda", dtype=torch.float16) * 0.02
        tb = torch.randn(C, device="cuda", dtype=torch.float16) * 0.02
        txc, twc = tx.to(memory_format=torch.channels_last), tw.to(memory_format=torch.channels_last)
        out["conv"].append((timed(lambda: TF.conv2d(tx, tw, tb, padding=1)),
                            timed(lambda: TF.conv2d(txc, twc, tb, padding=1))))
    for M, N, K in VENDOR_LINEAR:
        tx = torch.randn(M, K, device="cuda", dtype=torch.float16) * 0.5
        tw = torch.randn(N, K, device="cuda", dtype=torch.float16) * 0.05
        tb = torch.randn(N, device="cuda", dtype=torch.float16) * 0.05
        out["linear"].append(timed(lambda: TF.linear(tx, tw, tb)))
    return out


def run_vendor(args):
    """The contractions of the hot path against the vendor libraries PyTorch-ROCm calls on the same
    box: F.conv2d (MIOpen, NCHW and channels-last) and F.linear (hipBLASLt) in fp16.  Each side is
    timed as a graph of 20 calls replayed `steps` times between two events on its own library's
    stream (the torch side falls back to eager calls where capture is refused, and says so); the
    torch side runs in a child process.  A comparison, not the headline."""
    import subprocess

    import mtorch_amd as mt

    F = mt.nn.functional
    reps = args.steps
    child = subprocess.run([sys.executable, os.path.abspath(__file__), "--workload", "vendor_torch", "--steps", str(reps)],
                           capture_output=True, text=True, timeout=600)
    if child.returncode != 0:
        raise SystemExit("bench.py vendor: the torch child failed:\n" + child.stderr[-2000:])
    theirs = json.loads(child.stdout.strip().splitlines()[-1])

    def ours(fn):
        """µs per call: a HIP graph of 20 calls replayed `reps` times."""
        for _ in range(3):
            fn()
        mt.cuda.synchronize()
        g = mt.cuda.CUDAGraph()
        with mt.cuda.graph(g):
            for _ in range(20):
                fn()
        g.replay()
        mt.cuda.synchronize()
        s, e = mt.cuda.Event(), mt.cuda.Event()
        s.record()
        for _ in range(reps):
            g.replay()
        e.record()
        mt.cuda.synchronize()
        return s.elapsed_time(e) * 1e3 / (reps * 20)

    rows = []
    mt.manual_seed(0)
    for (C, hw), ((nchw, how_a), (nhwc, how_b)) in zip(VENDOR_CONV, theirs["conv"]):
        flop = 2.0 * 2 * hw * hw * C * C * 9
        x = (mt.randn(2, C, hw, hw).to("cuda")).half()
        w = (mt.randn(C, C, 3, 3).to("cuda") * 0.02).half()
        b = (mt.randn(C).to("cuda") * 0.02).half()
        us = ours(lambda: F.conv2d(x, w, b, padding=1))
        rows.append({"op": f"conv3x3 fp16 [2,{C},{hw},{hw}] {C}->{C}", "libmthip_us": round(us, 2),
                     "libmthip_tflops": round(flop / us / 1e6, 1), "miopen_nchw_us": round(nchw, 2),
                     "miopen_nchw_tflops": round(flop / nchw / 1e6, 1), "miopen_nhwc_us": round(nhwc, 2),
                     "miopen_nhwc_tflops": round(flop / nhwc / 1e6, 1), "miopen_timing": [how_a, how_b]})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        del x, w, b
    for (M, N, K), (th, how) in zip(VENDOR_LINEAR, theirs["linear"]):
        flop = 2.0 * M * N * K
        x = (mt.randn(M, K).to("cuda") * 0.5).half()
        w = (mt.randn(N, K).to("cuda") * 0.05).half()
        b = (mt.randn(N).to("cuda") * 0.05).half()
        us = ours(lambda: F.linear(x, w, b))
        rows.append({"op": f"linear fp16 [{M},{K}]x[{N},{K}]^T + b", "libmthip_us": round(us, 2),
                     "libmthip_tflops": round(flop / us / 1e6, 1), "hipblaslt_us": round(th, 2),
                     "hipblaslt_tflops": round(flop / th / 1e6, 1), "hipblaslt_timing": how})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        del x, w, b
    return {"metric": "fp16 conv3x3 / linear TFLOP/s against MIOpen / hipBLASLt (torch " + theirs["torch"] + ")",
            "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 3, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
            "config": {"workload": "SD-1.5 conv and linear shapes, graph-replayed x20 per side"}, "rows": rows}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="resnet", choices=["resnet", "linear_gelu", "unet", "copy_calibration", "suite", "vendor",
                                                                 "vendor_torch"])
    ap.add_argument("--no-cpu", dest="cpu", action="store_false")
    ap.add_argument("--no-extras", dest="extras", action="store_false",
                    help="resnet workload: skip the UNet step and per-config contraction keys")
    args = ap.parse_args()
    if args.workload == "vendor_torch":  # child of --workload vendor: torch only, libmthip never loaded
        print(json.dumps(_vendor_torch_rows(args.steps)), flush=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this backend measures one MI355X; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import mtorch_amd as mt

    if not mt.cuda.is_available():
        raise SystemExit("bench.py: no GPU visible to libmthip")
    with mt.no_grad():
        run = {"resnet": run_resnet, "linear_gelu": run_linear_gelu, "unet": run_unet,
               "copy_calibration": run_copy_calibration, "suite": run_suite, "vendor": run_vendor}
        out = run[args.workload](args)
    out["device"] = mt.cuda.get_device_name(0)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
