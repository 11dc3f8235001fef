#!/usr/bin/env python3
"""Benchmark of the dense-contraction hot path on one MI355X.

Headline (the `value`): float16 `mm` 8192x8192x8192 (config C5 "square") in
TFLOP/s through the C ABI (tvk_gemm), inputs resident in HBM, N(0,1) from a
fixed seed. One step = one tvk_gemm call over the whole problem. K timed steps
are bracketed by torch.cuda.synchronize(); the dominant kernel's average
duration comes from HIP events recorded on the stream the kernel runs on.

Secondary figures (same JSON line, under "extra"): the C2 MLP GEMM chain
forward+backward step in ms, the C5 skinny 16x4096x14336 GEMM in GB/s with
B rotated over buffers larger than the 256 MB Infinity Cache, and C1 fp32
1024^3 mm.

cpu_baseline: the oracle's restatement of the reference SIMD tile
(oracle/gemm_oracle.c, kind "port") timed on the host cores on a bounded
sample of the same workload (whole rows of the 8192^3 product).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_F16_TFLOPS = 2516.6   # MI355X dense fp16/bf16 MFMA, AMD spec sheet
PEAK_F32_TFLOPS = 157.3    # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

# HBM bytes per launch of the headline kernel, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# (KiB per dispatch) scaled by what the same counters read for a 1 GiB copy (x2.0 and x1.0):
# profiles/gemm_fp16_8192_counters.md. Counters need their own profiler runs, so the figure is
# recorded here per kernel plan rather than measured inside the timed region.
MEASURED_TRAFFIC = {
    "gemm16_dma_256x256": {"bytes": 1.764e9, "fetch_kib": 795667, "write_kib": 131072},
}
# HBM bytes per step of the other bench rows (FETCH_SIZE x 2 + WRITE_SIZE, summed over
# each step's kernels; profiles/bench_rows_counters.md)
MEASURED_ROW_TRAFFIC = {
    "source": "profiles/bench_rows_counters.md",
    "c2_mlp_gemm_step": {"bytes": 4.717e8, "algorithmic": 2.5e8},
    "c2_256x4096x4096_product_with_reduce": {"bytes": 8.624e7, "algorithmic": 3.77e7},
    "c2_dw_4096x4096x256": {"bytes": 4.683e7, "algorithmic": 3.77e7},
    "c3_dx_8192x512x3072": {"bytes": 1.731e8, "algorithmic": 6.13e7},
    "c4_conv_step": {"bytes": 5.64e8, "algorithmic": 2.76e8},
    "c5_ragged_with_repack": {"bytes": 2.834e7, "algorithmic": 1.22e7},
    "c5_baddbmm": {"bytes": 1.033e8, "algorithmic": 8.39e7},
    "c3_attention_fwd": {"bytes": 3.397e7},
    "c3_attention_bwd": {"bytes": 7.689e7},
}

# the headline kernel and the MFMA ceiling loop under counters
MEASURED_COUNTERS = {
    "gemm16_dma_256x256": {"mfma_busy_pct": [70.6, 74.0], "shader_clock_ghz": [1.28, 1.70],
                           "source": "profiles/gemm_fp16_8192_counters.md",
                           "ceiling_loop_random": {"mfma_busy_pct": [95.1, 97.2], "shader_clock_ghz": [1.83, 1.90]},
                           "ceiling_loop_zero": {"mfma_busy_pct": [98.6, 98.7], "shader_clock_ghz": [2.30, 2.39]},
                           "ceiling_source": "profiles/mfma_ceiling_calibration.md"},
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-extra", action="store_true", help="headline only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--profile-kernel", choices=["gemm", "skinny", "copy", "ceiling", "ceiling_zero"],
                   help="launch only this kernel --steps times and exit (for rocprofv3 counter passes); "
                        "'copy' is torch's copy of a 1 GiB buffer, the calibration for FETCH_SIZE/WRITE_SIZE; "
                        "'ceiling' the random-operand MFMA loop of tvk_calibrate_mfma (two waves per SIMD), "
                        "'ceiling_zero' the same loop on all-zero operands")
    p.add_argument("--only", default=None,
                   help="comma-separated run_extra sections to run alone (c2, skinny, c4, c3, c3_bmm, attn, ragged, "
                        "baddbmm, memops, c1, dropin), printing their results; for rocprofv3 passes over one workload")
    p.add_argument("--vendor", action="store_true",
                   help="time the C2 GEMM chain, the C3 layer GEMMs, the C4 conv layers and the C5 products "
                        "through torch on this GPU (hipBLASLt, MIOpen) with the same shapes and data, print one "
                        "JSON line and exit")
    return p.parse_args()


def vendor_baseline():
    """The vendor libraries on the same workloads, for calibration: torch's
    fp16 addmm/mm (hipBLASLt) on the C2 MLP chain and its 256x4096x4096
    products and on the C3 layer GEMMs, aten.convolution /
    convolution_backward (MIOpen) on the C4
    layers, and mm / baddbmm on the C5 products, all on torch's stream with
    HIP events (the mean of N launches after a warm-up)."""
    import json

    import torch

    dev = torch.device("cuda:0")
    f16 = torch.float16
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def us(fn, n=50, w=10):
        for _ in range(w):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / n * 1e3, 2)

    g = torch.Generator().manual_seed(1)
    out = {"what": "torch on this GPU: hipBLASLt (fp16 addmm/mm), MIOpen (fp16 convolution)"}
    B, dims = 256, [784, 4096, 4096, 4096, 10]
    xs = [torch.rand((B, dims[0]), generator=g).to(f16).to(dev)]
    ws = [((torch.rand((dims[i + 1], dims[i]), generator=g) * 2 - 1) * dims[i] ** -0.5).to(f16).to(dev) for i in range(4)]
    bs = [((torch.rand((dims[i + 1],), generator=g) * 2 - 1) * dims[i] ** -0.5).to(f16).to(dev) for i in range(4)]
    dys = [torch.randn((B, d), generator=g).to(f16).to(dev) for d in dims[1:]]
    h1 = torch.randn((B, 4096), generator=g).to(f16).to(dev)
    out["c2_fwd_256x4096x4096_us"] = us(lambda: torch.addmm(bs[1], h1, ws[1].t()))
    out["c2_dx_256x4096x4096_us"] = us(lambda: torch.mm(dys[1], ws[1]))
    out["c2_dw_4096x4096x256_us"] = us(lambda: torch.mm(dys[1].t(), h1))

    def chain():
        h, acts = xs[0], [xs[0]]
        for i in range(4):
            h = torch.addmm(bs[i], h, ws[i].t())
            acts.append(h)
        for i in reversed(range(4)):
            torch.mm(dys[i].t(), acts[i])
            if i > 0:
                torch.mm(dys[i], ws[i])

    out["c2_mlp_gemm_fwd_bwd_us"] = us(chain, 20, 5)
    progress("vendor: C2 done")
    # C3: the transformer layer's six projections, forward and both gradients
    T, calls3 = 8192, []
    for fin, fout in [(512, 512), (512, 256), (512, 256), (512, 512), (512, 3072), (1536, 512)]:
        x = torch.randn((T, fin), generator=g).to(f16).to(dev)
        w = (torch.randn((fout, fin), generator=g) * 0.02).to(f16).to(dev)
        dy = torch.randn((T, fout), generator=g).to(f16).to(dev)
        calls3 += [lambda x=x, w=w: torch.mm(x, w.t()), lambda dy=dy, w=w: torch.mm(dy, w),
                   lambda dy=dy, x=x: torch.mm(dy.t(), x)]

    def c3():
        for c in calls3:
            c()

    out["c3_llm_layer_gemm_fwd_bwd_us"] = us(c3, 20, 5)
    del calls3
    progress("vendor: C3 done")
    layers = [(3, 64, 3, 1, 1, 32), (64, 64, 3, 1, 1, 32), (64, 128, 3, 2, 1, 32), (128, 256, 3, 2, 1, 16),
              (64, 128, 1, 2, 0, 32), (128, 256, 1, 2, 0, 16)]
    calls, per = [], []
    for cin, cout, k, st, pd, hw in layers:
        x = torch.randn((128, cin, hw, hw), generator=g).to(f16).to(dev)
        w = (torch.randn((cout, cin, k, k), generator=g) * (2.0 / (cin * k * k)) ** 0.5).to(f16).to(dev)
        ho = (hw + 2 * pd - k) // st + 1
        dy = torch.randn((128, cout, ho, ho), generator=g).to(f16).to(dev)
        fwd = lambda x=x, w=w, st=st, pd=pd: torch.ops.aten.convolution(x, w, None, [st, st], [pd, pd], [1, 1], False, [0, 0], 1)
        bwd = lambda x=x, w=w, dy=dy, st=st, pd=pd: torch.ops.aten.convolution_backward(
            dy, x, w, None, [st, st], [pd, pd], [1, 1], False, [0, 0], 1, [True, True, False])
        per.append({"layer": f"{cin}->{cout} {k}x{k} s{st}", "fwd_us": us(fwd, 20, 3), "dgrad_wgrad_us": us(bwd, 20, 3)})
        calls += [fwd, bwd]

    def c4():
        for c in calls:
            c()

    out["c4_layers"] = per
    out["c4_resnet_conv_fwd_bwd_us"] = us(c4, 10, 2)
    progress("vendor: C4 done")
    del calls, per
    # C5: the headline square product, the skinny one (B rotated over three
    # buffers past the 256 MB Infinity Cache), the ragged one and baddbmm
    n = 8192
    a = torch.randn((n, n), generator=g).to(f16).to(dev)
    b = torch.randn((n, n), generator=g).to(f16).to(dev)
    c = torch.empty((n, n), dtype=f16, device=dev)
    t = us(lambda: torch.mm(a, b, out=c), 20, 5)
    out["c5_square_8192_us"] = t
    out["c5_square_8192_tflops"] = round(2 * n ** 3 / (t * 1e-6) / 1e12, 1)
    del a, b, c
    M, K, N = 16, 4096, 14336
    a = torch.randn((M, K), generator=g).to(f16).to(dev)
    bufs = [torch.randn((K, N), generator=g).to(f16).to(dev) for _ in range(3)]
    c = torch.empty((M, N), dtype=f16, device=dev)
    idx = [0]

    def skinny():
        torch.mm(a, bufs[idx[0] % 3], out=c)
        idx[0] += 1

    out["c5_skinny_us"] = us(skinny, 150, 30)
    del bufs
    a = torch.randn((1000, 777), generator=g).to(f16).to(dev)
    b = torch.randn((777, 3000), generator=g).to(f16).to(dev)
    out["c5_ragged_us"] = us(lambda: torch.mm(a, b))
    x1 = torch.randn((64, 512, 128), generator=g).to(f16).to(dev)
    x2 = torch.randn((64, 128, 512), generator=g).to(f16).to(dev)
    inp = torch.randn((64, 512, 512), generator=g).to(f16).to(dev)
    out["c5_baddbmm_us"] = us(lambda: torch.baddbmm(inp, x1, x2, beta=1.0, alpha=0.5))
    progress("vendor: C5 done")
    print(json.dumps(out), flush=True)


def profile_kernel(which, steps):
    """Launches one kernel `steps` times with nothing else on the GPU but the
    inputs' initialisation, so that per-dispatch counters read cleanly."""
    import ctypes as C

    import torch
    from torchvulkan_amd import _abi

    lib = _abi.load()
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream(dev).cuda_stream
    if which in ("ceiling", "ceiling_zero"):
        for _ in range(steps):
            tf, _ = _abi.calibrate_mfma(0, 2, 40000, zeros=which == "ceiling_zero")
        print(f"{which}: {steps} launches, last {tf:.1f} TFLOP/s", flush=True)
        return
    if which == "copy":
        x = torch.ones((1 << 29,), dtype=torch.float16, device=dev)   # 1 GiB
        y = torch.empty_like(x)
        for _ in range(steps):
            y.copy_(x)
        torch.cuda.synchronize()
        print(f"copy: {steps} x {x.numel() * 2} bytes read + written", flush=True)
        return
    if which == "gemm":
        n = 8192
        a = torch.randn((n, n), device=dev).to(torch.float16)
        b = torch.randn((n, n), device=dev).to(torch.float16)
        c = torch.empty((n, n), dtype=torch.float16, device=dev)
        descs = [_abi.make_gemm_desc(a, b, c, stream=s)]
    else:
        M, K, N = 16, 4096, 14336
        a = torch.randn((M, K), device=dev).to(torch.float16)
        bufs = [torch.randn((K, N), device=dev).to(torch.float16) for _ in range(3)]
        c = torch.empty((M, N), dtype=torch.float16, device=dev)
        descs = [_abi.make_gemm_desc(a, bb, c, stream=s) for bb in bufs]
    for i in range(steps):
        _abi.check(lib.tvk_gemm(C.byref(descs[i % len(descs)])))
    torch.cuda.synchronize()
    print(f"{which}: {steps} launches of {_abi.gemm_plan(a, (bufs[0] if which == 'skinny' else b), c)}", flush=True)


# --only: the run_extra sections that launch anything (for rocprofv3 passes over
# one workload); the others build their inputs but time nothing
_ONLY = None
_SECTION = None


def section(name: str) -> bool:
    """Enters a run_extra section; True when it runs its kernels."""
    global _SECTION
    _SECTION = name
    return _ONLY is None or name in _ONLY


def progress(msg: str) -> None:
    """A progress line on stderr (stdout carries only the result line)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


def timed(fn, steps, warmup, stream):
    """Runs fn warmup times, then times `steps` calls with events on `stream`.

    Returns (ms per step from events, ms per step from the host clock)."""
    import torch

    if _ONLY is not None and _SECTION not in _ONLY:
        return 1.0, 1.0
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return start.elapsed_time(end) / steps, (t1 - t0) * 1e3 / steps


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} (WORLD_SIZE={world}) is not supported. "
              "The path shards by splitting N or M across GPUs with no exchange; see DESIGN.md.", file=sys.stderr)
        sys.exit(2)

    if args.profile_kernel:
        profile_kernel(args.profile_kernel, args.steps)
        return
    if args.vendor:
        vendor_baseline()
        return

    import torch
    from torchvulkan_amd import _abi

    _abi.load()  # fails loudly when the HIP library is not built
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    props = _abi.DeviceProps()
    _abi.check(_abi.load().tvk_device_properties(0, props))

    if args.only:
        global _ONLY
        _ONLY = set(args.only.split(","))
        res = run_extra(torch, _abi, dev, stream, args.steps, args.warmup)
        keep = {k: v for k, v in res.items() if any(k.startswith(x) for x in ("c1", "c2", "c3", "c4", "c5", "dropin"))}
        print(json.dumps({"only": sorted(_ONLY), "extra": keep}, default=str), flush=True)
        return

    # ---- headline: fp16 8192^3 --------------------------------------------
    n = 8192
    g = torch.Generator().manual_seed(0)
    a = torch.randn((n, n), generator=g).to(torch.float16).to(dev)
    b = torch.randn((n, n), generator=g).to(torch.float16).to(dev)
    c = torch.empty((n, n), dtype=torch.float16, device=dev)
    plan = _abi.gemm_plan(a, b, c)
    desc = _abi.make_gemm_desc(a, b, c, stream=stream.cuda_stream)
    lib = _abi.load()
    import ctypes as C
    dref = C.byref(desc)

    def step():
        st = lib.tvk_gemm(dref)
        if st:
            _abi.check(st)

    ms, host_ms = timed(step, args.steps, args.warmup, stream)
    progress(f"headline done: {ms:.4f} ms per step")
    flops = 2.0 * n * n * n
    tflops = flops / (ms * 1e-3) / 1e12
    roofline = {
        "kernel": plan,
        "bound": "mfma",
        "achieved": round(tflops, 2),
        "peak": PEAK_F16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / PEAK_F16_TFLOPS, 4),
        "traffic": MEASURED_TRAFFIC.get(plan, {}).get("bytes"),
        "traffic_source": "profiles/gemm_fp16_8192_counters.md" if plan in MEASURED_TRAFFIC else None,
        "algorithmic_unit": "2*M*N*K flops per launch",
        "algorithmic_bytes": 3 * n * n * 2,
        "avg_kernel_ms": round(ms, 5),
    }
    # the ceiling on this box: the issue-saturated MFMA loop of tvk_calibrate_mfma
    # with random fp16 operands (the power-limited rate a GEMM on random data can
    # reach) and with all-zero operands (the pipe's issue rate at the full clock)
    ceiling = {}
    _abi.calibrate_mfma(0, 2, 40000)   # the clock settles under the load first
    for w in (1, 2, 4):
        tf, _ = _abi.calibrate_mfma(0, w, 40000)
        ceiling[f"waves_per_simd_{w}"] = round(tf, 1)
    top = max(ceiling.values())
    zero_tf = max(_abi.calibrate_mfma(0, 2, 40000, zeros=True)[0] for _ in range(2))
    m32_tf = max(_abi.calibrate_mfma(0, 2, 40000, mfma32=True)[0] for _ in range(2))
    roofline["ceiling"] = {
        "what": "v_mfma_f32_16x16x32_f16 loop, 16 accumulators, no memory traffic (tvk_calibrate_mfma): random fp16 "
                "operands; zero_operands is the same loop on all-zero operands; mfma32_random the same flops on "
                "v_mfma_f32_32x32x16_f16 with random operands",
        "unit": "TFLOP/s", **ceiling, "max": top, "zero_operands": round(zero_tf, 1), "mfma32_random": round(m32_tf, 1),
        "frac_of_ceiling": round(tflops / top, 4),
    }
    roofline["counters"] = MEASURED_COUNTERS.get(plan)
    progress("MFMA ceiling done")

    extra = {}
    if not args.no_extra:
        extra = run_extra(torch, _abi, dev, stream, max(5, args.steps // 5), max(2, args.warmup // 2))
    del a, b, c
    torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline()

    line = {
        "metric": "fp16 GEMM TFLOP/s & % MFMA peak; fwd+bwd step ms (MLP/LLM/ResNet shapes)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "host_ms_per_step": round(host_ms, 5),
        "pct_mfma_peak": round(100.0 * tflops / PEAK_F16_TFLOPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "C5 square: fp16 mm 8192x8192x8192, N(0,1) seed 0, row-major operands, via tvk_gemm",
                   "M": n, "N": n, "K": n, "kernel": plan},
        "device": {"name": props.name.decode(), "arch": props.arch.decode(), "compute_units": props.compute_units,
                   "clock_mhz": props.clock_khz / 1000.0},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


def bound_us(flops: float, nbytes: float) -> float:
    """Roofline time of a launch: the larger of its dense fp16 MFMA time and its HBM time."""
    return max(flops / (PEAK_F16_TFLOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)) * 1e6


def run_extra(torch, _abi, dev, stream, steps, warmup):
    out = {}
    # ---- C2 MLP chain fwd+bwd (GEMMs only, fp16) ----------------------------
    section("c2")
    dims = [784, 4096, 4096, 4096, 10]
    g = torch.Generator().manual_seed(1)
    B = 256
    xs = [torch.rand((B, dims[0]), generator=g).to(torch.float16).to(dev)]
    ws, bs = [], []
    for i in range(4):
        bound = dims[i] ** -0.5
        ws.append(((torch.rand((dims[i + 1], dims[i]), generator=g) * 2 - 1) * bound).to(torch.float16).to(dev))
        bs.append(((torch.rand((dims[i + 1],), generator=g) * 2 - 1) * bound).to(torch.float16).to(dev))
    for i in range(4):
        xs.append(torch.empty((B, dims[i + 1]), dtype=torch.float16, device=dev))
    dys = [torch.randn((B, d), generator=g).to(torch.float16).to(dev) for d in dims[1:]]
    dxs = [torch.empty((B, d), dtype=torch.float16, device=dev) for d in dims[:-1]]
    dws = [torch.empty_like(w) for w in ws]
    s = stream.cuda_stream
    descs = []
    for i in range(4):  # forward: x_{i+1} = x_i W_i^T + b_i
        descs.append(_abi.make_gemm_desc(xs[i], ws[i].t(), xs[i + 1], bias=bs[i], beta=1.0, stream=s))
    for i in reversed(range(4)):  # backward: dW_i = dY_i^T x_i ; dX_i = dY_i W_i (not for the input layer)
        descs.append(_abi.make_gemm_desc(dys[i].t(), xs[i], dws[i], stream=s))
        if i > 0:
            descs.append(_abi.make_gemm_desc(dys[i], ws[i], dxs[i], stream=s))
    lib = _abi.load()
    import ctypes as C
    refs = [C.byref(d) for d in descs]

    def mlp_step():
        for r in refs:
            st = lib.tvk_gemm(r)
            if st:
                _abi.check(st)

    ms, _ = timed(mlp_step, steps, warmup, stream)
    fl = 0
    c2_bound = 0.0
    for d in descs:
        fl += 2 * d.M * d.N * d.K
        c2_bound += bound_us(2 * d.M * d.N * d.K, 2 * (d.M * d.K + d.K * d.N + d.M * d.N + (d.N if d.bias else 0)))
    out["c2_mlp_gemm_fwd_bwd_ms"] = round(ms, 4)
    progress("C2 chain done")
    out["c2_mlp_gemm_tflops"] = round(fl / (ms * 1e-3) / 1e12, 2)
    out["c2_bound_ms"] = round(c2_bound / 1e3, 4)
    out["c2_roofline_frac"] = round(c2_bound / 1e3 / ms, 4)
    # the batch-256 layers alone: 256x4096x4096 (x W^T and dY W) and 4096x4096x256 (dY^T x)
    for name, i in (("c2_fwd_256x4096x4096_us", 1), ("c2_dx_256x4096x4096_us", 7), ("c2_dw_4096x4096x256_us", 6)):
        r = refs[i]

        def one(r=r):
            st = lib.tvk_gemm(r)
            if st:
                _abi.check(st)

        ms1, _ = timed(one, steps * 4, warmup, stream)
        d = descs[i]
        b1 = bound_us(2 * d.M * d.N * d.K, 2 * (d.M * d.K + d.K * d.N + d.M * d.N))
        out[name] = {"us": round(ms1 * 1e3, 2), "bound_us": round(b1, 2), "frac": round(b1 / (ms1 * 1e3), 4),
                     "kernel": gemm_plan_of(_abi, d)}

    # ---- C5 skinny 16x4096x14336 fp16, B rotated past the Infinity Cache ----
    section("skinny")
    M, K, N = 16, 4096, 14336
    a = torch.randn((M, K), generator=g).to(torch.float16).to(dev)
    bufs = [torch.randn((K, N), generator=g).to(torch.float16).to(dev) for _ in range(3)]
    c = torch.empty((M, N), dtype=torch.float16, device=dev)
    sd = [_abi.make_gemm_desc(a, bb, c, stream=s) for bb in bufs]
    srefs = [C.byref(d) for d in sd]
    idx = [0]

    def skinny_step():
        r = srefs[idx[0] % 3]
        idx[0] += 1
        st = lib.tvk_gemm(r)
        if st:
            _abi.check(st)

    ms, _ = timed(skinny_step, steps * 3, warmup, stream)
    byts = 2 * (M * K + K * N + M * N)
    progress("C5 skinny done")
    out["c5_skinny_kernel"] = _abi.gemm_plan(a, bufs[0], c)
    out["c5_skinny_us"] = round(ms * 1e3, 2)
    out["c5_skinny_GBps"] = round(byts / (ms * 1e-3) / 1e9, 1)
    out["c5_skinny_pct_hbm"] = round(100 * byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 2)
    # the practical read ceiling on this box: a plain streaming read of the same
    # B size over three rotating windows (tvk_calibrate_hbm)
    rd_gbps, rd_ms = _abi.calibrate_hbm(0, K * N * 2, 60) if section("skinny") else (1.0, 1.0)
    out["c5_read_ceiling"] = {"what": "plain streaming read, 512 workgroups, three rotating windows of B's size "
                                      "(tvk_calibrate_hbm)", "GBps": round(rd_gbps, 1), "us_for_B": round(rd_ms * 1e3, 2),
                              "skinny_frac_of_ceiling": round(byts / (ms * 1e-3) / 1e9 / rd_gbps, 4)}
    del bufs

    # ---- C4 ResNet convs: fwd + dgrad + wgrad of each layer, fp16, batch 128 -
    section("c4")
    layers = [(3, 64, 3, 1, 1, 32), (64, 64, 3, 1, 1, 32), (64, 128, 3, 2, 1, 32), (128, 256, 3, 2, 1, 16),
              (64, 128, 1, 2, 0, 32), (128, 256, 1, 2, 0, 16)]
    conv_calls = []
    conv_flops = 0
    keep = []
    for cin, cout, k, st, pd, hw in layers:
        x = torch.randn((128, cin, hw, hw), generator=g).to(torch.float16).to(dev)
        w = (torch.randn((cout, cin, k, k), generator=g) * (2.0 / (cin * k * k)) ** 0.5).to(torch.float16).to(dev)
        ho = (hw + 2 * pd - k) // st + 1
        y = torch.empty((128, cout, ho, ho), dtype=torch.float16, device=dev)
        dy = torch.randn((128, cout, ho, ho), generator=g).to(torch.float16).to(dev)
        dx = torch.empty_like(x)
        dw = torch.empty_like(w)
        keep += [x, w, y, dy, dx, dw]
        base = dict(stride=st, padding=pd, stream=s)
        conv_calls.append(("tvk_conv2d_fwd", _abi.make_conv_desc(x.shape, w.shape, torch.float16, x=x, weight=w, y=y, **base)))
        conv_calls.append(("tvk_conv2d_dgrad", _abi.make_conv_desc(x.shape, w.shape, torch.float16, x=dx, weight=w, y=dy, **base)))
        conv_calls.append(("tvk_conv2d_wgrad", _abi.make_conv_desc(x.shape, w.shape, torch.float16, x=x, weight=dw, y=dy, **base)))
        conv_flops += 3 * 2 * 128 * cout * ho * ho * cin * k * k
    conv_refs = [(getattr(lib, fn), C.byref(d)) for fn, d in conv_calls]

    def conv_step():
        for fn, r in conv_refs:
            st_ = fn(r)
            if st_:
                _abi.check(st_)

    ms, _ = timed(conv_step, steps, warmup, stream)
    out["c4_resnet_conv_fwd_bwd_ms"] = round(ms, 4)
    progress("C4 chain done")
    out["c4_resnet_conv_tflops"] = round(conv_flops / (ms * 1e-3) / 1e12, 2)
    # per layer: each direction's time and its roofline (conv flops at the MFMA peak, or the
    # NCHW bytes it must move: two activations and the weights, at the HBM peak)
    per_layer = []
    c4_bound = 0.0
    for li, (cin, cout, k, st, pd, hw) in enumerate(layers):
        ho = (hw + 2 * pd - k) // st + 1
        fl1 = 2 * 128 * cout * ho * ho * cin * k * k
        by1 = 2 * (128 * cin * hw * hw + 128 * cout * ho * ho + cout * cin * k * k)
        row = {"layer": f"{cin}->{cout} {k}x{k} s{st}", "bound_us": round(bound_us(fl1, by1), 2)}
        for j, dirn in enumerate(("fwd", "dgrad", "wgrad")):
            fn, r = conv_refs[3 * li + j]

            def one(fn=fn, r=r):
                st_ = fn(r)
                if st_:
                    _abi.check(st_)

            ms1, _ = timed(one, steps * 2, warmup, stream)
            row[f"{dirn}_us"] = round(ms1 * 1e3, 2)
            row[f"{dirn}_frac"] = round(bound_us(fl1, by1) / (ms1 * 1e3), 4)
            c4_bound += bound_us(fl1, by1)
        per_layer.append(row)
    out["c4_layers"] = per_layer
    progress("C4 layers done")
    out["c4_bound_ms"] = round(c4_bound / 1e3, 4)
    out["c4_roofline_frac"] = round(c4_bound / 1e3 / ms, 4)
    del keep, conv_refs, conv_calls

    # ---- C3 transformer layer GEMMs (fp16, tokens 8192): fwd + bwd ----------
    section("c3")
    T = 8192
    shapes = [(512, 512), (512, 256), (512, 256), (512, 512), (512, 3072), (1536, 512)]  # q, k, v, out, gate_up, down
    llm_descs = []
    keep = []
    llm_flops = 0
    for fin, fout in shapes:
        x = torch.randn((T, fin), generator=g).to(torch.float16).to(dev)
        w = (torch.randn((fout, fin), generator=g) * 0.02).to(torch.float16).to(dev)
        y = torch.empty((T, fout), dtype=torch.float16, device=dev)
        dy = torch.randn((T, fout), generator=g).to(torch.float16).to(dev)
        dx = torch.empty_like(x)
        dw = torch.empty_like(w)
        keep += [x, w, y, dy, dx, dw]
        llm_descs += [_abi.make_gemm_desc(x, w.t(), y, stream=s), _abi.make_gemm_desc(dy, w, dx, stream=s),
                      _abi.make_gemm_desc(dy.t(), x, dw, stream=s)]
        llm_flops += 3 * 2 * T * fin * fout
    llm_bound = 0.0
    for d in llm_descs:
        llm_bound += bound_us(2 * d.M * d.N * d.K, 2 * (d.M * d.K + d.K * d.N + d.M * d.N))
    llm_refs = [C.byref(d) for d in llm_descs]

    def llm_step():
        for r in llm_refs:
            st_ = lib.tvk_gemm(r)
            if st_:
                _abi.check(st_)

    ms, _ = timed(llm_step, steps, warmup, stream)
    out["c3_llm_layer_gemm_fwd_bwd_ms"] = round(ms, 4)
    progress("C3 GEMMs done")
    out["c3_llm_layer_gemm_tflops"] = round(llm_flops / (ms * 1e-3) / 1e12, 2)
    out["c3_llm_layer_gemm_roofline_frac"] = round(llm_bound / 1e3 / ms, 4)
    del keep, llm_refs, llm_descs

    section("c3_bmm")
    # attention products on head-strided views, as the math path meets them: per sequence,
    # q [L, H, D] and k, v [S, H, D] from the projections (GQA's kv heads already repeated to H),
    # S = q k^T and O = P v as batches over the H heads (batch stride D, row stride H*D)
    Bq, H, L, D = 32, 8, 256, 64
    qs = torch.randn((Bq, L, H, D), generator=g).to(torch.float16).to(dev)
    ks = torch.randn((Bq, L, H, D), generator=g).to(torch.float16).to(dev)
    vs = torch.randn((Bq, L, H, D), generator=g).to(torch.float16).to(dev)
    ss = torch.empty((Bq, H, L, L), dtype=torch.float16, device=dev)
    os_ = torch.empty((Bq, L, H, D), dtype=torch.float16, device=dev)
    hd = []
    for bi in range(Bq):
        hd.append(_abi.make_gemm_desc(qs[bi].transpose(0, 1), ks[bi].transpose(0, 1).transpose(1, 2), ss[bi], stream=s))
        hd.append(_abi.make_gemm_desc(ss[bi], vs[bi].transpose(0, 1), os_[bi].transpose(0, 1), stream=s))
    hrefs = [C.byref(d) for d in hd]

    def bmm_step():
        for r in hrefs:
            st_ = lib.tvk_gemm(r)
            if st_:
                _abi.check(st_)

    ms, _ = timed(bmm_step, steps, warmup, stream)
    bmm_fl = 2 * 2 * Bq * H * L * L * D
    bmm_by = 2 * (4 * Bq * L * H * D + 2 * Bq * H * L * L)
    out["c3_head_strided_bmm_per_sequence_us"] = round(ms * 1e3, 2)
    out["c3_head_strided_bmm_per_sequence_kernels"] = [gemm_plan_of(_abi, hd[0]), gemm_plan_of(_abi, hd[1])]
    out["c3_head_strided_bmm_per_sequence_roofline_frac"] = round(bound_us(bmm_fl, bmm_by) / (ms * 1e3), 4)
    del hd, hrefs

    # the same products as torch.matmul runs them on the 4-D views [B, H, L, D] (the math SDPA):
    # batch and head do not merge into one stride, so matmul's reshape to [B*H, ., .] copies q,
    # k^T and v (the scores are already contiguous), then one bmm of batch B*H each
    qc = torch.empty((Bq * H, L, D), dtype=torch.float16, device=dev)
    ktc = torch.empty((Bq * H, D, L), dtype=torch.float16, device=dev)
    vc = torch.empty((Bq * H, L, D), dtype=torch.float16, device=dev)
    sc = torch.empty((Bq * H, L, L), dtype=torch.float16, device=dev)
    oc = torch.empty((Bq * H, L, D), dtype=torch.float16, device=dev)
    cds = [_abi.make_copy_desc(qs.transpose(1, 2), qc.view(Bq, H, L, D), stream=s),
           _abi.make_copy_desc(ks.permute(0, 2, 3, 1), ktc.view(Bq, H, D, L), stream=s),
           _abi.make_copy_desc(vs.transpose(1, 2), vc.view(Bq, H, L, D), stream=s)]
    gds = [_abi.make_gemm_desc(qc, ktc, sc, stream=s), _abi.make_gemm_desc(sc, vc, oc, stream=s)]
    crefs, grefs = [C.byref(d) for d in cds], [C.byref(d) for d in gds]

    def matmul_step():
        for r in crefs:
            st_ = lib.tvk_copy(r)
            if st_:
                _abi.check(st_)
        for r in grefs:
            st_ = lib.tvk_gemm(r)
            if st_:
                _abi.check(st_)

    ms, _ = timed(matmul_step, steps, warmup, stream)
    copy_by = 3 * 2 * 2 * Bq * L * H * D
    out["c3_head_strided_bmm_reshape_copies_us"] = round(ms * 1e3, 2)
    out["c3_head_strided_bmm_reshape_copies_path"] = "3 reshape copies to [B*H, ., .] + 2 bmm of batch B*H (torch's composite matmul)"

    # the same products as the device's matmul runs them: the [B, H, L, D] views as
    # they are, one product each over two batch dimensions (B, and H with its own stride)
    q4, k4t, v4 = qs.permute(0, 2, 1, 3), ks.permute(0, 2, 3, 1), vs.permute(0, 2, 1, 3)
    s4 = torch.empty((Bq, H, L, L), dtype=torch.float16, device=dev)
    o4 = torch.empty((Bq, H, L, D), dtype=torch.float16, device=dev)
    g2 = [_abi.make_gemm_desc(q4, k4t, s4, stream=s), _abi.make_gemm_desc(s4, v4, o4, stream=s)]
    g2refs = [C.byref(d) for d in g2]

    def two_level_step():
        for r in g2refs:
            st_ = lib.tvk_gemm(r)
            if st_:
                _abi.check(st_)

    ms, _ = timed(two_level_step, steps, warmup, stream)
    out["c3_head_strided_bmm_us"] = round(ms * 1e3, 2)
    out["c3_head_strided_bmm_path"] = ("torch.matmul on [B, H, L, D] views on the vulkan device: one product each over two "
                                       "batch dimensions (tvk_gemm_desc.batch_inner), no copies")
    out["c3_head_strided_bmm_kernels"] = [gemm_plan_of(_abi, g2[0]), gemm_plan_of(_abi, g2[1])]
    out["c3_head_strided_bmm_roofline_frac"] = round(bound_us(bmm_fl, bmm_by) / (ms * 1e3), 4)
    progress("C3 head-strided bmm done")
    del qs, ks, vs, ss, os_, qc, ktc, vc, sc, oc, cds, gds, crefs, grefs, s4, o4, g2, g2refs

    # ---- C3 attention: fused forward, batch 32, 8 query / 2 kv heads, seq 256, head_dim 64, causal
    section("attn")
    qa = torch.randn((32, 8, 256, 64), generator=g).to(torch.float16).to(dev)
    ka = torch.randn((32, 2, 256, 64), generator=g).to(torch.float16).to(dev)
    va = torch.randn((32, 2, 256, 64), generator=g).to(torch.float16).to(dev)
    oa = torch.empty_like(qa)
    la = torch.empty((32, 8, 256), dtype=torch.float32, device=dev)
    ad = _abi.make_attention_desc(qa, ka, va, oa, la, causal=True, stream=s)
    ar = C.byref(ad)

    def attn_step():
        st_ = lib.tvk_attention_fwd(ar)
        if st_:
            _abi.check(st_)

    ms, _ = timed(attn_step, steps * 4, warmup, stream)
    # causal: the unmasked half of the L x S scores (i >= j), two products of 2*D flops each
    att_flops = 32 * 8 * (256 * 257 // 2) * 64 * 2 * 2
    att_bytes = 2 * (2 * 32 * 8 * 256 * 64 + 2 * 32 * 2 * 256 * 64) + 4 * 32 * 8 * 256
    out["c3_attention_fwd_us"] = round(ms * 1e3, 2)
    out["c3_attention_fwd_tflops"] = round(att_flops / (ms * 1e-3) / 1e12, 2)
    out["c3_attention_fwd_roofline_frac"] = round(bound_us(att_flops, att_bytes) / (ms * 1e3), 4)
    # backward: five products over the unmasked half (S, dP, dV, dQ, dK; S is recomputed in both passes)
    da = torch.randn(oa.shape, generator=g).to(torch.float16).to(dev)
    gq, gk, gv = torch.empty_like(qa), torch.empty_like(ka), torch.empty_like(va)
    bd = _abi.AttentionBwdDesc()
    bd.fwd = ad
    bd.dout, bd.dout_stride = da.data_ptr(), _abi.I64x4(*da.stride())
    bd.dq, bd.dq_stride = gq.data_ptr(), _abi.I64x4(*gq.stride())
    bd.dk, bd.dk_stride = gk.data_ptr(), _abi.I64x4(*gk.stride())
    bd.dv, bd.dv_stride = gv.data_ptr(), _abi.I64x4(*gv.stride())
    br_ = C.byref(bd)

    def attn_bwd_step():
        st_ = lib.tvk_attention_bwd(br_)
        if st_:
            _abi.check(st_)

    ms, _ = timed(attn_bwd_step, steps * 4, warmup, stream)
    out["c3_attention_bwd_us"] = round(ms * 1e3, 2)
    progress("C3 attention done")
    out["c3_attention_bwd_tflops"] = round(att_flops * 5 / 2 / (ms * 1e-3) / 1e12, 2)
    out["c3_attention_bwd_roofline_frac"] = round(bound_us(att_flops * 5 / 2, 2 * att_bytes) / (ms * 1e3), 4)
    del qa, ka, va, oa, la, da, gq, gk, gv

    # ---- C5 ragged [1000,777]x[777,3000] and baddbmm in[64,512,512] + 0.5*bmm ----
    section("ragged")
    a = torch.randn((1000, 777), generator=g).to(torch.float16).to(dev)
    b = torch.randn((777, 3000), generator=g).to(torch.float16).to(dev)
    c = torch.empty((1000, 3000), dtype=torch.float16, device=dev)
    dr = _abi.make_gemm_desc(a, b, c, stream=s)
    rr = C.byref(dr)

    def ragged_step():
        st_ = lib.tvk_gemm(rr)
        if st_:
            _abi.check(st_)

    ms, _ = timed(ragged_step, steps * 4, warmup, stream)
    out["c5_ragged_kernel"] = _abi.gemm_plan(a, b, c)
    out["c5_ragged_us"] = round(ms * 1e3, 2)
    out["c5_ragged_tflops"] = round(2 * 1000 * 777 * 3000 / (ms * 1e-3) / 1e12, 2)
    out["c5_ragged_roofline_frac"] = round(bound_us(2 * 1000 * 777 * 3000, 2 * (1000 * 777 + 777 * 3000 + 1000 * 3000))
                                           / (ms * 1e3), 4)
    section("baddbmm")
    x1 = torch.randn((64, 512, 128), generator=g).to(torch.float16).to(dev)
    x2 = torch.randn((64, 128, 512), generator=g).to(torch.float16).to(dev)
    inp = torch.randn((64, 512, 512), generator=g).to(torch.float16).to(dev)
    cb = torch.empty((64, 512, 512), dtype=torch.float16, device=dev)
    db_ = _abi.make_gemm_desc(x1, x2, cb, bias=inp, alpha=0.5, beta=1.0, stream=s)
    rb_ = C.byref(db_)

    def baddbmm_step():
        st_ = lib.tvk_gemm(rb_)
        if st_:
            _abi.check(st_)

    ms, _ = timed(baddbmm_step, steps * 4, warmup, stream)
    byts = 2 * (64 * 512 * 128 * 2 + 2 * 64 * 512 * 512)   # A, B, C-in, C-out
    out["c5_baddbmm_kernel"] = _abi.gemm_plan(x1, x2, cb, bias=inp, alpha=0.5, beta=1.0)
    out["c5_baddbmm_us"] = round(ms * 1e3, 2)
    out["c5_baddbmm_GBps"] = round(byts / (ms * 1e-3) / 1e9, 1)
    out["c5_baddbmm_pct_hbm"] = round(100 * byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 2)
    del a, b, c, x1, x2, inp, cb

    # ---- copies, casts, sums and adds on both sides of the contractions ----
    if section("memops"):
        out.update(run_memory_ops(torch, _abi, dev, stream, steps, warmup, g))

    # ---- C1 fp32 1024^3 ----------------------------------------------------
    section("c1")
    a = torch.randn((1024, 1024), generator=g).to(dev)
    b = torch.randn((1024, 1024), generator=g).to(dev)
    c = torch.empty((1024, 1024), device=dev)
    d1 = _abi.make_gemm_desc(a, b, c, stream=s)
    r1 = C.byref(d1)

    def c1_step():
        st = lib.tvk_gemm(r1)
        if st:
            _abi.check(st)

    ms, _ = timed(c1_step, steps, warmup, stream)
    out["c1_fp32_mm_1024_us"] = round(ms * 1e3, 2)
    out["c1_fp32_tflops"] = round(2 * 1024 ** 3 / (ms * 1e-3) / 1e12, 2)
    out["c1_fp32_roofline_frac"] = round(max(2 * 1024 ** 3 / (PEAK_F32_TFLOPS * 1e12), 12 * 1024 ** 2 / (PEAK_HBM_GBS * 1e9))
                                         * 1e6 / (ms * 1e3), 4)
    out["c1_kernel"] = _abi.gemm_plan(a, b, c)

    out["measured_traffic"] = MEASURED_ROW_TRAFFIC

    # ---- the drop-in path: whole fwd+bwd steps through autograd on "vulkan" ----
    if section("dropin"):
        out["dropin_steps"] = run_dropin(torch, out)
        progress("drop-in steps done")
    return out


def run_dropin(torch, chains):
    """Whole training steps through the vulkan device, timed as the reference's
    benchmark times them (benchmark/benchmark.py:208-223): zero_grad, then
    synchronize, loss.backward() over the forward, synchronize, and the median
    over 10 steps after 3 warm-ups. Everything between the two synchronizes
    counts: dispatch, autograd, the allocator, casts and the bias and loss sums,
    besides the products the C-ABI chains time alone. The models hold only ops
    on the path (no activations: ops outside it run on the CPU fallback), and
    strict mode is on while they run, so any fallback would fail the run."""
    import statistics

    import torchvulkan_amd as tv

    V = "vulkan"
    g = torch.Generator().manual_seed(3)
    res = {}

    def median_step(params, loss_fn, iters=10, warm=3):
        times = []
        for i in range(warm + iters):
            for q in params:
                q.grad = None
            tv.synchronize()
            t0 = time.perf_counter()
            loss_fn().backward()
            tv.synchronize()
            t1 = time.perf_counter()
            if i >= warm:
                times.append((t1 - t0) * 1e3)
        return statistics.median(times)

    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    try:
        # C2: the MLP 784-4096-4096-4096-10, fp16, batch 256, inputs U(0,1), nn.Linear's initialisation
        dims = [784, 4096, 4096, 4096, 10]
        torch.manual_seed(3)
        layers = [torch.nn.Linear(dims[i], dims[i + 1]).to(torch.float16).to(V) for i in range(4)]
        params = [q for lay in layers for q in lay.parameters()]
        x = torch.rand((256, dims[0]), generator=g).to(torch.float16).to(V)

        def mlp_loss():
            y = x
            for lay in layers:
                y = lay(y)
            return y.sum()

        ms = median_step(params, mlp_loss)
        res["c2_mlp_fwd_bwd_ms"] = round(ms, 4)
        res["c2_vs_gemm_chain"] = round(ms / chains["c2_mlp_gemm_fwd_bwd_ms"], 2) if chains.get("c2_mlp_gemm_fwd_bwd_ms") else None
        del layers, params, x
        # C4: the ResNet layers as one block chain, fp16, batch 128, 32x32, Kaiming-normal weights: stem 3->64,
        # 3x3 64->64, then two stride-2 stages whose 1x1 downsample convs are added to the 3x3 ones
        def kconv(cin, cout, k):
            w = torch.randn((cout, cin, k, k), generator=g) * (2.0 / (cin * k * k)) ** 0.5
            return w.to(torch.float16).to(V).requires_grad_()

        ws = {"stem": kconv(3, 64, 3), "c64": kconv(64, 64, 3), "c128": kconv(64, 128, 3), "d128": kconv(64, 128, 1),
              "c256": kconv(128, 256, 3), "d256": kconv(128, 256, 1)}
        xi = torch.randn((128, 3, 32, 32), generator=g).to(torch.float16).to(V)
        F = torch.nn.functional

        def block_loss():
            h1 = F.conv2d(xi, ws["stem"], padding=1)
            h2 = F.conv2d(h1, ws["c64"], padding=1)
            h3 = F.conv2d(h2, ws["c128"], stride=2, padding=1) + F.conv2d(h2, ws["d128"], stride=2)
            h4 = F.conv2d(h3, ws["c256"], stride=2, padding=1) + F.conv2d(h3, ws["d256"], stride=2)
            return h4.sum()

        ms = median_step(list(ws.values()), block_loss)
        res["c4_block_fwd_bwd_ms"] = round(ms, 4)
        res["c4_vs_conv_chain"] = (round(ms / chains["c4_resnet_conv_fwd_bwd_ms"], 2)
                                   if chains.get("c4_resnet_conv_fwd_bwd_ms") else None)
        del ws, xi
        # C3: one transformer layer, 8192 tokens (32 sequences x 256), d 512, 8 query and 2 key/value heads of 64,
        # fp16, N(0, 0.02) weights: q, k, v projections, causal GQA attention (the fused SDPA), out projection and
        # residual, gate and up projections multiplied (SwiGLU without its SiLU: no activation is on the path),
        # down projection and residual; loss = sum in float32. No norms (off the path)
        Bs, Ls, dm, Hq, Hkv, Dh, Ff = 32, 256, 512, 8, 2, 64, 1536

        def lin(fin, fout):
            return (torch.randn((fout, fin), generator=g) * 0.02).to(torch.float16).to(V).requires_grad_()

        lw = {"q": lin(dm, Hq * Dh), "k": lin(dm, Hkv * Dh), "v": lin(dm, Hkv * Dh), "o": lin(Hq * Dh, dm),
              "gate": lin(dm, Ff), "up": lin(dm, Ff), "down": lin(Ff, dm)}
        xt = torch.randn((Bs * Ls, dm), generator=g).to(torch.float16).to(V)

        def layer_loss():
            q = F.linear(xt, lw["q"]).view(Bs, Ls, Hq, Dh).transpose(1, 2)
            k = F.linear(xt, lw["k"]).view(Bs, Ls, Hkv, Dh).transpose(1, 2)
            v = F.linear(xt, lw["v"]).view(Bs, Ls, Hkv, Dh).transpose(1, 2)
            a = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
            h = xt + F.linear(a.transpose(1, 2).reshape(Bs * Ls, Hq * Dh), lw["o"])
            y = h + F.linear(F.linear(h, lw["gate"]) * F.linear(h, lw["up"]), lw["down"])
            return y.float().sum()

        ms = median_step(list(lw.values()), layer_loss)
        res["c3_layer_fwd_bwd_ms"] = round(ms, 4)
        c3_chain = chains.get("c3_llm_layer_gemm_fwd_bwd_ms")
        res["c3_layer_note"] = ("q/k/v/out/gate/up/down products (k, v at 128 columns each: 2 kv heads) plus the "
                                "fused causal GQA attention forward and backward; the C-ABI GEMM chain beside it "
                                f"(c3_llm_layer_gemm_fwd_bwd_ms, k and v at 256 columns) took {c3_chain} ms")
        res["fallbacks"] = 0
        res["note"] = ("median of 10 after 3 (zero_grad, sync, loss.backward(), sync; the reference's time_pass); "
                       "strict mode on, so no op left the device; the C4 block's input needs no gradient, so the "
                       "stem's grad input is not computed")
    finally:
        if old is None:
            del os.environ["TORCHVULKAN_STRICT"]
        else:
            os.environ["TORCHVULKAN_STRICT"] = old
    return res


def run_memory_ops(torch, _abi, dev, stream, steps, warmup, g):
    """HBM-bound kernels next to the GEMMs: GB/s of algorithmic bytes (each
    operand read once, the result written once) and the fraction of 8 TB/s.
    Sizes are far above the 256 MB Infinity Cache where they can be."""
    import ctypes as C

    lib = _abi.load()
    s = stream.cuda_stream
    res = {}

    def measure(name, call, nbytes):
        ms, _ = timed(call, steps * 2, warmup, stream)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "GBps": round(gbs, 1), "pct_hbm": round(100 * gbs / PEAK_HBM_GBS, 2)}
        progress(f"{name} done")

    def copy_call(src, dst):
        d = _abi.make_copy_desc(src, dst, stream=s)
        r = C.byref(d)
        return (lambda: _abi.check(lib.tvk_copy(r))), d

    n = 16384
    w = torch.randn((n, n), generator=g).to(torch.float16).to(dev)               # 512 MiB
    wt = torch.empty((n, n), dtype=torch.float16, device=dev)
    f, keep = copy_call(w.t(), wt)
    measure("copy_transpose_f16_16384sq", f, 2 * w.numel() * 2)
    x32 = torch.randn((1 << 27,), generator=g).to(dev)                            # 512 MiB
    x16 = torch.empty((1 << 27,), dtype=torch.float16, device=dev)
    f, keep2 = copy_call(x32, x16)
    measure("cast_f32_to_f16_128M", f, x32.numel() * 6)
    a = torch.randn((256, 64, 56, 56), generator=g).to(torch.float16).to(dev)    # 98 MiB each way
    cl = torch.empty_like(a, memory_format=torch.channels_last)
    f, keep3 = copy_call(a, cl)
    measure("nchw_to_nhwc_f16_256x64x56x56", f, 2 * a.numel() * 2)
    del w, wt, x32, keep, keep2, keep3

    dy = torch.randn((65536, 3072), generator=g).to(torch.float16).to(dev)       # 384 MiB
    bgrad = torch.empty((3072,), dtype=torch.float16, device=dev)
    rd = _abi.ReduceDesc()
    rd.src_dtype, rd.dst_dtype, rd.ndim, rd.reduce_mask = _abi.TVK_F16, _abi.TVK_F16, 2, 1
    rd.sizes = _abi.I64xD(*dy.shape)
    rd.src, rd.src_strides = dy.data_ptr(), _abi.I64xD(*dy.stride())
    rd.dst, rd.dst_strides = bgrad.data_ptr(), _abi.I64xD(0, 1)
    rd.stream = s
    rr = C.byref(rd)
    measure("sum_dim0_f16_65536x3072", lambda: _abi.check(lib.tvk_reduce_sum(rr)), dy.numel() * 2)
    p_ = torch.randn((1 << 27,), generator=g).to(torch.float16).to(dev)
    bd = _abi.BinaryDesc()
    bd.op, bd.dtype, bd.ndim, bd.reserved = _abi.TVK_BIN_ADD, _abi.TVK_F16, 1, 0
    bd.sizes = _abi.I64xD(p_.numel())
    bd.a, bd.a_strides = p_.data_ptr(), _abi.I64xD(1)
    bd.b, bd.b_strides = x16.data_ptr(), _abi.I64xD(1)
    bd.out, bd.out_strides = p_.data_ptr(), _abi.I64xD(1)
    bd.alpha, bd.stream = -0.01, s
    br = C.byref(bd)
    measure("add_inplace_alpha_f16_128M", lambda: _abi.check(lib.tvk_binary(br)), p_.numel() * 6)
    del dy, p_, x16
    torch.cuda.empty_cache()
    return {"memory_ops": res}


def gemm_plan_of(_abi, desc) -> str:
    import ctypes as C

    buf = C.create_string_buffer(128)
    _abi.check(_abi.load().tvk_gemm_plan(C.byref(desc), buf, 128))
    return buf.value.decode()


def host_info() -> dict:
    """The host CPU as lscpu reports it, and the cores this process may use."""
    import subprocess

    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model, "cpu_count": os.cpu_count(), "usable_cores": usable}


def lavapipe_status() -> str:
    """The reference's own shaders run on Mesa lavapipe only when its ICD and slangc exist on the host."""
    import glob
    import shutil

    icds = [f for d in ("/usr/share/vulkan/icd.d", "/etc/vulkan/icd.d", "/usr/local/share/vulkan/icd.d")
            for f in glob.glob(os.path.join(d, "lvp_icd*.json"))]
    if icds and shutil.which("slangc"):
        return "lavapipe and slangc present; not run (the reference builds against torch 2.15 with CMake and Slang codegen)"
    return "lavapipe baseline unavailable (no Mesa lavapipe / Slang on host)"


def median_ms(fn, reps: int, warmup: int) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def torch_cpu_baselines(cores: int) -> dict:
    """torch on the host cores, as the reference's benchmark times its CPU
    device (median of 10 after 3 warm-ups, benchmark/benchmark.py:208-223):
    rows of the headline product in float32, float16 and bfloat16 (float16 and
    bfloat16 are the CPU's slow low-precision paths), and the C2 MLP GEMM chain
    and the C4 convolution layers forward + backward in float32."""
    import torch
    import torch.nn.functional as F

    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    n = 8192
    out = {}
    a = torch.randn((1024, n), generator=g)
    b = torch.randn((n, n), generator=g)
    samples = []
    for name, dt in (("f32", torch.float32), ("f16", torch.float16), ("bf16", torch.bfloat16)):
        bb = b.to(dt)
        # rows sized so one call takes about 0.25 s (the CPU's low-precision paths can be slow)
        probe = a[:16].to(dt)
        t0 = time.perf_counter()
        torch.mm(probe, bb)
        t16 = time.perf_counter() - t0
        rows = int(min(1024, max(16, 16 * 0.25 / max(t16, 1e-6)))) // 16 * 16
        aa = a[:rows].to(dt)
        ms = median_ms(lambda: torch.mm(aa, bb), 10, 3)
        out[f"mm_{name}_tflops"] = round(2.0 * rows * n * n / (ms * 1e-3) / 1e12, 4)
        samples.append(f"{name} {rows} rows")
        progress(f"cpu baseline: torch {name} mm done")
    out["mm_sample"] = "rows of the 8192^3 mm (" + ", ".join(samples) + "), median of 10 after 3 warm-ups"
    # C2: the MLP's forward and backward GEMMs (784-4096-4096-4096-10, batch 256)
    dims = [784, 4096, 4096, 4096, 10]
    xs = [torch.rand((256, dims[0]), generator=g)]
    ws = [torch.randn((dims[i + 1], dims[i]), generator=g) * dims[i] ** -0.5 for i in range(4)]
    bs = [torch.randn((dims[i + 1],), generator=g) * 0.01 for i in range(4)]
    dys = [torch.randn((256, d), generator=g) for d in dims[1:]]

    def c2():
        x = xs[0]
        acts = [x]
        for i in range(4):
            x = torch.addmm(bs[i], x, ws[i].t())
            acts.append(x)
        for i in reversed(range(4)):
            torch.mm(dys[i].t(), acts[i])
            if i > 0:
                torch.mm(dys[i], ws[i])

    out["c2_mlp_gemm_fwd_bwd_ms_f32"] = round(median_ms(c2, 10, 3), 3)
    progress("cpu baseline: torch C2 chain done")
    # C4: every layer's forward, grad input and grad weight
    layers = [(3, 64, 3, 1, 1, 32), (64, 64, 3, 1, 1, 32), (64, 128, 3, 2, 1, 32), (128, 256, 3, 2, 1, 16),
              (64, 128, 1, 2, 0, 32), (128, 256, 1, 2, 0, 16)]
    data = []
    for cin, cout, k, st, pd, hw in layers:
        x = torch.randn((128, cin, hw, hw), generator=g)
        w = torch.randn((cout, cin, k, k), generator=g) * (2.0 / (cin * k * k)) ** 0.5
        ho = (hw + 2 * pd - k) // st + 1
        dy = torch.randn((128, cout, ho, ho), generator=g)
        data.append((x, w, dy, st, pd))

    def c4():
        for x, w, dy, st, pd in data:
            F.conv2d(x, w, stride=st, padding=pd)
            torch.ops.aten.convolution_backward(dy, x, w, None, [st, st], [pd, pd], [1, 1], False, [0, 0], 1,
                                                [True, True, False])

    out["c4_resnet_conv_fwd_bwd_ms_f32"] = round(median_ms(c4, 5, 1), 3)
    progress("cpu baseline: torch C4 chain done")
    out["chains_sample"] = "whole C2 and C4 steps (float32); C2 median of 10 after 3, C4 median of 5 after 1"
    return out


def cpu_baseline():
    """The reference path on the host cores. `value`: the oracle (the
    reference SIMD tile's algorithm restated in C, oracle/gemm_oracle.c,
    sequential-k float32 FMA per output) on whole rows of the headline fp16
    8192^3 product; torch's CPU device and the lavapipe probe beside it."""
    import numpy as np
    from oracle import oracle as orc

    orc.load()
    host = host_info()
    cores = max(1, host["usable_cores"])
    n, rows = 8192, 256
    rng = np.random.default_rng(0)
    a = rng.standard_normal((rows, n)).astype(np.float16).view(np.uint16)
    b = rng.standard_normal((n, n)).astype(np.float16).view(np.uint16)
    t0 = time.perf_counter()
    orc.gemm(a, b, orc.F16, threads=cores)
    dt = time.perf_counter() - t0
    progress(f"cpu baseline: oracle rows done ({dt:.1f} s)")
    tfl = 2.0 * rows * n * n / dt / 1e12
    return {
        "value": round(tfl, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "label": "reference algorithm restated on CPU",
        "sample": f"{rows} of 8192 rows of the fp16 8192^3 mm (oracle/gemm_oracle.c, sequential-k fp32 FMA), "
                  f"{dt:.2f} s on {cores} threads",
        "host": host,
        "lavapipe": lavapipe_status(),
        "torch_cpu": torch_cpu_baselines(cores),
    }


if __name__ == "__main__":
    main()
