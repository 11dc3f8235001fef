"""Times every kernel of the GEMM kernel-choice table on a set of products.

    python -m torchvulkan_amd.tune                 # the benchmark configs' products, a table on stdout
    python -m torchvulkan_amd.tune --record        # and record each product's fastest kernel in the tuning file
    python -m torchvulkan_amd.tune --shape 4096x1024x512:f16:nt ...
    python -m torchvulkan_amd.tune --conv [--record]   # the C4 convolutions' kernel families, each direction

For each product it lists tvk_gemm_candidates, records one candidate at a
time with tvk_gemm_choose (memory only), times tvk_gemm over 7 spans of 10
launches (median, HIP events on the library's stream) and prints the
shape-chosen kernel beside the fastest. With --record the fastest is persisted
to the tuning file (tvk_gemm_choose with persist), so later processes pick it
for the product's shape class. This is the reference's first-call tuning
(src/vulkan/autotuner.cpp:123-223) run ahead of time over chosen products.

Products are "MxNxK[:dtype[:layout[:batch[:bias]]]]"; layout is two letters,
n (row-major) or t (transposed view), for A and B; bias is "n" (broadcast row
vector) or "c" (a full C-in with alpha 0.5, beta 1).
"""
from __future__ import annotations

import argparse
import ctypes as C
import statistics

import torch

from torchvulkan_amd import _abi

DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}

# (name, M, N, K, dtype, layout, batch, bias): the products of the benchmark configs
CONFIG_PRODUCTS = [
    ("C1 fp32 1024^3", 1024, 1024, 1024, "f32", "nn", 0, None),
    ("C2 fwd 256x784->4096 (+bias)", 256, 4096, 784, "f16", "nt", 0, "n"),
    ("C2 fwd 256x4096->4096 (+bias)", 256, 4096, 4096, "f16", "nt", 0, "n"),
    ("C2 fwd 256x4096->10 (+bias)", 256, 10, 4096, "f16", "nt", 0, "n"),
    ("C2 bwd dX 256x4096x4096", 256, 4096, 4096, "f16", "nn", 0, None),
    ("C2 bwd dX 256x784x4096", 256, 784, 4096, "f16", "nn", 0, None),
    ("C2 bwd dW 4096x4096x256", 4096, 4096, 256, "f16", "tn", 0, None),
    ("C2 bwd dW 4096x784x256", 4096, 784, 256, "f16", "tn", 0, None),
    ("C2 bwd dW 10x4096x256", 10, 4096, 256, "f16", "tn", 0, None),
    ("C3 q 8192x512x512", 8192, 512, 512, "f16", "nt", 0, None),
    ("C3 kv 8192x256x512", 8192, 256, 512, "f16", "nt", 0, None),
    ("C3 gate_up 8192x3072x512", 8192, 3072, 512, "f16", "nt", 0, None),
    ("C3 down 8192x512x1536", 8192, 512, 1536, "f16", "nt", 0, None),
    ("C3 head 8192x96x512", 8192, 96, 512, "f16", "nt", 0, None),
    ("C3 bwd dW 512x3072x8192", 512, 3072, 8192, "f16", "tn", 0, None),
    ("C3 bwd dX 8192x512x3072", 8192, 512, 3072, "f16", "nn", 0, None),
    ("C3 QK^T 256x(256x256x64)", 256, 256, 64, "f16", "nt", 256, None),
    ("C3 PV 256x(256x64x256)", 256, 64, 256, "f16", "nn", 256, None),
    ("C5 8192^3 f16", 8192, 8192, 8192, "f16", "nn", 0, None),
    ("C5 8192^3 bf16", 8192, 8192, 8192, "bf16", "nn", 0, None),
    ("C5 8192^3 f16 A^T", 8192, 8192, 8192, "f16", "tn", 0, None),
    ("C5 8192^3 f16 B^T", 8192, 8192, 8192, "f16", "nt", 0, None),
    ("C5 skinny 16x14336x4096", 16, 14336, 4096, "f16", "nn", 0, None),
    ("C5 ragged 1000x3000x777", 1000, 3000, 777, "f16", "nn", 0, None),
    ("C5 baddbmm 64x(512x512x128)", 512, 512, 128, "f16", "nn", 64, "c"),
]


def parse_shape(text: str):
    parts = text.split(":")
    M, N, K = (int(v) for v in parts[0].split("x"))
    dt = parts[1] if len(parts) > 1 else "f16"
    lay = parts[2] if len(parts) > 2 else "nn"
    batch = int(parts[3]) if len(parts) > 3 else 0
    bias = parts[4] if len(parts) > 4 else None
    return (text, M, N, K, dt, lay, batch, bias)


def operands(M, N, K, dt, lay, batch, bias, gen):
    dtype = DTYPES[dt]
    lead = (batch,) if batch else ()

    def mat(rows, cols, trans):
        shape = lead + ((cols, rows) if trans else (rows, cols))
        x = torch.randn(shape, generator=gen).to(dtype).to("cuda")
        return x.transpose(-1, -2) if trans else x

    a = mat(M, K, lay[0] == "t")
    b = mat(K, N, lay[1] == "t")
    c = torch.empty(lead + (M, N), dtype=dtype, device="cuda")
    kw = {}
    if bias == "n":
        kw = dict(bias=torch.randn((N,), generator=gen).to(dtype).to("cuda"), beta=1.0)
    elif bias == "c":
        kw = dict(bias=torch.randn(lead + (M, N), generator=gen).to(dtype).to("cuda"), alpha=0.5, beta=1.0)
    return a, b, c, kw


def time_calls(call, spans=7, per_span=10) -> float:
    """Median over spans of the average time of `call` (us). Each span starts behind a short GPU wait
    (torch.cuda._sleep, on the same stream), so the host has queued the whole span before the GPU reaches
    it and the span measures the kernels back to back rather than the host's launch rate."""
    for _ in range(3):
        _abi.check(call())
    torch.cuda.synchronize()
    out = []
    for _ in range(spans):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(200_000)
        e0.record()
        for _ in range(per_span):
            call()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3 / per_span)
    return statistics.median(out)


def time_launches(lib, desc, spans=7, per_span=10) -> float:
    """Median over spans of the average tvk_gemm launch time (us)."""
    return time_calls(lambda: lib.tvk_gemm(C.byref(desc)), spans, per_span)


def tune_product(lib, spec, gen, record: bool):
    name, M, N, K, dt, lay, batch, bias = spec
    a, b, c, kw = operands(M, N, K, dt, lay, batch, bias, gen)
    stream = torch.cuda.current_stream().cuda_stream
    names = _abi.gemm_candidates(a, b, c, **kw)
    desc = _abi.make_gemm_desc(a, b, c, kw.get("bias"), kw.get("alpha", 1.0), kw.get("beta", 0.0), 0, stream)
    # Two passes over the candidates, each keeping its faster median: the clock
    # ramps up over the first milliseconds after an idle spell (the operand
    # set-up), which in one pass counts against whichever candidate runs first.
    times = {}
    for _ in range(2):
        for n in names:
            _abi.tune_reset()
            _abi.gemm_choose(a, b, c, n, **kw)
            t = time_launches(lib, desc)
            times[n] = min(times.get(n, t), t)
    _abi.tune_reset()
    best = min(times, key=times.get)
    if record:
        _abi.gemm_choose(a, b, c, best, persist=True, **kw)
    flops = 2.0 * M * N * K * max(batch, 1)
    return name, names[0], times[names[0]], best, times[best], flops, times


# (name, c_in, c_out, kernel, stride, padding, input size): the C4 ResNet convolutions at batch 128
CONV_LAYERS = [
    ("3->64 3x3 s1", 3, 64, 3, 1, 1, 32),
    ("64->64 3x3 s1", 64, 64, 3, 1, 1, 32),
    ("64->128 3x3 s2", 64, 128, 3, 2, 1, 32),
    ("128->256 3x3 s2", 128, 256, 3, 2, 1, 16),
    ("64->128 1x1 s2", 64, 128, 1, 2, 0, 32),
    ("128->256 1x1 s2", 128, 256, 1, 2, 0, 16),
]
CONV_MODES = (("fwd", _abi.TVK_CONV_FWD), ("dgrad", _abi.TVK_CONV_DGRAD), ("wgrad", _abi.TVK_CONV_WGRAD))


def tune_conv(lib, layer, gen, record: bool, batch: int = 128):
    """Every kernel family of the layer's three directions (tvk_conv_candidates), each recorded in turn
    (tvk_conv_choose, memory only) and timed through the ordinary entry point; two passes, the faster
    median kept."""
    name, cin, cout, k, s, p, hw = layer
    f16 = torch.float16
    ho = (hw + 2 * p - k) // s + 1
    x = torch.randn((batch, cin, hw, hw), generator=gen).to(f16).to("cuda")
    w = (torch.randn((cout, cin, k, k), generator=gen) * (2.0 / (cin * k * k)) ** 0.5).to(f16).to("cuda")
    y = torch.randn((batch, cout, ho, ho), generator=gen).to(f16).to("cuda")
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    rows = []
    for mode_name, mode in CONV_MODES:
        d = _abi.conv_problem(*((x, w, y) if mode == _abi.TVK_CONV_FWD else (dx, w, y) if mode == _abi.TVK_CONV_DGRAD
                                else (x, dw, y)), stride=s, padding=p)
        entry = getattr(lib, _abi._CONV_ENTRY[mode])
        names = _abi.conv_candidates(d, mode)
        times = {}
        for _ in range(2):
            for n in names:
                _abi.tune_reset()
                _abi.conv_choose(d, mode, n)
                t = time_calls(lambda: entry(C.byref(d)))
                times[n] = min(times.get(n, t), t)
        _abi.tune_reset()
        best = min(times, key=times.get)
        if record:
            _abi.conv_choose(d, mode, best, persist=True)
        rows.append((name, mode_name, names[0], times[names[0]], best, times[best], times))
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", action="append", default=[], help="MxNxK[:dtype[:layout[:batch[:bias]]]]")
    ap.add_argument("--record", action="store_true", help="persist each product's fastest kernel")
    ap.add_argument("--all", action="store_true", help="print every candidate's time")
    ap.add_argument("--conv", action="store_true", help="the C4 convolutions' kernel families instead of products")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("torchvulkan_amd.tune needs a GPU")
    lib = _abi.load()
    if args.conv:
        gen = torch.Generator().manual_seed(0)
        print("| layer (batch 128, fp16) | direction | shape rule's family | us | fastest family | us | ratio |")
        print("|---|---|---|---|---|---|---|")
        for layer in CONV_LAYERS:
            for name, mode, chosen, t0, best, t1, times in tune_conv(lib, layer, gen, args.record):
                print(f"| {name} | {mode} | `{chosen}` | {t0:.2f} | `{best}` | {t1:.2f} | {t0 / t1:.2f} |", flush=True)
                if args.all:
                    print("|  |  | " + ", ".join(f"`{n}` {t:.1f}" for n, t in sorted(times.items(), key=lambda x: x[1]))
                          + " | | | | |")
        if args.record:
            print(f"recorded in {_abi.tune_path()}")
        return 0
    specs = [parse_shape(s) for s in args.shape] or CONFIG_PRODUCTS
    gen = torch.Generator().manual_seed(0)
    print("| product | shape rule's kernel | us | fastest kernel | us | ratio | TFLOP/s (fastest) |")
    print("|---|---|---|---|---|---|---|")
    for spec in specs:
        name, chosen, t0, best, t1, flops, times = tune_product(lib, spec, gen, args.record)
        print(f"| {name} | `{chosen}` | {t0:.2f} | `{best}` | {t1:.2f} | {t0 / t1:.2f} | {flops / (t1 * 1e-6) / 1e12:.1f} |",
              flush=True)
        if args.all:
            print("|  | " + ", ".join(f"`{n}` {t:.1f}" for n, t in sorted(times.items(), key=lambda x: x[1])) + " | | | | | |")
    if args.record:
        print(f"recorded in {_abi.tune_path()}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
