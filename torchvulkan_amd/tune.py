"""Times every kernel of the GEMM kernel-choice table on a set of products.

    python -m torchvulkan_amd.tune                 # the benchmark configs' products, a table on stdout
    python -m torchvulkan_amd.tune --record        # and record each product's fastest kernel in the tuning file
    python -m torchvulkan_amd.tune --shape 4096x1024x512:f16:nt ...

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


def time_launches(lib, desc, spans=7, per_span=10) -> float:
    """Median over spans of the average launch time (us)."""
    for _ in range(3):
        _abi.check(lib.tvk_gemm(C.byref(desc)))
    torch.cuda.synchronize()
    out = []
    for _ in range(spans):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(per_span):
            lib.tvk_gemm(C.byref(desc))
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3 / per_span)
    return statistics.median(out)


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


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", action="append", default=[], help="MxNxK[:dtype[:layout[:batch[:bias]]]]")
    ap.add_argument("--record", action="store_true", help="persist each product's fastest kernel")
    ap.add_argument("--all", action="store_true", help="print every candidate's time")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("torchvulkan_amd.tune needs a GPU")
    lib = _abi.load()
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
