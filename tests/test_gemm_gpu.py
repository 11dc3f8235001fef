"""GEMM parity on the GPU, through the C ABI (tvk_gemm), against the oracle.

Cases follow the configs of the path: C1 fp32 mm 1024^3 (+relu, sum), the
MLP addmm chain and its backward GEMMs (C2), the transformer linears and
head-strided bmm (C3), and the sweep (C5): square 8192^3, skinny
16x4096x14336, ragged 1000x777x3000, baddbmm 64x512x512x128 with alpha=0.5,
beta=1, and transposed / sliced views. Edge cases follow the reference's
rules (src/api/ops/matmul.cpp:259,284-288): empty outputs, K == 0, beta == 0
with a NaN bias. Tolerances are in tests/gemm_cases.py.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gemm_cases import (TOL, gen, assert_bit_exact, assert_close, decode, oracle_mm, randint, randn, to_np)

pytestmark = pytest.mark.gpu

DEV = "cuda"
F16_TYPES = [torch.float16, torch.bfloat16]
ALL_TYPES = [torch.float32, torch.float16, torch.bfloat16]


def run(abi, a, b, out_shape, dtype, bias=None, alpha=1.0, beta=0.0, act=0, exact=False, kernel=None):
    """Runs tvk_gemm on device copies of host views a/b (strides kept); `kernel`
    records that candidate for the product in the kernel-choice table first."""
    da = a.to(DEV) if a.is_contiguous() else _device_view(a)
    db = b.to(DEV) if b.is_contiguous() else _device_view(b)
    dbias = None if bias is None else bias.to(DEV)
    c = torch.empty(out_shape, dtype=dtype, device=DEV)
    kw = dict(bias=dbias, alpha=alpha, beta=beta, activation=act, exact=exact)
    if kernel:
        abi.gemm_choose(da, db, c, kernel, **kw)
    try:
        abi.gemm(da, db, c, **kw)
        torch.cuda.synchronize()
        plan = abi.gemm_plan(da, db, c, **kw)
    finally:
        if kernel:
            abi.tune_reset()
    return decode(to_np(c), dtype), plan


def _device_view(t: torch.Tensor) -> torch.Tensor:
    """Device tensor with the same strides as the host view (copies its storage)."""
    base = t.as_strided((t.untyped_storage().nbytes() // t.element_size(),), (1,), 0)
    dbase = base.to(DEV)
    return dbase.as_strided(t.shape, t.stride(), t.storage_offset())


# ---------------------------------------------------------------------------
# bit-exact cases
# ---------------------------------------------------------------------------

def test_c1_fp32_mm_1024_bit_exact(gpu):
    a = randn((1024, 1024), torch.float32, 0)
    b = randn((1024, 1024), torch.float32, 1)
    got, plan = run(gpu, a, b, (1024, 1024), torch.float32)
    ref = oracle_mm(a, b, torch.float32)
    assert plan.startswith("gemm_seq_mfma")
    assert_bit_exact(got, ref, plan)
    # the config's tail: relu then sum (ops the reference runs on its CPU fallback)
    assert np.maximum(got, 0).astype(np.float64).sum() == np.maximum(ref, 0).astype(np.float64).sum()


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("shape", [(256, 256, 256), (300, 520, 136), (64, 80, 24), (1024, 1024, 160), (4096, 1024, 160)])
def test_integer_exact_all_layouts(gpu, dtype, ta, tb, shape):
    # integer operands: every summation order gives identical bits. The first
    # four have fewer 128x128 tiles than half the CUs (64x64 tiles); the last
    # takes the 128x128 ring
    M, N, K = shape
    a = randint((K, M) if ta else (M, K), dtype, 10)
    b = randint((N, K) if tb else (K, N), dtype, 11)
    a = a.t() if ta else a
    b = b.t() if tb else b
    got, plan = run(gpu, a, b, (M, N), dtype)
    ref = oracle_mm(a, b, dtype)
    assert np.array_equal(got, ref), plan


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_integer_exact_ragged_unaligned(gpu, dtype):
    # K rows of 777 halves are not 16-byte aligned: the element-wise load path
    a = randint((100, 77), dtype, 12)
    b = randint((77, 300), dtype, 13)
    got, plan = run(gpu, a, b, (100, 300), dtype)
    assert "mfma" in plan
    assert np.array_equal(got, oracle_mm(a, b, dtype)), plan


# ---------------------------------------------------------------------------
# the 256x256 LDS-ring kernel (gemm16_dma_256x256): integer operands keep the
# fp32 accumulator exact, so the result is the exact sum rounded once to T, in
# any summation order; float64 numpy plus one torch rounding is the reference
# ---------------------------------------------------------------------------

def _exact_ref(a, b, dtype):
    r = a.double().numpy() @ b.double().numpy()
    return decode(to_np(torch.from_numpy(r).to(dtype)), dtype)


DMA_SHAPES = [
    (4096, 3072, 96),    # K shorter than the four-stage ring
    (4000, 3000, 32),    # one stage; ragged M and N
    (2560, 5120, 1024),
]


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("shape", DMA_SHAPES)
def test_dma_kernel_integer_exact(gpu, dtype, ta, tb, shape):
    M, N, K = shape
    lo, hi = (-4, 5) if K <= 128 else (-2, 3)
    a = randint((K, M) if ta else (M, K), dtype, 14, lo, hi)
    b = randint((N, K) if tb else (K, N), dtype, 15, lo, hi)
    a = a.t() if ta else a
    b = b.t() if tb else b
    got, plan = run(gpu, a, b, (M, N), dtype)
    assert plan == "gemm16_dma_256x256"
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("shape", [(1000, 1024, 96), (8192, 512, 512), (4000, 136, 64)])
def test_dma_kernel_128_tiles_integer_exact(gpu, dtype, ta, tb, shape):
    # mid-size products take the same ring on 128x128 tiles (recorded in the
    # kernel-choice table where the shape rule prefers another kernel)
    M, N, K = shape
    a = randint((K, M) if ta else (M, K), dtype, 28, -2, 3)
    b = randint((N, K) if tb else (K, N), dtype, 29, -2, 3)
    a = a.t() if ta else a
    b = b.t() if tb else b
    got, plan = run(gpu, a, b, (M, N), dtype, kernel="gemm16_dma_128x128")
    assert plan == "gemm16_dma_128x128"
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan


# C-in through the 256x256 kernel's epilogue (16-byte bias chunks requested
# before the first pass): K of 3, 4 and 32 ring stages; ragged M, a partial
# 8-column N tile, bias broadcast over the batch or over the rows, a bias of
# padded rows, relu
BIAS_RING_CASES = [
    # batch, M, N, K, bias kind, activation
    (3, 300, 520, 96, "full", 0),
    (2, 512, 512, 128, "batch_broadcast", 0),
    (1, 1000, 776, 1024, "row_broadcast", 1),
    (2, 256, 264, 256, "padded_rows", 0),
]


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("case", BIAS_RING_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}x{c[3]}-{c[4]}")
def test_dma256_c_in_epilogue(gpu, dtype, case):
    B, M, N, K, kind, act = case
    a = randint((B, M, K), dtype, 33, -3, 4)
    b = randint((B, K, N), dtype, 34, -3, 4)
    if kind == "full":
        bias_h = randint((B, M, N), dtype, 35)
        bias = bias_h.to(DEV)
    elif kind == "batch_broadcast":
        bias_h = randint((M, N), dtype, 35).expand(B, M, N)
        bias = bias_h[0].to(DEV).expand(B, M, N)
    elif kind == "row_broadcast":
        bias_h = randint((N,), dtype, 35).expand(B, M, N)
        bias = bias_h[0, 0].to(DEV).expand(B, M, N)
    else:
        full = randint((B, M, N + 8), dtype, 35)
        bias_h = full[:, :, :N]
        bias = full.to(DEV)[:, :, :N]
    da, db = a.to(DEV), b.to(DEV)
    c = torch.empty((B, M, N), dtype=dtype, device=DEV)
    kw = dict(bias=bias, alpha=0.5, beta=2.0, activation=act)
    gpu.gemm_choose(da, db, c, "gemm16_dma_256x256", **kw)
    try:
        c.fill_(float("nan"))
        gpu.gemm(da, db, c, **kw)
        torch.cuda.synchronize()
        assert gpu.gemm_plan(da, db, c, **kw) == "gemm16_dma_256x256"
    finally:
        gpu.tune_reset()
    # integer operands: the product, alpha * it + beta * bias and relu are exact
    # in float32, so the one rounding to the dtype gives the reference's bits
    r = 0.5 * (a.double().numpy() @ b.double().numpy()) + 2.0 * bias_h.double().numpy()
    if act == 1:
        r = np.maximum(r, 0.0)
    want = decode(to_np(torch.from_numpy(r).to(dtype)), dtype)
    assert np.array_equal(decode(to_np(c), dtype), want)


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_dma_kernel_128_tiles_batched_epilogue(gpu, dtype):
    # baddbmm-like: batched, C-in through the fused epilogue, alpha and beta
    a = randn((4, 512, 512), dtype, 30)
    b = randn((4, 512, 384), dtype, 31)
    inp = randn((4, 512, 384), dtype, 32)
    got, plan = run(gpu, a, b, (4, 512, 384), dtype, bias=inp, alpha=0.5, beta=1.0, kernel="gemm16_dma_128x128")
    assert plan == "gemm16_dma_128x128"
    assert_close(got, oracle_mm(a, b, dtype, bias=inp, alpha=0.5, beta=1.0), dtype, plan)


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("kernel", ["gemm16_dma_128x128", "gemm16_dma_128x256", "gemm16_dma_256x128", "gemm16_dma_256x256"])
def test_dma_epilogue_variants_exact(gpu, dtype, kernel):
    """The LDS-ring kernels' epilogue on integer-valued data, where every result is exact: no bias, a row
    bias, a full C-in, ReLU and none, alpha 0.5 and beta 2. The output rows hold 256 elements of which
    N = 250 are the product (a last chunk of two columns), and one C-in has an odd row stride (the
    per-element path) while the others have 16-byte rows (the select path). Elements past N stay zero."""
    from torchvulkan_amd import _abi
    M, N, K = 300, 250, 32
    a = randint((M, K), dtype, 60, lo=-2, hi=3).to(DEV)
    w = randint((N, K), dtype, 61, lo=-2, hi=3).to(DEV)
    cbuf = torch.zeros((M, 256), dtype=dtype, device=DEV)
    c = cbuf[:, :N]
    if kernel not in _abi.gemm_candidates(a, w.t(), c):
        pytest.skip(f"{kernel} is not a candidate for {M}x{N}x{K}")
    exact = a.double().cpu() @ w.double().cpu().t()
    biases = [None, randint((N,), dtype, 62, lo=-2, hi=3), randint((M, N), dtype, 63, lo=-2, hi=3),
              randint((M, N + 1), dtype, 64, lo=-2, hi=3)[:, :N]]
    for bi, bias in enumerate(biases):
        for act in (orc.ACT_NONE, orc.ACT_RELU):
            dbias = None if bias is None else (bias.to(DEV) if bias.is_contiguous() else _device_view(bias))
            kw = dict(bias=dbias, alpha=0.5, beta=2.0 if bias is not None else 0.0, activation=act)
            cbuf.zero_()
            _abi.gemm_choose(a, w.t(), c, kernel, **kw)
            try:
                _abi.gemm(a, w.t(), c, **kw)
                torch.cuda.synchronize()
                plan = _abi.gemm_plan(a, w.t(), c, **kw)
            finally:
                _abi.tune_reset()
            assert plan == kernel
            ref = exact * 0.5 + (0.0 if bias is None else 2.0 * bias.double())
            if act == orc.ACT_RELU:
                ref = ref.clamp(min=0.0)
            got = cbuf.cpu()
            assert torch.equal(got[:, :N].double(), ref.to(dtype).double()), f"bias case {bi}, act {act}"
            assert (got[:, N:] == 0).all(), "wrote past N"


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_dma_kernel_column_edge_inside_a_chunk(gpu, dtype):
    # N = 3001 of rows strided 3008: the last 16-byte chunk of a B row would
    # straddle N, so the ring kernel declines and another kernel runs
    K = 64
    a = randint((4096, K), dtype, 16)
    wide = randint((K, 3008), dtype, 17)
    b = wide[:, :3001]
    got, plan = run(gpu, a, b, (4096, 3001), dtype)
    assert plan != "gemm16_dma_256x256"
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_dma_kernel_batched(gpu, dtype):
    a = randint((3, 1024, 320), dtype, 18)
    b = randint((3, 320, 4096), dtype, 19)
    got, plan = run(gpu, a, b, (3, 1024, 4096), dtype)
    assert plan == "gemm16_dma_256x256"
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("act", [orc.ACT_NONE, orc.ACT_RELU, orc.ACT_GELU])
def test_dma_kernel_epilogue_sampled_rows(gpu, dtype, act):
    M, N, K = 4096, 3072, 320
    a = randn((M, K), dtype, 20)
    b = randn((N, K), dtype, 21).t()
    bias = randn((N,), dtype, 22)
    got, plan = run(gpu, a, b, (M, N), dtype, bias=bias, alpha=0.5, beta=2.0, act=act)
    assert plan == "gemm16_dma_256x256"
    rows = np.r_[0:3, 255:258, 1000:1003, M - 3:M]
    ref = oracle_mm(a[rows], b, dtype, bias=bias, alpha=0.5, beta=2.0, act=act)
    assert_close(got[rows], ref, dtype, plan)


# ---------------------------------------------------------------------------
# operands whose rows miss the 16-byte layout are copied once into an aligned,
# zero-padded layout (workspace) before the vectorized kernels run
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("case", [
    ((1000, 777), False, (777, 3000), False, None),    # C5 ragged: A rows of 777
    ((777, 1000), True, (777, 3001), False, None),     # A m-contiguous view, B rows of 3001
    ((3000, 777), False, (3000, 777), True, None),     # B = W^T with K = 777
    ((600, 333), False, (333, 700), False, 3),         # batched, both repacked
    # K off the 32 grid on the LDS-ring split-K kernel (its last k step runs
    # whole, reading zeros past K): A repacked with zero-padded rows, both
    # repacked, and no repack at all (rows past K outside both buffer ranges)
    ((512, 8190), False, (8190, 512), False, None),
    ((512, 8190), False, (512, 8190), True, None),
    ((8190, 512), True, (8190, 512), False, None),
])
def test_repacked_operands_integer_exact(gpu, dtype, case):
    ashape, ta, bshape, tb, batch = case
    lead = (batch,) if batch else ()
    a = randint(lead + ashape, dtype, 26, -2, 3)
    b = randint(lead + bshape, dtype, 27, -2, 3)
    a = a.transpose(-1, -2) if ta else a
    b = b.transpose(-1, -2) if tb else b
    M, N = a.shape[-2], b.shape[-1]
    got, plan = run(gpu, a, b, lead + (M, N), dtype)
    assert "mfma" in plan or "dma" in plan, plan
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan


# ---------------------------------------------------------------------------
# split-K (few output tiles, long K): float32 partials summed in split order
# ---------------------------------------------------------------------------

SPLIT_CASES = [
    # (M, N, K, ta, tb, batch): dW = dY^T X of a transformer layer, a batch-256
    # MLP layer, K not a multiple of the chunk, and a batched case
    (512, 512, 8192, True, False, 1),
    (256, 4096, 4096, False, True, 1),
    (384, 320, 5000, False, False, 1),
    (256, 256, 4096, False, False, 2),
]


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("case", SPLIT_CASES)
def test_split_k_integer_exact(gpu, dtype, case):
    M, N, K, ta, tb, batch = case
    lead = (batch,) if batch > 1 else ()
    a = randint(lead + ((K, M) if ta else (M, K)), dtype, 23, -2, 3)
    b = randint(lead + ((N, K) if tb else (K, N)), dtype, 24, -2, 3)
    a = a.transpose(-1, -2) if ta else a
    b = b.transpose(-1, -2) if tb else b
    got, plan = run(gpu, a, b, lead + (M, N), dtype)
    # the LDS-ring kernel takes the split where it applies (K a multiple of 32)
    assert plan == ("gemm16_dma_128x128_splitk" if K % 32 == 0 else "gemm16_mfma_128x128_splitk")
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan
    if K % 32 == 0:
        # the register-staged split kernel on the same product, and an odd split count
        for kernel in ("gemm16_mfma_128x128_splitk:4", "gemm16_dma_128x128_splitk:2"):
            got, plan = run(gpu, a, b, lead + (M, N), dtype, kernel=kernel)
            assert plan == kernel.split(":")[0]
            assert np.array_equal(got, _exact_ref(a, b, dtype)), kernel


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("act", [orc.ACT_NONE, orc.ACT_RELU, orc.ACT_GELU])
def test_split_k_epilogue_sampled_rows(gpu, dtype, act):
    # C2 forward layer: addmm(bias, x, W^T) with the fused activation
    M, N, K = 256, 4096, 4096
    a = torch.rand((M, K), generator=gen(25)).to(dtype)
    b = ((torch.rand((N, K), generator=gen(26)) * 2 - 1) * K ** -0.5).to(dtype).t()
    bias = ((torch.rand((N,), generator=gen(27)) * 2 - 1) * K ** -0.5).to(dtype)
    got, plan = run(gpu, a, b, (M, N), dtype, bias=bias, alpha=1.0, beta=1.0, act=act)
    assert plan == "gemm16_dma_128x128_splitk"
    rows = np.r_[0:4, 127:130, M - 4:M]
    ref = oracle_mm(a[rows], b, dtype, bias=bias, alpha=1.0, beta=1.0, act=act)
    assert_close(got[rows], ref, dtype, plan)


# ---------------------------------------------------------------------------
# C2: MLP addmm chain (fp16 / fp32 accumulate), forward and backward
# ---------------------------------------------------------------------------

MLP = [784, 4096, 4096, 4096, 10]


@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("layer", range(4))
def test_c2_mlp_forward_addmm(gpu, dtype, layer):
    fin, fout = MLP[layer], MLP[layer + 1]
    bound = 1.0 / np.sqrt(fin)
    g = torch.Generator().manual_seed(20 + layer)
    x = torch.rand((256, fin), generator=g).to(dtype)
    w = ((torch.rand((fout, fin), generator=g) * 2 - 1) * bound).to(dtype)
    bias = ((torch.rand((fout,), generator=g) * 2 - 1) * bound).to(dtype)
    got, plan = run(gpu, x, w.t(), (256, fout), dtype, bias=bias, beta=1.0)
    ref = oracle_mm(x, w.t(), dtype, bias=bias, beta=1.0)
    assert_close(got, ref, dtype, plan)


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_c2_mlp_backward_gemms(gpu, dtype):
    g = torch.Generator().manual_seed(30)
    dy = torch.randn((256, 4096), generator=g).to(dtype)
    w = (torch.randn((4096, 4096), generator=g) * 0.02).to(dtype)
    x = torch.rand((256, 784), generator=g).to(dtype)
    dy1 = torch.randn((256, 4096), generator=g).to(dtype)
    # dX = dY . W   (W is [out, in] row-major: B is n-contiguous)
    got, plan = run(gpu, dy, w, (256, 4096), dtype)
    assert_close(got, oracle_mm(dy, w, dtype), dtype, "dX " + plan)
    # dW = dY^T . X (dY^T is an m-contiguous transposed view)
    got, plan = run(gpu, dy1.t(), x, (4096, 784), dtype)
    assert_close(got, oracle_mm(dy1.t(), x, dtype), dtype, "dW " + plan)


# ---------------------------------------------------------------------------
# C3: transformer linears and head-strided bmm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("fin,fout", [(512, 512), (512, 256), (512, 3072), (1536, 512), (512, 96)])
def test_c3_linear(gpu, dtype, fin, fout):
    x = randn((8192, fin), dtype, 40)
    w = randn((fout, fin), dtype, 41, std=0.02)
    got, plan = run(gpu, x, w.t(), (8192, fout), dtype)
    assert_close(got, oracle_mm(x, w.t(), dtype), dtype, plan)


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_c3_head_strided_bmm(gpu, dtype):
    # one sequence of the batch: q/k/v as [heads, seq, head_dim] views of [seq, heads*head_dim]
    q = randn((256, 8 * 64), dtype, 50)
    k = randn((256, 8 * 64), dtype, 51)
    qh = q.view(256, 8, 64).transpose(0, 1)            # [8, 256, 64] strides (64, 512, 1)
    kt = k.view(256, 8, 64).transpose(0, 1).transpose(1, 2)  # [8, 64, 256] strides (64, 1, 512)
    got, plan = run(gpu, qh, kt, (8, 256, 256), dtype)
    assert plan == "gemm16_mfma_64x64"
    assert_close(got, oracle_mm(qh, kt, dtype), dtype, "QK^T " + plan)
    p = randn((8, 256, 256), dtype, 52, std=0.1)
    v = randn((256, 8 * 64), dtype, 53)
    vh = v.view(256, 8, 64).transpose(0, 1)            # [8, 256, 64]
    got, plan = run(gpu, p, vh, (8, 256, 64), dtype)
    assert_close(got, oracle_mm(p, vh, dtype), dtype, "PV " + plan)


# ---------------------------------------------------------------------------
# C5: sweep
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ALL_TYPES)
def test_c5_ragged(gpu, dtype):
    a = randn((1000, 777), dtype, 60)
    b = randn((777, 3000), dtype, 61)
    got, plan = run(gpu, a, b, (1000, 3000), dtype)
    ref = oracle_mm(a, b, dtype)
    if dtype == torch.float32:
        assert_bit_exact(got, ref, plan)
    assert_close(got, ref, dtype, plan)


@pytest.mark.parametrize("dtype", ALL_TYPES)
def test_c5_baddbmm(gpu, dtype):
    inp = randn((64, 512, 512), dtype, 70)
    b1 = randn((64, 512, 128), dtype, 71)
    b2 = randn((64, 128, 512), dtype, 72)
    got, plan = run(gpu, b1, b2, (64, 512, 512), dtype, bias=inp, alpha=0.5, beta=1.0)
    ref = oracle_mm(b1, b2, dtype, bias=inp, alpha=0.5, beta=1.0)
    if dtype == torch.float32:
        assert_bit_exact(got, ref, plan)
    assert_close(got, ref, dtype, plan)


@pytest.mark.parametrize("dtype", ALL_TYPES)
def test_c5_skinny(gpu, dtype):
    a = randn((16, 4096), dtype, 80)
    b = randn((4096, 14336), dtype, 81)
    got, plan = run(gpu, a, b, (16, 14336), dtype)
    assert_close(got, oracle_mm(a, b, dtype), dtype, plan)


@pytest.mark.parametrize("dtype", ALL_TYPES)
def test_c5_square_8192(gpu, dtype):
    # Full-size run. The oracle checks one seeded row in every 256-row band,
    # so every output tile is crossed by a checked row; a row-sum property
    # then covers all of C: sum_j C[i,j] == (A @ (B @ 1))[i] within the
    # spread the per-element rounding allows.
    a = randn((8192, 8192), dtype, 90)
    b = randn((8192, 8192), dtype, 91)
    got, plan = run(gpu, a, b, (8192, 8192), dtype)
    rng = np.random.default_rng(0)
    rows = np.arange(0, 8192, 256) + rng.integers(0, 256, 32)
    ref = oracle_mm(a[torch.from_numpy(rows)], b, dtype)
    if dtype == torch.float32:
        assert_bit_exact(got[rows], ref, plan)
    assert_close(got[rows], ref, dtype, plan)
    bsum = decode(to_np(b), dtype).astype(np.float64).sum(axis=1)
    rs = decode(to_np(a), dtype).astype(np.float64) @ bsum
    g64 = got.astype(np.float64)
    ulp = np.spacing(np.abs(got).astype(np.float16 if dtype == torch.float16 else np.float32)).astype(np.float64)
    if dtype == torch.bfloat16:
        ulp = np.abs(g64) * 2.0 ** -7
    var = (ulp ** 2).sum(axis=1) / 12 + ((1e-5 * (np.abs(g64) + 1)) ** 2).sum(axis=1) / 3
    assert np.all(np.abs(g64.sum(axis=1) - rs) <= 8 * np.sqrt(var) + 1e-9), plan


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_c5_transposed_and_sliced_views(gpu, dtype):
    big = randn((1100, 900), dtype, 100)
    a = big[50:1050:1, 100:877]               # [1000, 777] rows of stride 900
    b = randn((3000, 800), dtype, 101)[:, :777].t()   # [777, 3000] k-contiguous, sliced
    got, plan = run(gpu, a, b, (1000, 3000), dtype)
    assert_close(got, oracle_mm(a, b, dtype), dtype, plan)


# ---------------------------------------------------------------------------
# epilogue and edge cases
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ALL_TYPES)
@pytest.mark.parametrize("act", [orc.ACT_RELU, orc.ACT_GELU])
def test_activation_epilogue(gpu, dtype, act):
    a = randn((300, 200), dtype, 110)
    b = randn((200, 260), dtype, 111)
    bias = randn((260,), dtype, 112)
    got, plan = run(gpu, a, b, (300, 260), dtype, bias=bias, alpha=0.5, beta=2.0, act=act)
    assert_close(got, oracle_mm(a, b, dtype, bias=bias, alpha=0.5, beta=2.0, act=act), dtype, plan)


@pytest.mark.parametrize("dtype", ALL_TYPES)
def test_beta_zero_ignores_nan_bias(gpu, dtype):
    a = randn((64, 32), dtype, 120)
    b = randn((32, 48), dtype, 121)
    bias = torch.full((64, 48), float("nan"), dtype=dtype)
    got, _ = run(gpu, a, b, (64, 48), dtype, bias=bias, beta=0.0)
    assert not np.isnan(got).any()
    assert_close(got, oracle_mm(a, b, dtype), dtype)


@pytest.mark.parametrize("dtype", ALL_TYPES)
def test_k_zero(gpu, dtype):
    a = torch.empty((5, 0), dtype=dtype)
    b = torch.empty((0, 7), dtype=dtype)
    bias = randn((7,), dtype, 130)
    got, plan = run(gpu, a, b, (5, 7), dtype, bias=bias, beta=3.0)
    assert plan == "gemm_k0_fill"
    assert_close(got, oracle_mm(a, b, dtype, bias=bias, beta=3.0), dtype)
    got, _ = run(gpu, a, b, (5, 7), dtype)
    assert np.array_equal(got, np.zeros((5, 7), np.float32))


def test_empty_output_is_a_no_op(gpu):
    a = torch.empty((0, 8), dtype=torch.float16)
    b = randn((8, 4), torch.float16, 140)
    got, plan = run(gpu, a, b, (0, 4), torch.float16)
    assert got.shape == (0, 4) and plan == "none"


def test_fully_strided_operands_generic_path(gpu):
    # neither stride of A is 1: only the generic kernel accepts it
    big = randn((64, 96), torch.float16, 150)
    a = big[::2, ::3]          # [32, 32], strides (192, 3)
    b = randn((32, 40), torch.float16, 151)
    got, plan = run(gpu, a, b, (32, 40), torch.float16)
    assert plan == "gemm_generic"
    assert_close(got, oracle_mm(a, b, torch.float16), torch.float16, plan)


# ---------------------------------------------------------------------------
# TVK_GEMM_EXACT: every dtype in the reference SIMD tile's order, bit for bit
# ---------------------------------------------------------------------------

def _exact_cases(dtype):
    g = torch.Generator().manual_seed(160)
    x = torch.rand((256, 784), generator=g).to(dtype)
    w = ((torch.rand((4096, 784), generator=g) * 2 - 1) / 28.0).to(dtype)
    bias = ((torch.rand((4096,), generator=g) * 2 - 1) / 28.0).to(dtype)
    yield "mlp_fwd_addmm", x, w.t(), (256, 4096), dict(bias=bias, beta=1.0)
    dy = torch.randn((256, 1024), generator=g).to(dtype)
    yield "mlp_dW_transposed", dy.t(), x, (1024, 784), {}
    yield "ragged", randn((1000, 777), dtype, 161), randn((777, 300), dtype, 162), (1000, 300), {}
    q = randn((256, 512), dtype, 163)
    k = randn((256, 512), dtype, 164)
    yield ("head_strided_qk", q.view(256, 8, 64).transpose(0, 1),
           k.view(256, 8, 64).transpose(0, 1).transpose(1, 2), (8, 256, 256), {})
    inp = randn((8, 512, 512), dtype, 165)
    yield ("baddbmm", randn((8, 512, 128), dtype, 166), randn((8, 128, 512), dtype, 167), (8, 512, 512),
           dict(bias=inp, alpha=0.5, beta=1.0))
    yield "gelu", randn((300, 200), dtype, 168), randn((200, 260), dtype, 169), (300, 260), dict(act=orc.ACT_RELU)


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_exact_mode_bit_identical(gpu, dtype):
    for name, a, b, shape, kw in _exact_cases(dtype):
        got, plan = run(gpu, a, b, shape, dtype, exact=True, **kw)
        assert plan.startswith("gemm_seq_mfma"), plan
        ref = oracle_mm(a, b, dtype, **kw)
        assert_bit_exact(got, ref, f"{name} {plan}")


# ---------------------------------------------------------------------------
# M <= 16: the HBM-streaming kernels (gemm16_skinny_ring for B n-contiguous
# with aligned rows, split K with an ordered float32 reduction; the LDS
# transpose kernel otherwise)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", F16_TYPES)
@pytest.mark.parametrize("M,N,K,bt,aligned", [
    (16, 14336, 4096, False, True),   # C5 skinny, B row-major
    (16, 14336, 4096, True, True),    # B as a transposed weight view (k-contiguous)
    (1, 4096, 4096, True, True),      # one token through a linear
    (7, 1000, 2000, False, True),     # ragged rows / last strip (K % 32 != 0: not the ring)
    (9, 4000, 1024, False, True),     # ring, 8-way split, partial last strip
    (3, 32768, 96, False, True),      # ring without a split: direct epilogue
    (5, 777, 999, False, False),      # K and N not multiples of 8: element loads
    (16, 256, 64, True, True),        # K too small to split
])
def test_skinny_shapes(gpu, dtype, M, N, K, bt, aligned):
    a = randn((M, K), dtype, 200)
    b = randn((N, K), dtype, 201).t() if bt else randn((K, N), dtype, 201)
    bias = randn((N,), dtype, 202)
    got, plan = run(gpu, a, b, (M, N), dtype, bias=bias, alpha=0.5, beta=1.0)
    assert plan.startswith("gemm16_skinny"), plan
    assert_close(got, oracle_mm(a, b, dtype, bias=bias, alpha=0.5, beta=1.0), dtype, plan)


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_skinny_batched_and_repeated(gpu, dtype):
    # batched decode-like bmm; two calls in a row reuse the arrival counters
    a = randn((6, 4, 512), dtype, 210)
    b = randn((6, 512, 640), dtype, 211)
    for _ in range(2):
        got, plan = run(gpu, a, b, (6, 4, 640), dtype)
        assert plan.startswith("gemm16_skinny"), plan
        assert_close(got, oracle_mm(a, b, dtype), dtype, plan)


@pytest.mark.parametrize("dtype", F16_TYPES)
def test_skinny_ring_integer_exact(gpu, dtype):
    # integer operands: partials of every split are exact, so the split sum is
    # the exact sum rounded once
    a = randint((16, 4096), dtype, 230, -2, 3)
    b = randint((4096, 14336), dtype, 231, -2, 3)
    got, plan = run(gpu, a, b, (16, 14336), dtype)
    assert plan == "gemm16_skinny_ring_splitk"
    assert np.array_equal(got, _exact_ref(a, b, dtype)), plan


def test_skinny_exact_mode_uses_sequential_kernel(gpu):
    a = randn((16, 1024), torch.float16, 220)
    b = randn((1024, 2048), torch.float16, 221)
    got, plan = run(gpu, a, b, (16, 2048), torch.float16, exact=True)
    assert plan.startswith("gemm_seq_mfma"), plan
    assert_bit_exact(got, oracle_mm(a, b, torch.float16), plan)


# ---------------------------------------------------------------------------
# an operand past the tiled kernels' 2 GiB buffer range runs in row blocks
# ---------------------------------------------------------------------------

def test_operand_past_2gib_runs_in_row_blocks(gpu):
    # A is [2^20, 2048] float16 (4 GiB): three row blocks of 524032, 524032 and 512 rows, each on the ring kernel;
    # integer operands make every summation order exact, so the rows on both sides of each block edge match bit for bit
    dtype = torch.float16
    M, N, K = 1 << 20, 256, 2048
    a = torch.randint(-2, 3, (M, K), generator=gen(90), dtype=torch.int8).to(DEV).to(dtype)
    b = randint((K, N), dtype, 91, -2, 3)
    c = torch.empty((M, N), dtype=dtype, device=DEV)
    gpu.gemm(a, b.to(DEV), c)
    torch.cuda.synchronize()
    assert gpu.gemm_plan(a, b.to(DEV), c) == "gemm16_dma_256x256"
    rows = np.r_[0:2, 524030:524034, 1048062:1048066, M - 2:M]
    ah = a[torch.from_numpy(rows).to(DEV)].cpu()
    ref = oracle_mm(ah, b, dtype)
    assert_bit_exact(decode(to_np(c[torch.from_numpy(rows).to(DEV)].cpu()), dtype), ref, "row blocks past 2 GiB")
    del a, c
    torch.cuda.empty_cache()


def test_calibrate_mfma_reports_a_plausible_rate(gpu):
    # the random-operand MFMA loop: positive, below the dense peak, and more
    # waves per SIMD never slower than one by much; bad arguments are rejected
    rates = {w: gpu.calibrate_mfma(0, w, 4000)[0] for w in (1, 2, 4)}
    for w, tf in rates.items():
        assert 50.0 < tf < 2600.0, (w, tf)
    assert rates[4] > 0.8 * rates[1]
    # the 32x32x16 form and the zero operands run the same flops
    for zeros in (False, True):
        assert 50.0 < gpu.calibrate_mfma(0, 2, 4000, zeros=zeros, mfma32=True)[0] < 2600.0
    with pytest.raises(gpu.TvkError):
        gpu.calibrate_mfma(0, 0, 100)
    tf, ms = gpu.C.c_double(), gpu.C.c_double()
    assert gpu.load().tvk_calibrate_mfma_operands(0, 2, 100, 4, gpu.C.byref(tf), gpu.C.byref(ms)) == gpu.TVK_ERR_INVALID
    with pytest.raises(gpu.TvkError):
        gpu.calibrate_mfma(0, 2, 0)


def test_calibrate_hbm_reports_a_plausible_rate(gpu):
    # the streaming read: positive and below the 8 TB/s HBM peak (windows of
    # 128 MiB, three in rotation, so the 256 MB Infinity Cache cannot hold the
    # next one); bad arguments are rejected
    gbps, ms = gpu.calibrate_hbm(0, 128 << 20, 20)
    assert 1000.0 < gbps < 8000.0 and ms > 0.0, (gbps, ms)
    with pytest.raises(gpu.TvkError):
        gpu.calibrate_hbm(0, 100, 10)
    with pytest.raises(gpu.TvkError):
        gpu.calibrate_hbm(0, 1 << 20, 0)
