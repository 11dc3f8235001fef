"""tvk_binary and tvk_reduce_sum on the GPU through the C ABI.

binary: bit-exact against oracle.binary (every dtype, op and alpha; broadcast
and strided operands; in place). sum: bit-exact on integer-valued inputs,
where every summation order is exact (a dropped, repeated or misplaced term
shows), and on integer dtypes; within a float32 error bound of the exact
float64 sum on random inputs; edge shapes (empty reductions, keepdim, full
reductions, size-1 and expanded dimensions)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from torchvulkan_amd import _abi

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CODE = {torch.float32: orc.F32, torch.float16: orc.F16, torch.bfloat16: orc.BF16, torch.float64: orc.F64,
        torch.int64: orc.I64, torch.int32: orc.I32, torch.int16: orc.I16, torch.int8: orc.I8, torch.uint8: orc.U8}


def np_storage(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype in (torch.float16, torch.bfloat16) else t.numpy()


def values(dtype, shape, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype.is_floating_point:
        return (torch.randn(shape, generator=g) * 4).to(dtype)
    info = torch.iinfo(dtype)
    return torch.randint(max(info.min, -1000), min(info.max, 1000), shape, generator=g).to(dtype)


def check_binary(a, b, out, op, alpha, what):
    _abi.binary(a, b, out, op, alpha)
    torch.cuda.synchronize()
    dt = CODE[out.dtype]
    want = orc.binary(np_storage(a.expand(out.shape)), np_storage(b.expand(out.shape)), dt, op, alpha)
    got = np_storage(out)
    if out.dtype.is_floating_point:
        gf, wf = orc.to_f32(got, dt) if dt != orc.F64 else got, orc.to_f32(want, dt) if dt != orc.F64 else want
        same_nan = np.isnan(gf) == np.isnan(wf)
        assert same_nan.all(), what
        got, want = got[~np.isnan(gf)], want[~np.isnan(wf)]
    bad = np.nonzero(got.reshape(-1) != want.reshape(-1))[0]
    assert bad.size == 0, f"{what}: {bad.size} differ, first {bad[0]}: {got.reshape(-1)[bad[0]]} vs {want.reshape(-1)[bad[0]]}"


@pytest.mark.parametrize("dtype", list(CODE))
def test_binary_all_dtypes(gpu, dtype):
    a = values(dtype, (257, 33), 1).to(DEV)
    b = values(dtype, (257, 33), 2).to(DEV)
    alphas = [1.0, 0.5, -1.25, 3.0] if dtype.is_floating_point else [1, 3, -2]
    for op in (orc.BIN_ADD, orc.BIN_SUB, orc.BIN_MUL):
        for alpha in alphas:
            out = torch.empty_like(a)
            check_binary(a, b, out, op, alpha, f"{dtype} op {op} alpha {alpha}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_binary_broadcast_strided_inplace(gpu, dtype):
    x = values(dtype, (64, 48), 3).to(DEV)
    bias = values(dtype, (48,), 4).to(DEV)
    out = torch.empty_like(x)
    check_binary(x, bias, out, orc.BIN_ADD, 1.0, "row broadcast")
    col = values(dtype, (64, 1), 5).to(DEV)
    check_binary(x.t(), col.t(), torch.empty((48, 64), dtype=dtype, device=DEV), orc.BIN_MUL, 1.0, "transposed operands")
    big = torch.zeros((64, 96), dtype=dtype, device=DEV)
    check_binary(x, bias, big[:, ::2], orc.BIN_SUB, 0.5, "strided out")
    assert (big.cpu()[:, 1::2] == 0).all()
    y = x.clone()
    before = y.cpu()
    _abi.binary(y, bias, y, orc.BIN_ADD, -1.25)
    torch.cuda.synchronize()
    want = orc.binary(np_storage(before), np_storage(bias.expand(64, 48)), CODE[dtype], orc.BIN_ADD, -1.25)
    assert (np_storage(y) == want).all(), "in place"
    dense = values(dtype, (1 << 20) + 3, 6).to(DEV)
    check_binary(dense, dense.flip(0), torch.empty_like(dense), orc.BIN_ADD, 0.5, "dense + tail")


def exact_sum(x: torch.Tensor, dims, keepdim=False) -> torch.Tensor:
    return x.double().sum(dim=dims, keepdim=keepdim)


def reduce_check(x, dims, keepdim=False, out_dtype=None, exact=False):
    got = _abi.reduce_sum(x, dims, keepdim, out_dtype)
    torch.cuda.synchronize()
    xc = x.cpu()
    ref = exact_sum(xc, dims if dims else list(range(x.dim())), keepdim)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    g = got.cpu().double()
    if exact:
        assert torch.equal(g, ref.to(got.dtype).double()), f"dims {dims}: exact sums differ"
        return
    # float32 accumulation: an error bound of the summation tree (depth <= terms/256 + 8 + splits <= 2e3 here)
    n = xc.numel() // max(1, ref.numel())
    l1 = xc.double().abs().sum(dim=dims if dims else list(range(x.dim())), keepdim=keepdim)
    depth = min(n, math.ceil(n / 64) + 8 + 1024)
    tol = 1e-5 * (ref.abs() + 1) + depth * 2.0**-24 * l1
    if got.dtype in (torch.float16, torch.bfloat16):
        tol = tol + ref.abs() * (2.0**-11 if got.dtype == torch.float16 else 2.0**-8)
    assert ((g - ref).abs() <= tol).all(), f"dims {dims}: max err {(g - ref).abs().max().item()}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_sum_integer_valued_is_exact(gpu, dtype):
    g = torch.Generator().manual_seed(7)
    x = torch.randint(-8, 9, (32, 48, 40), generator=g).to(dtype).to(DEV)
    out = torch.float32
    for dims in ([0], [1], [2], [0, 2], [1, 2], [0, 1], [], [0, 1, 2]):
        reduce_check(x, dims, out_dtype=out, exact=True)
        reduce_check(x, dims, keepdim=True, out_dtype=out, exact=True)
    # long reductions split into chunks: still exact on integers (|partial sums| < 2^24)
    y = torch.randint(-3, 4, (1 << 22,), generator=g).to(dtype).to(DEV)
    reduce_check(y, [0], out_dtype=out, exact=True)
    z = torch.randint(-3, 4, (4096, 1024), generator=g).to(dtype).to(DEV)
    reduce_check(z, [0], out_dtype=out, exact=True)
    reduce_check(z, [1], out_dtype=out, exact=True)
    # 32 or more splits: the grouped fold (32 outputs a workgroup, 8 thread
    # groups over the splits), for a column sum and a row sum
    w = torch.randint(-3, 4, (65536, 384), generator=g).to(dtype).to(DEV)
    reduce_check(w, [0], out_dtype=out, exact=True)
    r = torch.randint(-3, 4, (4, 1 << 20), generator=g).to(dtype).to(DEV)
    reduce_check(r, [1], out_dtype=out, exact=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_sum_whole_tensor_paths(gpu, dtype):
    """Whole-tensor sums (a training loss): the 16-byte row kernel over many chunks and the wide fold
    (one workgroup an output), exact on integers and within the tree bound on random data; and the
    element-wise row kernel where the 16-byte one does not apply (a source off 16-byte alignment, a row
    length that is not whole vectors)."""
    g = torch.Generator().manual_seed(17)
    out = torch.float32
    for shape in ((8192, 512), (128, 256, 8, 8), (3, 1 << 21), (16 * 1024 + 8,)):
        xi = torch.randint(-3, 4, shape, generator=g).to(dtype).to(DEV)
        reduce_check(xi, list(range(len(shape))), out_dtype=out, exact=True)
        reduce_check(xi, [len(shape) - 1], out_dtype=out, exact=True)
    xr = values(dtype, (8192, 512), 18).to(DEV)
    reduce_check(xr, [0, 1], out_dtype=out)
    reduce_check(xr, [0, 1])                       # the result in the source dtype
    base = torch.randint(-3, 4, ((1 << 20) + 1,), generator=g).to(dtype).to(DEV)
    reduce_check(base[1:], [0], out_dtype=out, exact=True)           # 2 bytes off alignment
    odd = torch.randint(-3, 4, (5, 100003), generator=g).to(dtype).to(DEV)
    reduce_check(odd, [1], out_dtype=out, exact=True)                # rows of a partial vector
    reduce_check(odd, [0, 1], out_dtype=out, exact=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_sum_short_columns_one_launch(gpu, dtype):
    """Column sums of at most 1024 rows over few outputs (bias gradients): the one-launch kernel with
    row groups and a tree, exact on integers and within the tree bound on random data; one reduced
    dimension made of two merged ones, keepdim, and the result in the source dtype."""
    g = torch.Generator().manual_seed(19)
    out = torch.float32
    for shape, dims in (((256, 4096), [0]), ((1000, 3000), [0]), ((7, 64), [0]), ((3, 256, 40), [0, 1]),
                        ((1024, 8), [0]), ((33, 520), [0])):
        xi = torch.randint(-3, 4, shape, generator=g).to(dtype).to(DEV)
        reduce_check(xi, dims, out_dtype=out, exact=True)
        reduce_check(xi, dims, keepdim=True, out_dtype=out, exact=True)
        xr = values(dtype, shape, 20).to(DEV)
        reduce_check(xr, dims, out_dtype=out)
        reduce_check(xr, dims)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
def test_sum_random_within_bound(gpu, dtype):
    x = values(dtype, (128, 64, 16, 16), 8).to(DEV)
    for dims in ([0, 2, 3], [0], [3], [1, 3], []):
        reduce_check(x, dims)
    y = values(dtype, (8192, 1536), 9).to(DEV)   # the bias gradient of the transformer down projection
    reduce_check(y, [0])


def test_sum_integer_dtypes_and_bool(gpu):
    x = values(torch.int32, (300, 77), 10).to(DEV)
    reduce_check(x, [0], out_dtype=torch.int64, exact=True)
    reduce_check(x, [1], out_dtype=torch.int64, exact=True)
    b = (values(torch.float32, (1000,), 11) > 0).to(DEV)
    got = _abi.reduce_sum(b, [0], out_dtype=torch.int64)
    assert got.item() == int(b.cpu().sum())
    h = values(torch.float16, (500, 30), 12).to(DEV)
    reduce_check(h, [0], out_dtype=torch.float32)


def test_sum_edges(gpu):
    e = torch.empty((0, 5), device=DEV)
    got = _abi.reduce_sum(e, [0])
    torch.cuda.synchronize()
    assert got.shape == (5,) and (got.cpu() == 0).all()
    one = torch.tensor([2.5], device=DEV)
    assert _abi.reduce_sum(one, [0]).item() == 2.5
    x = values(torch.float32, (1, 7, 1), 13).to(DEV)
    reduce_check(x, [1])
    reduce_check(x, [0, 2], keepdim=True, exact=False)
    s = torch.tensor(3.0, device=DEV)
    assert _abi.reduce_sum(s, []).item() == 3.0
    ex = torch.arange(6.0, device=DEV).view(1, 6).expand(1000, 6)
    reduce_check(ex, [0], exact=True)
