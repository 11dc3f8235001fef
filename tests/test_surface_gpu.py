"""The rest of the reference's operator surface on the vulkan device, each run
under TORCHVULKAN_STRICT=1 (a CPU fallback would raise) and checked against
the oracle: mm.dtype / mm.dtype_out, addbmm.out / addbmm_, addmv (+ .out,
addmv_, and torch.mv / matmul(matrix, vector) through it), the legacy
convolution aliases, im2col / col2im (F.unfold / F.fold), and torch.Event on
the device's stream.

Tolerances are the north_star's (tests/gemm_cases.py): float32 1e-5*(|ref|+1),
float16/bfloat16 5e-3*(|ref|+1); paths that run the float32 sequential-order
kernel are held to the oracle's bits."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.gemm_cases import ORC_DT, assert_bit_exact, assert_close, decode, gen, oracle_mm, randint, randn, to_np

pytestmark = pytest.mark.gpu

V = "vulkan"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(scope="module")
def tv(gpu):
    import torchvulkan_amd

    assert torchvulkan_amd.is_available()
    return torchvulkan_amd


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


def host(t):
    return t.detach().to("cpu")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mm_dtype_float32_output(tv, strict, dtype):
    a, b = randn((257, 130), dtype, 1), randn((130, 190), dtype, 2)
    got = torch.ops.aten.mm.dtype(a.to(V), b.to(V), torch.float32)
    assert got.dtype == torch.float32 and got.shape == (257, 190)
    # the float32 product of the widened operands, in the sequential-order kernel: the oracle's bits
    assert_bit_exact(host(got).numpy(), oracle_mm(a.float(), b.float(), torch.float32), "mm.dtype")
    out = torch.empty((0,), dtype=torch.float32, device=V)
    torch.ops.aten.mm.dtype_out(a.to(V), b.to(V), torch.float32, out=out)
    assert out.shape == (257, 190)
    assert_bit_exact(host(out).numpy(), host(got).numpy(), "mm.dtype_out")
    same = torch.ops.aten.mm.dtype(a.to(V), b.to(V), dtype)
    assert same.dtype == dtype
    assert_close(decode(to_np(host(same)), dtype), oracle_mm(a, b, dtype), dtype, "mm.dtype same")


def test_mm_dtype_rejects_other_outputs(tv):
    a = torch.zeros((4, 4), device=V)
    with pytest.raises(RuntimeError, match="out_dtype must be the same as input dtype or fp32 for fp16/bf16 inputs"):
        torch.ops.aten.mm.dtype(a, a, torch.float16)


@pytest.mark.parametrize("dtype", DTYPES)
def test_addbmm_out_and_inplace(tv, strict, dtype):
    b1, b2 = randn((6, 40, 24), dtype, 3), randn((6, 24, 33), dtype, 4)
    inp = randn((40, 33), dtype, 5)
    # addbmm is one product over the batch-concatenated K (the reference folds it the same way)
    a2 = b1.permute(1, 0, 2).reshape(40, 6 * 24)
    bb = b2.reshape(6 * 24, 33)
    ref = oracle_mm(a2, bb, dtype, bias=inp, alpha=0.5, beta=2.0)
    out = torch.empty((0,), dtype=dtype, device=V)
    torch.addbmm(inp.to(V), b1.to(V), b2.to(V), beta=2.0, alpha=0.5, out=out)
    assert out.shape == (40, 33)
    assert_close(decode(to_np(host(out)), dtype), ref, dtype, "addbmm.out")
    x = inp.to(V)
    ptr = x.data_ptr()
    x.addbmm_(b1.to(V), b2.to(V), beta=2.0, alpha=0.5)
    assert x.data_ptr() == ptr
    assert_close(decode(to_np(host(x)), dtype), ref, dtype, "addbmm_")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mk", [(4096, 4096), (1000, 777), (64, 3000), (5, 0)])
def test_addmv_family(tv, strict, dtype, mk):
    M, K = mk
    mat, vec, inp = randn((M, K), dtype, 6), randn((K,), dtype, 7), randn((M,), dtype, 8)
    # out^T = vec^T . mat^T: the oracle's one-row product
    ref = oracle_mm(vec.reshape(1, K), mat.t(), dtype, bias=inp.reshape(1, M), alpha=1.5, beta=0.5).reshape(M)
    got = torch.addmv(inp.to(V), mat.to(V), vec.to(V), beta=0.5, alpha=1.5)
    assert got.shape == (M,)
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "addmv")
    out = torch.empty((0,), dtype=dtype, device=V)
    torch.addmv(inp.to(V), mat.to(V), vec.to(V), beta=0.5, alpha=1.5, out=out)
    assert_close(decode(to_np(host(out)), dtype), ref, dtype, "addmv.out")
    x = inp.to(V)
    x.addmv_(mat.to(V), vec.to(V), beta=0.5, alpha=1.5)
    assert_close(decode(to_np(host(x)), dtype), ref, dtype, "addmv_")
    plain = oracle_mm(vec.reshape(1, K), mat.t(), dtype).reshape(M)
    assert_close(decode(to_np(host(torch.mv(mat.to(V), vec.to(V)))), dtype), plain, dtype, "mv")
    assert_close(decode(to_np(host(torch.matmul(mat.to(V), vec.to(V)))), dtype), plain, dtype, "matmul(matrix, vector)")
    # a transposed matrix view is read in place
    matt = randn((K, M), dtype, 9)
    ref_t = oracle_mm(vec.reshape(1, K), matt, dtype).reshape(M)
    assert_close(decode(to_np(host(torch.mv(matt.to(V).t(), vec.to(V)))), dtype), ref_t, dtype, "mv(mat.t())")


def test_addmv_scalar_self_and_errors(tv, strict):
    mat, vec = randn((70, 90), torch.float32, 10), randn((90,), torch.float32, 11)
    s = torch.tensor(2.0)
    got = torch.addmv(s.to(V), mat.to(V), vec.to(V))
    ref = oracle_mm(vec.reshape(1, 90), mat.t(), torch.float32, bias=s.expand(1, 70).contiguous(), beta=1.0).reshape(70)
    assert_bit_exact(host(got).numpy(), ref, "addmv with a 0-d self")
    cases = [
        lambda d: torch.addmv(torch.zeros(3, device=d), torch.zeros(3, 4, device=d), torch.zeros(5, device=d)),
        lambda d: torch.addmv(torch.zeros(3, device=d), torch.zeros(3, 4, 1, device=d), torch.zeros(4, device=d)),
        lambda d: torch.addmv(torch.zeros(2, device=d), torch.zeros(3, 4, device=d), torch.zeros(4, device=d)),
        lambda d: torch.addmv(torch.zeros(3, device=d), torch.zeros(3, 4, device=d), torch.zeros(4, dtype=torch.float64, device=d)),
    ]
    for case in cases:
        msgs = []
        for dev in ("cpu", V):
            with pytest.raises(RuntimeError) as e:
                case(dev)
            msgs.append(str(e.value).splitlines()[0])
        assert msgs[0] == msgs[1]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_legacy_conv_aliases(tv, strict, dtype):
    od = ORC_DT[dtype]
    x = randn((3, 8, 15, 13), dtype, 20)
    w = randn((12, 8, 3, 3), dtype, 21, std=0.2)
    b = randn((12,), dtype, 22)
    xv, wv, bv = x.to(V), w.to(V), b.to(V)

    got = torch.ops.aten._slow_conv2d_forward(xv, wv, [3, 3], bv, [2, 1], [1, 0])
    ref = decode(orc.conv2d(to_np(x), to_np(w), od, bias=to_np(b), stride=(2, 1), padding=(1, 0)), dtype)
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "_slow_conv2d_forward")
    out = torch.empty((0,), dtype=dtype, device=V)
    torch.ops.aten._slow_conv2d_forward.output(xv, wv, [3, 3], bv, [2, 1], [1, 0], output=out)
    assert_close(decode(to_np(host(out)), dtype), ref, dtype, "_slow_conv2d_forward.output")

    got = torch.ops.aten.slow_conv_dilated2d(xv, wv, [3, 3], bv, [1, 1], [2, 2], [2, 2])
    ref = decode(orc.conv2d(to_np(x), to_np(w), od, bias=to_np(b), padding=(2, 2), dilation=(2, 2)), dtype)
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "slow_conv_dilated2d")

    wd = randn((8, 1, 3, 3), dtype, 23, std=0.3)
    got = torch.ops.aten._conv_depthwise2d(xv, wd.to(V), [3, 3], None, [1, 1], [1, 1], [1, 1])
    ref = decode(orc.conv2d(to_np(x), to_np(wd), od, padding=(1, 1), groups=8), dtype)
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "_conv_depthwise2d")

    wt = randn((8, 5, 3, 3), dtype, 24, std=0.3)
    got = torch.ops.aten.slow_conv_transpose2d(xv, wt.to(V), [3, 3], None, [2, 2], [1, 1], [1, 1])
    # a transposed convolution is the input gradient of the forward one
    h = (15 - 1) * 2 - 2 + 3 + 1
    wdt = (13 - 1) * 2 - 2 + 3 + 1
    ref = decode(orc.conv2d_dgrad(to_np(x), to_np(wt), (3, 5, h, wdt), od, (2, 2), (1, 1)), dtype)
    assert got.shape == (3, 5, h, wdt)
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "slow_conv_transpose2d")

    with pytest.raises(RuntimeError, match="must match weight spatial dimensions"):
        torch.ops.aten._slow_conv2d_forward(xv, wv, [2, 3], bv, [1, 1], [0, 0])


UNFOLD_CASES = [
    # (n, c, h, w), kernel, dilation, padding, stride
    ((2, 3, 9, 11), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 4, 10, 7), (2, 3), (2, 1), (0, 2), (2, 3)),
    ((3, 2, 5, 5), (1, 1), (1, 1), (0, 0), (2, 2)),
]


@pytest.mark.parametrize("case", range(len(UNFOLD_CASES)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.int32])
def test_im2col_col2im(tv, strict, case, dtype):
    shape, k, d, p, s = UNFOLD_CASES[case]
    # integer values: the column sums of col2im are exact in every dtype, so the device must match the float64
    # CPU result bit for bit (the CPU has no integer im2col, so int32 is checked against it too)
    x = randint(shape, dtype, 30 + case)
    cols = F.unfold(x.to(V), k, dilation=d, padding=p, stride=s)
    want = F.unfold(x.double(), k, dilation=d, padding=p, stride=s).to(dtype)
    assert cols.shape == want.shape and cols.is_contiguous()
    assert torch.equal(host(cols), want)
    back = F.fold(cols, shape[2:], k, dilation=d, padding=p, stride=s)
    want_back = F.fold(want.double(), shape[2:], k, dilation=d, padding=p, stride=s).to(dtype)
    assert torch.equal(host(back), want_back)
    # unbatched forms
    assert torch.equal(host(torch.ops.aten.im2col(x[0].to(V), k, d, p, s)), want[0])
    assert torch.equal(host(torch.ops.aten.col2im(want[0].to(V), shape[2:], k, d, p, s)), want_back[0])


def test_im2col_errors_match_cpu(tv):
    cases = [
        lambda dv: torch.ops.aten.im2col(torch.zeros(2, 3, 5, 6, device=dv), [0, 3], [1, 1], [1, 1], [1, 1]),
        lambda dv: torch.ops.aten.im2col(torch.zeros(2, 3, 5, 6, device=dv), [9, 3], [1, 1], [1, 1], [1, 1]),
        lambda dv: torch.ops.aten.col2im(torch.zeros(2, 27, 30, device=dv), [5, 7], [3, 3], [1, 1], [1, 1], [1, 1]),
        lambda dv: torch.ops.aten.col2im(torch.zeros(2, 26, 30, device=dv), [5, 6], [3, 3], [1, 1], [1, 1], [1, 1]),
    ]
    for case in cases:
        msgs = []
        for dev in ("cpu", V):
            with pytest.raises(RuntimeError) as e:
                case(dev)
            msgs.append(str(e.value).splitlines()[0])
        assert msgs[0] == msgs[1]


def test_events_on_the_device_stream(tv):
    a = randn((2048, 2048), torch.float16, 40).to(V)
    start = torch.Event(device=V, enable_timing=True)
    end = torch.Event(device=V, enable_timing=True)
    start.record()
    for _ in range(20):
        c = torch.mm(a, a)
    end.record()
    end.synchronize()
    assert end.query()
    ms = start.elapsed_time(end)
    # 20 products of 17.2 GFLOP: positive, and far below a second on the GPU clock
    assert 0.0 < ms < 1000.0
    # a plain event (no timing) still orders work and reports completion
    e = torch.Event(device=V)
    e.record()
    e.wait()
    e.synchronize()
    assert e.query()
    tv.synchronize()
    assert c.shape == (2048, 2048)
