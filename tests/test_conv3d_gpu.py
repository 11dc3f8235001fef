"""Three (and one) spatial dimensions on the GPU: tvk_conv_fwd / dgrad / wgrad
through the C ABI against the 3-D oracle, and conv3d / conv_transpose3d /
the 3-D legacy aliases through the vulkan device under strict mode (any CPU
fallback raises).

The reference takes 1-3 spatial dimensions on its device
(src/api/ops/conv.cpp:295-311, geometry block :313-343, gathers
src/shaders/helpers/conv.slang:93-117). Bars (tests/gemm_cases.py):
float32, and every dtype in exact mode, bit-identical to the oracle's k order
(c, kd, kh, kw) for forward and grad input; float16/bfloat16 within
5e-3 (|ref| + 1); float32 grad weight within the K-term reduction allowance
the 2-D tests state; float64 products against torch's CPU float64 result.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.gemm_cases import ORC_DT, assert_bit_exact, assert_close, decode, gen, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"
V = "vulkan"


def _x(shape, dtype, seed):
    return torch.randn(shape, generator=gen(seed)).to(dtype)


def _w(shape, dtype, seed):
    fan_in = int(np.prod(shape[1:]))
    return (torch.randn(shape, generator=gen(seed)) * np.sqrt(2.0 / fan_in)).to(dtype)


def _t3(v):
    return (v, v, v) if isinstance(v, int) else tuple(v)


def _assert_wgrad3_f32(got, ref64, x, dy, w_shape, s, p, d, groups):
    """float32 grad weight against the float64 sum: 1e-5 (|ref| + 1) plus 4 float32 ulps of R sqrt(K), R^2 the
    exact sum of squared terms (a K-term float32 reduction's spread; a dropped or misplaced term exceeds it)."""
    xs = to_np(x).astype(np.float32)
    ys = to_np(dy).astype(np.float32)
    r2 = orc.conv3d_wgrad(xs * xs, ys * ys, w_shape, orc.F32, s, p, d, groups, acc64=True).astype(np.float64)
    K = dy.shape[0] * int(np.prod(dy.shape[2:]))
    tol = 1e-5 * (np.abs(ref64) + 1) + 4 * 2.0 ** -24 * np.sqrt(K) * np.sqrt(r2)
    worst = float((np.abs(got.astype(np.float64) - ref64) / tol).max())
    assert worst <= 1.0, f"wgrad: max error is {worst:.3f}x the allowance"


CASES3 = [
    # n, cin, cout, kernel, stride, padding, dilation, groups, spatial (D, H, W)
    dict(n=2, cin=8, cout=16, k=3, s=1, p=1, d=1, g=1, sp=(6, 8, 8)),
    dict(n=2, cin=16, cout=32, k=3, s=2, p=1, d=1, g=1, sp=(8, 10, 9)),
    dict(n=1, cin=6, cout=9, k=(3, 1, 3), s=(1, 2, 2), p=(1, 0, 2), d=(2, 1, 1), g=3, sp=(7, 6, 7)),
    dict(n=3, cin=12, cout=24, k=1, s=(1, 2, 2), p=0, d=1, g=1, sp=(4, 6, 6)),
    dict(n=2, cin=8, cout=8, k=3, s=1, p=1, d=(1, 2, 1), g=8, sp=(5, 7, 6)),   # depthwise
    dict(n=1, cin=70, cout=140, k=(2, 3, 3), s=(2, 1, 1), p=(0, 1, 1), d=1, g=1, sp=(5, 9, 9)),   # M > 128
]


def _run3(abi, dtype, c, seed, exact=False):
    k, s, p, d = _t3(c["k"]), _t3(c["s"]), _t3(c["p"]), _t3(c["d"])
    x = _x((c["n"], c["cin"]) + c["sp"], dtype, seed)
    w = _w((c["cout"], c["cin"] // c["g"]) + k, dtype, seed + 1)
    bias = _x((c["cout"],), dtype, seed + 2)
    y = abi.conv_fwd(x.to(DEV), w.to(DEV), bias.to(DEV), s, p, d, c["g"], exact=exact)
    dy = _x(tuple(y.shape), dtype, seed + 3)
    gx = abi.conv_dgrad(dy.to(DEV), w.to(DEV), x.shape, s, p, d, c["g"], exact=exact)
    gw = abi.conv_wgrad(x.to(DEV), dy.to(DEV), w.shape, s, p, d, c["g"], exact=exact)
    torch.cuda.synchronize()
    return x, w, bias, dy, y, gx, gw, (k, s, p, d)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("case", CASES3, ids=[f"case{i}" for i in range(len(CASES3))])
def test_conv3d_abi_all_directions(gpu, dtype, case):
    x, w, bias, dy, y, gx, gw, (k, s, p, d) = _run3(gpu, dtype, case, 40)
    od, g = ORC_DT[dtype], case["g"]
    ref_y = decode(orc.conv3d(to_np(x), to_np(w), od, bias=to_np(bias), stride=s, padding=p, dilation=d, groups=g), dtype)
    ref_gx = decode(orc.conv3d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, s, p, d, g), dtype)
    ref_gw = decode(orc.conv3d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, s, p, d, g, acc64=True), dtype)
    got_y, got_gx, got_gw = decode(to_np(y), dtype), decode(to_np(gx), dtype), decode(to_np(gw), dtype)
    assert got_y.shape == ref_y.shape
    if dtype == torch.float32:
        assert_bit_exact(got_y, ref_y, "conv3d fwd")
        assert_bit_exact(got_gx, ref_gx, "conv3d dgrad")
        _assert_wgrad3_f32(got_gw, ref_gw, x, dy, tuple(w.shape), s, p, d, g)
    else:
        assert_close(got_y, ref_y, dtype, "conv3d fwd")
        assert_close(got_gx, ref_gx, dtype, "conv3d dgrad")
        assert_close(got_gw, ref_gw, dtype, "conv3d wgrad")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_conv3d_exact_mode_bit_identical(gpu, dtype):
    c = CASES3[1]
    x, w, bias, dy, y, gx, gw, (k, s, p, d) = _run3(gpu, dtype, c, 50, exact=True)
    od = ORC_DT[dtype]
    assert_bit_exact(decode(to_np(y), dtype), decode(orc.conv3d(to_np(x), to_np(w), od, bias=to_np(bias), stride=s,
                                                                 padding=p, dilation=d), dtype), "exact fwd")
    assert_bit_exact(decode(to_np(gx), dtype), decode(orc.conv3d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, s, p, d),
                                                       dtype), "exact dgrad")


def test_conv1d_abi(gpu):
    """One spatial dimension runs the 2-D kernels with a height of 1."""
    dtype = torch.float16
    x = _x((4, 32, 100), dtype, 60)
    w = _w((48, 32, 5), dtype, 61)
    y = gpu.conv_fwd(x.to(DEV), w.to(DEV), None, 2, 2, 1, 1)
    dy = _x(tuple(y.shape), dtype, 62)
    gx = gpu.conv_dgrad(dy.to(DEV), w.to(DEV), x.shape, 2, 2, 1, 1)
    gw = gpu.conv_wgrad(x.to(DEV), dy.to(DEV), w.shape, 2, 2, 1, 1)
    torch.cuda.synchronize()
    od = ORC_DT[dtype]
    x4, w4, dy4 = x.unsqueeze(2), w.unsqueeze(2), dy.unsqueeze(2)
    ref_y = decode(orc.conv2d(to_np(x4), to_np(w4), od, stride=(1, 2), padding=(0, 2)), dtype)[:, :, 0]
    ref_gx = decode(orc.conv2d_dgrad(to_np(dy4), to_np(w4), tuple(x4.shape), od, (1, 2), (0, 2), (1, 1), 1), dtype)[:, :, 0]
    ref_gw = decode(orc.conv2d_wgrad(to_np(x4), to_np(dy4), tuple(w4.shape), od, (1, 2), (0, 2), (1, 1), 1), dtype)[:, :, 0]
    assert_close(decode(to_np(y), dtype), ref_y, dtype, "conv1d fwd")
    assert_close(decode(to_np(gx), dtype), ref_gx, dtype, "conv1d dgrad")
    assert_close(decode(to_np(gw), dtype), ref_gw, dtype, "conv1d wgrad")


def test_convnd_rejects_bad_geometry(gpu):
    d = gpu.make_convnd_desc((1, 4, 5, 5, 5), (4, 4, 3, 3, 3), torch.float16)
    d.out_size[0] = 7
    assert gpu.load().tvk_conv_fwd(gpu.C.byref(d)) == gpu.TVK_ERR_INVALID


# ---------------------------------------------------------------------------
# the vulkan device
# ---------------------------------------------------------------------------

@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
def test_conv3d_autograd_on_vulkan(gpu, strict, dtype):
    import torchvulkan_amd  # noqa: F401

    n, cin, cout = 2, 16, 32
    x = _x((n, cin, 6, 10, 10), dtype, 70)
    w = _w((cout, cin, 3, 3, 3), dtype, 71)
    b = _x((cout,), dtype, 72)
    xv, wv, bv = (t.to(V).requires_grad_() for t in (x, w, b))
    y = F.conv3d(xv, wv, bv, stride=(1, 2, 2), padding=1)
    dy = _x(tuple(y.shape), dtype, 73)
    y.backward(dy.to(V))
    od = ORC_DT[dtype]
    s, p, d = (1, 2, 2), (1, 1, 1), (1, 1, 1)
    ref_y = decode(orc.conv3d(to_np(x), to_np(w), od, bias=to_np(b), stride=s, padding=p), dtype)
    ref_gx = decode(orc.conv3d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, s, p, d), dtype)
    ref_gw = decode(orc.conv3d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, s, p, d, acc64=True), dtype)
    got_y = decode(to_np(y.detach().cpu()), dtype)
    got_gx = decode(to_np(xv.grad.cpu()), dtype)
    got_gw = decode(to_np(wv.grad.cpu()), dtype)
    if dtype == torch.float32:
        assert_bit_exact(got_y, ref_y, "conv3d fwd")
        assert_bit_exact(got_gx, ref_gx, "conv3d dgrad")
        _assert_wgrad3_f32(got_gw, ref_gw, x, dy, tuple(w.shape), s, p, d, 1)
    else:
        assert_close(got_y, ref_y, dtype, "conv3d fwd")
        assert_close(got_gx, ref_gx, dtype, "conv3d dgrad")
        assert_close(got_gw, ref_gw, dtype, "conv3d wgrad")
    db = dy.double().sum((0, 2, 3, 4)).numpy()
    assert_close(bv.grad.cpu().float().numpy(), db, dtype, "conv3d grad bias vs float64 sum")


def test_conv_transpose3d_on_vulkan(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    dtype = torch.float16
    x = _x((2, 24, 4, 5, 6), dtype, 80)
    w = _w((24, 12, 3, 3, 3), dtype, 81)   # [c_in, c_out, k...]
    b = _x((12,), dtype, 82)
    xv, wv = x.to(V).requires_grad_(), w.to(V).requires_grad_()
    y = F.conv_transpose3d(xv, wv, b.to(V), stride=2, padding=1, output_padding=1)
    dy = _x(tuple(y.shape), dtype, 83)
    y.backward(dy.to(V))
    ref = F.conv_transpose3d(x.double(), w.double(), b.double(), stride=2, padding=1, output_padding=1)
    assert tuple(y.shape) == tuple(ref.shape)
    assert_close(y.detach().cpu().float().numpy(), ref.numpy(), dtype, "conv_transpose3d vs float64")
    # the input gradient of a transposed convolution is the forward convolution of dy
    od = ORC_DT[dtype]
    ref_gx = decode(orc.conv3d(to_np(dy), to_np(w), od, stride=2, padding=1), dtype)
    assert_close(xv.grad.cpu().float().numpy(), ref_gx, dtype, "conv_transpose3d grad input vs oracle")
    xd, wd = x.double().requires_grad_(), w.double().requires_grad_()
    F.conv_transpose3d(xd, wd, None, stride=2, padding=1, output_padding=1).backward(dy.double())
    assert_close(wv.grad.cpu().float().numpy(), wd.grad.numpy(), dtype, "conv_transpose3d grad weight vs float64")


def test_legacy_3d_aliases_on_vulkan(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    dtype = torch.float16
    x = _x((2, 8, 5, 6, 7), dtype, 90)
    w = _w((8, 8, 3, 3, 3), dtype, 91)
    wd = _w((8, 1, 3, 3, 3), dtype, 92)
    b = _x((8,), dtype, 93)
    xv, wv, wdv, bv = x.to(V), w.to(V), wd.to(V), b.to(V)
    xd, wdd, wddw, bd = x.double(), w.double(), wd.double(), b.double()
    got = torch.ops.aten.slow_conv3d_forward(xv, wv, [3, 3, 3], bv, [1, 1, 1], [1, 1, 1])
    assert_close(got.cpu().float().numpy(), F.conv3d(xd, wdd, bd, 1, 1).numpy(), dtype, "slow_conv3d_forward")
    got = torch.ops.aten.conv_depthwise3d(xv, wdv, [3, 3, 3], bv, [1, 2, 2], [1, 1, 1], [1, 1, 1])
    assert_close(got.cpu().float().numpy(), F.conv3d(xd, wddw, bd, (1, 2, 2), 1, 1, 8).numpy(), dtype, "conv_depthwise3d")
    got = torch.ops.aten.slow_conv_dilated3d(xv, wv, [3, 3, 3], bv, [1, 1, 1], [2, 2, 2], [2, 1, 2])
    assert_close(got.cpu().float().numpy(), F.conv3d(xd, wdd, bd, 1, 2, (2, 1, 2)).numpy(), dtype, "slow_conv_dilated3d")
    got = torch.ops.aten.slow_conv_transpose3d(xv, wv, [3, 3, 3], bv, [2, 2, 2], [1, 1, 1], [1, 0, 1], [1, 1, 1])
    ref = F.conv_transpose3d(xd, wdd, bd, 2, 1, (1, 0, 1))
    assert_close(got.cpu().float().numpy(), ref.numpy(), dtype, "slow_conv_transpose3d")


def test_conv3d_float64_on_vulkan(gpu, strict):
    """float64 runs as device im2col plus the float64 GEMM (fma in k order), forward, transposed and backward."""
    import torchvulkan_amd  # noqa: F401

    x = torch.randn((2, 4, 5, 6, 5), generator=gen(100), dtype=torch.float64)
    w = torch.randn((6, 2, 3, 2, 3), generator=gen(101), dtype=torch.float64)
    b = torch.randn((6,), generator=gen(102), dtype=torch.float64)
    xv, wv, bv = (t.to(V).requires_grad_() for t in (x, w, b))
    y = F.conv3d(xv, wv, bv, stride=(2, 1, 1), padding=(1, 0, 1), groups=2)
    dy = torch.randn(tuple(y.shape), generator=gen(103), dtype=torch.float64)
    y.backward(dy.to(V))
    xr, wr, br = (t.clone().requires_grad_() for t in (x, w, b))
    yr = F.conv3d(xr, wr, br, stride=(2, 1, 1), padding=(1, 0, 1), groups=2)
    yr.backward(dy)
    for got, ref, what in ((y.detach(), yr.detach(), "fwd"), (xv.grad, xr.grad, "dgrad"), (wv.grad, wr.grad, "wgrad"),
                           (bv.grad, br.grad, "bias")):
        err = (got.cpu() - ref).abs().max().item()
        assert err <= 1e-12 * (ref.abs().max().item() + 1), f"float64 conv3d {what}: {err}"
    wt = torch.randn((4, 3, 3, 2, 3), generator=gen(104), dtype=torch.float64)   # [c_in, c_out, k...]
    t = F.conv_transpose3d(x.to(V), wt.to(V), b[:3].to(V), stride=2, padding=1)
    tr = F.conv_transpose3d(x, wt, b[:3], stride=2, padding=1)
    assert (t.cpu() - tr).abs().max().item() <= 1e-12 * (tr.abs().max().item() + 1)


def test_conv3d_integer_on_vulkan(gpu, strict):
    """Integer convolutions accumulate in their own type (wraparound); small values keep every sum exact, so the
    float64 convolution of the same values is the exact answer."""
    import torchvulkan_amd  # noqa: F401

    x = torch.randint(-3, 4, (2, 3, 4, 5, 6), generator=gen(110))
    w = torch.randint(-3, 4, (4, 3, 2, 3, 3), generator=gen(111))
    for dt in (torch.int32, torch.int64):
        got = F.conv3d(x.to(dt).to(V), w.to(dt).to(V), stride=(1, 2, 1), padding=(1, 1, 0))
        ref = F.conv3d(x.double(), w.double(), stride=(1, 2, 1), padding=(1, 1, 0))
        assert got.dtype == dt
        assert torch.equal(got.cpu().double(), ref)
