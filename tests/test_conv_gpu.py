"""Convolution parity on the GPU through the C ABI (tvk_conv2d_fwd / dgrad /
wgrad) against the oracle.

Cases: the C4 ResNet layers (batch 128, 32x32, NCHW; 3x3 3->64, 64->64,
64->128 s2, 128->256 s2, 1x1 downsamples, padding 1 for 3x3), forward,
grad-input and grad-weight, in float16 and float32, with Kaiming-normal
weights and N(0,1) activations; geometry edge cases (dilation, groups,
rectangular kernels, odd sizes); exact mode; and the reference's Winograd
path for the 3x3 stride-1 layer. Tolerances: tests/gemm_cases.py.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gemm_cases import ORC_DT, assert_bit_exact, assert_close, decode, gen, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _x(shape, dtype, seed):
    return torch.randn(shape, generator=gen(seed)).to(dtype)


def _w(shape, dtype, seed):
    fan_in = shape[1] * shape[2] * shape[3]
    return (torch.randn(shape, generator=gen(seed)) * np.sqrt(2.0 / fan_in)).to(dtype)


C4 = [
    # name, cin, cout, k, stride, pad, spatial
    ("stem_3_64", 3, 64, 3, 1, 1, 32),
    ("3x3_64_64", 64, 64, 3, 1, 1, 32),
    ("3x3_64_128_s2", 64, 128, 3, 2, 1, 32),
    ("3x3_128_256_s2", 128, 256, 3, 2, 1, 16),
    ("1x1_64_128_s2", 64, 128, 1, 2, 0, 32),
    ("1x1_128_256_s2", 128, 256, 1, 2, 0, 16),
]


def _check_all_directions(abi, dtype, n, cin, cout, k, s, p, hw, groups=1, dil=1, seed=0, exact=False, sample_n=None):
    kh, kw = (k, k) if isinstance(k, int) else k
    hh, ww = (hw, hw) if isinstance(hw, int) else hw
    x = _x((n, cin, hh, ww), dtype, seed)
    w = _w((cout, cin // groups, kh, kw), dtype, seed + 1)
    bias = _x((cout,), dtype, seed + 2)
    dx_, dw_, dy_ = x.to(DEV), w.to(DEV), None
    y = abi.conv2d_fwd(dx_, dw_, bias.to(DEV), s, p, dil, groups, exact=exact)
    dy = _x(tuple(y.shape), dtype, seed + 3)
    dy_ = dy.to(DEV)
    gx = abi.conv2d_dgrad(dy_, dw_, x.shape, s, p, dil, groups, exact=exact)
    gw = abi.conv2d_wgrad(dx_, dy_, w.shape, s, p, dil, groups, exact=exact)
    torch.cuda.synchronize()
    od = ORC_DT[dtype]
    # forward / grad-input: the oracle checks a sample of the batch (every output of those samples)
    ns = n if sample_n is None else sample_n
    ref_y = decode(orc.conv2d(to_np(x[:ns]), to_np(w), od, bias=to_np(bias), stride=(s, s), padding=(p, p),
                              dilation=(dil, dil), groups=groups), dtype)
    ref_gx = decode(orc.conv2d_dgrad(to_np(dy[:ns]), to_np(w), (ns,) + tuple(x.shape[1:]), od, (s, s), (p, p),
                                     (dil, dil), groups), dtype)
    ref_gw = decode(orc.conv2d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, (s, s), (p, p), (dil, dil), groups,
                                     acc64=not exact), dtype)
    got_y = decode(to_np(y[:ns]), dtype)
    got_gx = decode(to_np(gx[:ns]), dtype)
    got_gw = decode(to_np(gw), dtype)
    if exact or dtype == torch.float32:
        assert_bit_exact(got_y, ref_y, "fwd")
        assert_bit_exact(got_gx, ref_gx, "dgrad")
    assert_close(got_y, ref_y, dtype, "fwd")
    assert_close(got_gx, ref_gx, dtype, "dgrad")
    if dtype == torch.float32:
        _assert_wgrad_f32(got_gw, ref_gw, x, dy, tuple(w.shape), (s, s), (p, p), (dil, dil), groups)
    else:
        assert_close(got_gw, ref_gw, dtype, "wgrad")


def _assert_wgrad_f32(got, ref64, x, dy, w_shape, s, p, d, groups):
    """float32 grad-weight against the float64 sum.

    dW is a K = n*Ho*Wo term reduction whose partial sums reach
    R = sqrt(sum of squared terms) while the result can be near zero, so no
    float32 summation (the reference's split float32 partials + at::sum
    included) stays within 1e-5*(|ref|+1) of the exact value there. Allowed:
    that bound plus 4 float32 ulps of R*sqrt(K), the spread of a K-term
    float32 reduction; a dropped or misplaced term (|t| ~ 1) exceeds it."""
    xs = to_np(x).astype(np.float32)
    ys = to_np(dy).astype(np.float32)
    r2 = orc.conv2d_wgrad(xs * xs, ys * ys, w_shape, orc.F32, s, p, d, groups, acc64=True).astype(np.float64)
    K = dy.shape[0] * dy.shape[2] * dy.shape[3]
    tol = 1e-5 * (np.abs(ref64) + 1) + 4 * 2.0 ** -24 * np.sqrt(K) * np.sqrt(r2)
    err = np.abs(got.astype(np.float64) - ref64)
    worst = float((err / tol).max())
    assert worst <= 1.0, f"wgrad: max error is {worst:.3f}x the allowance"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("layer", C4, ids=[c[0] for c in C4])
def test_c4_resnet_layers(gpu, dtype, layer):
    _, cin, cout, k, s, p, hw = layer
    _check_all_directions(gpu, dtype, 128, cin, cout, k, s, p, hw, seed=10, sample_n=8)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", [
    dict(n=2, cin=4, cout=6, k=3, s=1, p=1, hw=9, groups=2, dil=2),
    dict(n=3, cin=5, cout=7, k=(5, 3), s=2, p=2, hw=11),
    dict(n=1, cin=16, cout=8, k=1, s=1, p=0, hw=7),
    dict(n=2, cin=8, cout=4, k=3, s=3, p=0, hw=10),
    dict(n=4, cin=12, cout=12, k=3, s=1, p=1, hw=5, groups=3),
])
def test_geometry_edge_cases(gpu, dtype, case):
    case = dict(case)
    _check_all_directions(gpu, dtype, case.pop("n"), case.pop("cin"), case.pop("cout"), case.pop("k"),
                          case.pop("s"), case.pop("p"), case.pop("hw"), seed=20, **case)


# channels-last ring kernels (channel counts in multiples of 32): odd sizes
# with strides 2 and 3 (sub-pixel grad-input phases of different sizes, and
# phases no tap reaches), dilation, a rectangular and a 4x4 kernel, a single
# image, and output planes whose pixel count is not a multiple of 32 (grad
# weight then takes the element-gather kernel)
RING_CASES = [
    dict(n=2, cin=32, cout=64, k=3, s=2, p=1, hw=15),
    dict(n=3, cin=64, cout=32, k=3, s=1, p=2, hw=12, dil=2),
    dict(n=2, cin=32, cout=96, k=(1, 3), s=1, p=1, hw=8),
    dict(n=1, cin=128, cout=256, k=3, s=3, p=0, hw=17),
    dict(n=2, cin=32, cout=32, k=4, s=2, p=1, hw=16),
    dict(n=1, cin=64, cout=128, k=1, s=2, p=0, hw=9),
    # the gathered side needs whole 32-channel stages; the other channel count
    # is a column count and may be anything (3-channel stem grad input, 10
    # output channels, 40 input channels in 8-channel grad-weight chunks)
    dict(n=2, cin=3, cout=64, k=3, s=1, p=1, hw=16),
    dict(n=2, cin=32, cout=10, k=3, s=1, p=1, hw=8),
    dict(n=2, cin=40, cout=32, k=3, s=2, p=1, hw=12),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", RING_CASES)
def test_ring_geometry(gpu, dtype, case):
    case = dict(case)
    _check_all_directions(gpu, dtype, case.pop("n"), case.pop("cin"), case.pop("cout"), case.pop("k"),
                          case.pop("s"), case.pop("p"), case.pop("hw"), seed=40, **case)


# few-input-channel kernels (c_in * kh * kw <= 32, c_in < 32): stem shapes with
# widths that leave idle threads in the grad-input tile (24, 200), stride 2,
# a 5x5 kernel on one channel, an odd output-channel count (the grad-input
# pairs), paddings 0 and 2 (halo offsets), dilation, and output tiles past M
SMALL_CASES = [
    dict(n=3, cin=3, cout=64, k=3, s=1, p=1, hw=24),
    dict(n=2, cin=3, cout=96, k=3, s=2, p=1, hw=16),
    dict(n=2, cin=1, cout=16, k=5, s=1, p=2, hw=16),
    dict(n=2, cin=4, cout=7, k=3, s=1, p=1, hw=8),
    dict(n=2, cin=2, cout=40, k=3, s=1, p=0, hw=18),
    dict(n=2, cin=3, cout=64, k=3, s=1, p=2, hw=14),
    dict(n=1, cin=3, cout=32, k=3, s=1, p=1, hw=13, dil=2),
    dict(n=1, cin=3, cout=16, k=3, s=1, p=1, hw=200),
    # the MFMA grad-input kernel (64 output channels, padding 1, W 8/16/32/64):
    # 1-3 input channels, heights that end in a partial row tile
    dict(n=3, cin=1, cout=64, k=3, s=1, p=1, hw=(20, 8)),
    dict(n=2, cin=2, cout=64, k=3, s=1, p=1, hw=(7, 64)),
    dict(n=2, cin=3, cout=64, k=3, s=1, p=1, hw=(12, 32)),
    dict(n=2, cin=3, cout=64, k=3, s=1, p=1, hw=(16, 16)),
    # grad weight with the input rows staged in LDS (whole-row 512-pixel
    # chunks, W 16/32/64): 1-3 input channels, partial output-channel blocks
    dict(n=3, cin=3, cout=64, k=3, s=1, p=1, hw=(16, 32)),
    dict(n=2, cin=1, cout=48, k=3, s=1, p=1, hw=(64, 16)),
    dict(n=2, cin=2, cout=80, k=3, s=1, p=1, hw=(8, 64)),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", SMALL_CASES)
def test_few_input_channels(gpu, dtype, case):
    case = dict(case)
    _check_all_directions(gpu, dtype, case.pop("n"), case.pop("cin"), case.pop("cout"), case.pop("k"),
                          case.pop("s"), case.pop("p"), case.pop("hw"), seed=50, **case)


# stride-1 3x3 padding-1 halo kernels. Forward and grad input: every tile
# width (64, 32, 16, 8 pixels; 4, 8, 16, 32 rows a tile), heights that end in
# a partial tile, one and three 32-channel chunks, output channel counts that
# leave a partial 64-channel tile, bias. Grad weight (64-channel blocks, whole
# 256-pixel tiles): two input-channel blocks, a partial output-channel block,
# fewer tiles than the four a workgroup sums
HALO_CASES = [
    dict(n=2, cin=32, cout=64, k=3, s=1, p=1, hw=(20, 16)),
    dict(n=1, cin=96, cout=96, k=3, s=1, p=1, hw=(10, 64)),
    dict(n=2, cin=64, cout=40, k=3, s=1, p=1, hw=(13, 8)),
    dict(n=3, cin=32, cout=32, k=3, s=1, p=1, hw=(9, 32)),
    dict(n=2, cin=64, cout=96, k=3, s=1, p=1, hw=(16, 16)),
    dict(n=1, cin=128, cout=64, k=3, s=1, p=1, hw=(64, 8)),
    dict(n=3, cin=64, cout=32, k=3, s=1, p=1, hw=(8, 32)),
    # grad weight in 32-output-channel blocks (one 64-channel input block and
    # at most 64 output channels): a partial second block, and 16-wide rows
    dict(n=3, cin=64, cout=48, k=3, s=1, p=1, hw=(16, 32)),
    dict(n=2, cin=64, cout=64, k=3, s=1, p=1, hw=(32, 16)),
    # stride-2 forward halo kernel (de-interleaved columns, 128-pixel tiles):
    # a partial row tile, a partial output-channel tile, three k chunks, and
    # 64-pixel images two a tile with the batch's last tile half empty
    dict(n=2, cin=32, cout=96, k=3, s=2, p=1, hw=(32, 16)),
    dict(n=1, cin=64, cout=64, k=3, s=2, p=1, hw=(12, 64)),
    dict(n=3, cin=96, cout=32, k=3, s=2, p=1, hw=(16, 32)),
    dict(n=3, cin=96, cout=32, k=3, s=2, p=1, hw=(8, 32)),
    # stride-2 grad input by phases: 128-position tiles of one image (rows of
    # 16 and 32 dy columns) and of two images with the batch's last tile half
    # empty; 64-position tiles holding two images of an odd batch
    dict(n=256, cin=64, cout=32, k=3, s=2, p=1, hw=(32, 32), sample_n=4),
    dict(n=32, cin=32, cout=32, k=3, s=2, p=1, hw=(64, 64), sample_n=3),
    dict(n=511, cin=64, cout=32, k=3, s=2, p=1, hw=(16, 16)),
    dict(n=5, cin=32, cout=64, k=3, s=2, p=1, hw=(8, 16)),
    # 128-position tiles of two images x 32-channel blocks, the last block
    # partial and the batch's last tile half empty
    dict(n=255, cin=48, cout=32, k=3, s=2, p=1, hw=(16, 16)),
    # 64 dy columns: one-row 64-position tiles, and two-row 128-position tiles
    dict(n=2, cin=32, cout=32, k=3, s=2, p=1, hw=(8, 128)),
    dict(n=128, cin=32, cout=32, k=3, s=2, p=1, hw=(8, 128), sample_n=2),
    # forward: 8x8 outputs two images a tile
    dict(n=3, cin=64, cout=96, k=3, s=2, p=1, hw=(16, 16)),
]

# 1x1 kernels from NCHW (stride 1 or 2, no padding). Grad weight (64-channel
# input blocks): a partial output-channel block, two input blocks, stride 1,
# non-square images. Forward and grad input (256- or 64-pixel tiles): both
# tile sizes, three 32-channel k steps, a plane that takes neither tile (the
# ring kernel), a partial 64-channel block of grad input at stride 2
POINT_CASES = [
    dict(n=2, cin=64, cout=40, k=1, s=2, p=0, hw=(16, 32)),
    dict(n=3, cin=128, cout=96, k=1, s=1, p=0, hw=(4, 16)),
    dict(n=1, cin=64, cout=64, k=1, s=2, p=0, hw=(8, 16)),
    dict(n=2, cin=96, cout=64, k=1, s=1, p=0, hw=(16, 16)),
    dict(n=2, cin=40, cout=64, k=1, s=2, p=0, hw=(16, 32)),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", POINT_CASES)
def test_pointwise_grad_weight(gpu, dtype, case):
    case = dict(case)
    _check_all_directions(gpu, dtype, case.pop("n"), case.pop("cin"), case.pop("cout"), case.pop("k"),
                          case.pop("s"), case.pop("p"), case.pop("hw"), seed=70, **case)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", HALO_CASES)
def test_halo_stride1_3x3(gpu, dtype, case):
    case = dict(case)
    _check_all_directions(gpu, dtype, case.pop("n"), case.pop("cin"), case.pop("cout"), case.pop("k"),
                          case.pop("s"), case.pop("p"), case.pop("hw"), seed=60, **case)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_exact_mode_bit_identical(gpu, dtype):
    _check_all_directions(gpu, dtype, 4, 16, 32, 3, 2, 1, 12, seed=30, exact=True)


def test_c4_64x64_within_tolerance_of_reference_winograd(gpu):
    # the reference runs this layer through Winograd F(2x2,3x3) with fp16 intermediates
    dtype = torch.float16
    x = _x((8, 64, 32, 32), dtype, 40)
    w = _w((64, 64, 3, 3), dtype, 41)
    b = _x((64,), dtype, 42)
    y = gpu.conv2d_fwd(x.to(DEV), w.to(DEV), b.to(DEV), 1, 1)
    torch.cuda.synchronize()
    wino = decode(orc.winograd_conv2d(to_np(x), to_np(w), orc.F16, bias=to_np(b), padding=(1, 1)), dtype)
    assert_close(decode(to_np(y), dtype), wino, dtype, "implicit GEMM vs reference Winograd")


def test_empty_batch_wgrad_is_zero(gpu):
    x = torch.empty((0, 4, 6, 6), dtype=torch.float16, device=DEV)
    dy = torch.empty((0, 8, 6, 6), dtype=torch.float16, device=DEV)
    gw = gpu.conv2d_wgrad(x, dy, (8, 4, 3, 3), 1, 1)
    torch.cuda.synchronize()
    assert torch.count_nonzero(gw).item() == 0
