"""Pins the convolution oracle (oracle/conv_oracle.c) against torch CPU in
float64: integer-valued operands make every summation order exact, so the
index maps (padding, stride, dilation, groups, 1x1, transposed gradients) are
held to equality; random operands check the Winograd restatement against the
direct convolution it must approximate."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

GEOMS = [
    # x shape, w shape, stride, padding, dilation, groups
    ((2, 3, 9, 9), (4, 3, 3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((2, 4, 10, 7), (6, 4, 3, 3), (2, 2), (1, 1), (1, 1), 1),
    ((1, 4, 9, 11), (6, 2, 3, 3), (2, 1), (1, 2), (1, 2), 2),
    ((3, 8, 6, 6), (4, 8, 1, 1), (2, 2), (0, 0), (1, 1), 1),
    ((1, 2, 5, 5), (2, 2, 5, 3), (1, 3), (2, 0), (1, 1), 1),
]


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.build()


def _ints(shape, seed, lo=-3, hi=4):
    return np.random.default_rng(seed).integers(lo, hi, shape).astype(np.float32)


@pytest.mark.parametrize("geom", GEOMS)
def test_forward_exact(geom):
    xs, ws, s, p, d, g = geom
    x, w, b = _ints(xs, 1), _ints(ws, 2), _ints((ws[0],), 3)
    got = orc.conv2d(x, w, orc.F32, bias=b, stride=s, padding=p, dilation=d, groups=g)
    want = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                      torch.from_numpy(b).double(), s, p, d, g).numpy()
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("geom", GEOMS)
def test_gradients_exact(geom):
    xs, ws, s, p, d, g = geom
    x = torch.from_numpy(_ints(xs, 4)).double().requires_grad_()
    w = torch.from_numpy(_ints(ws, 5)).double().requires_grad_()
    y = torch.nn.functional.conv2d(x, w, None, s, p, d, g)
    dy = torch.from_numpy(_ints(tuple(y.shape), 6)).double()
    y.backward(dy)
    dx = orc.conv2d_dgrad(dy.float().numpy(), w.detach().float().numpy(), xs, orc.F32, s, p, d, g)
    dw = orc.conv2d_wgrad(x.detach().float().numpy(), dy.float().numpy(), ws, orc.F32, s, p, d, g)
    dw32 = orc.conv2d_wgrad(x.detach().float().numpy(), dy.float().numpy(), ws, orc.F32, s, p, d, g, acc64=False)
    assert np.array_equal(dx, x.grad.numpy().astype(np.float32))
    assert np.array_equal(dw, w.grad.numpy().astype(np.float32))
    assert np.array_equal(dw32, w.grad.numpy().astype(np.float32))


def test_fp16_storage_rounds_once():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 8, 8, 8)).astype(np.float16)
    w = (rng.standard_normal((8, 8, 3, 3)) * 0.1).astype(np.float16)
    got = orc.conv2d(x.view(np.uint16), w.view(np.uint16), orc.F16, padding=(1, 1)).view(np.float16)
    want = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(), padding=1).numpy()
    # one rounding of a float32 accumulation: within half an fp16 ulp plus the fp32 sum error
    assert np.all(np.abs(got.astype(np.float64) - want) <= np.abs(want) * 2.0 ** -11 + 1e-4)


@pytest.mark.parametrize("dtype,tol", [(orc.F32, 1e-5), (orc.F16, 5e-3)])
def test_winograd_restatement_close_to_direct(dtype, tol):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 16, 9, 10)).astype(np.float32)
    w = (rng.standard_normal((16, 16, 3, 3)) * np.sqrt(2 / 144)).astype(np.float32)
    b = rng.standard_normal(16).astype(np.float32)
    if dtype == orc.F16:
        x, w, b = (v.astype(np.float16).view(np.uint16) for v in (x, w, b))
    wino = orc.to_f32(orc.winograd_conv2d(x, w, dtype, bias=b, padding=(1, 1)), dtype)
    direct = orc.to_f32(orc.conv2d(x, w, dtype, bias=b, padding=(1, 1)), dtype)
    assert np.all(np.abs(wino - direct) <= tol * (np.abs(direct) + 1))
    if dtype == orc.F16:
        # the rounded intermediates do change the result (the check has teeth)
        assert not np.array_equal(wino, direct)


@pytest.mark.parametrize("dtype", [orc.F32, orc.F16])
def test_winograd_transforms_exact_on_integers(dtype):
    # Weights in multiples of 4 and small integer inputs keep every intermediate of F(2x2, 3x3) an
    # integer far inside float16's exact range: the filter transform's halvings divide sums of
    # multiples of 4, the input transform and the products add integers (|M| < 2048 here). The
    # staged roundings are then all exact and Winograd equals direct convolution bit for bit; a wrong
    # coefficient, sign or index in G, B^T or A^T (or a mis-tiled output) breaks the equality.
    rng = np.random.default_rng(11)
    x = rng.integers(-2, 3, size=(2, 4, 7, 9)).astype(np.float32)
    w = (4 * rng.integers(-1, 2, size=(5, 4, 3, 3))).astype(np.float32)
    b = rng.integers(-3, 4, size=5).astype(np.float32)
    direct64 = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                          torch.from_numpy(b).double(), padding=1).numpy()
    assert np.abs(direct64).max() < 2048
    if dtype == orc.F16:
        x, w, b = (v.astype(np.float16).view(np.uint16) for v in (x, w, b))
    wino = orc.to_f32(orc.winograd_conv2d(x, w, dtype, bias=b, padding=(1, 1)), dtype)
    assert np.array_equal(wino, direct64.astype(np.float32))


# ---------------------------------------------------------------------------
# 3-D restatement (oracle_conv3d_*): the reference takes up to three spatial
# dimensions (src/api/ops/conv.cpp:295-311)
# ---------------------------------------------------------------------------

GEOMS3 = [
    # x shape, w shape, stride, padding, dilation, groups
    ((2, 3, 5, 6, 7), (4, 3, 3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), 1),
    ((1, 4, 7, 6, 9), (6, 4, 3, 3, 3), (2, 2, 2), (1, 1, 1), (1, 1, 1), 1),
    ((2, 4, 6, 5, 8), (6, 2, 3, 2, 3), (2, 1, 3), (1, 0, 2), (2, 1, 1), 2),
    ((1, 6, 4, 6, 6), (3, 6, 1, 1, 1), (1, 2, 2), (0, 0, 0), (1, 1, 1), 1),
    ((2, 3, 5, 5, 5), (3, 1, 3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 2, 1), 3),   # depthwise, dilated
]


@pytest.mark.parametrize("geom", GEOMS3)
def test_conv3d_forward_exact(geom):
    xs, ws, s, p, d, g = geom
    x, w, b = _ints(xs, 11), _ints(ws, 12), _ints((ws[0],), 13)
    got = orc.conv3d(x, w, orc.F32, bias=b, stride=s, padding=p, dilation=d, groups=g)
    want = torch.nn.functional.conv3d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                      torch.from_numpy(b).double(), s, p, d, g).numpy()
    assert got.shape == want.shape
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("geom", GEOMS3)
def test_conv3d_gradients_exact(geom):
    xs, ws, s, p, d, g = geom
    x = torch.from_numpy(_ints(xs, 14)).double().requires_grad_()
    w = torch.from_numpy(_ints(ws, 15)).double().requires_grad_()
    y = torch.nn.functional.conv3d(x, w, None, s, p, d, g)
    dy = torch.from_numpy(_ints(tuple(y.shape), 16)).double()
    y.backward(dy)
    dx = orc.conv3d_dgrad(dy.float().numpy(), w.detach().float().numpy(), xs, orc.F32, s, p, d, g)
    dw = orc.conv3d_wgrad(x.detach().float().numpy(), dy.float().numpy(), ws, orc.F32, s, p, d, g)
    dw32 = orc.conv3d_wgrad(x.detach().float().numpy(), dy.float().numpy(), ws, orc.F32, s, p, d, g, acc64=False)
    assert np.array_equal(dx, x.grad.numpy().astype(np.float32))
    assert np.array_equal(dw, w.grad.numpy().astype(np.float32))
    assert np.array_equal(dw32, w.grad.numpy().astype(np.float32))


def _columns(x, kernel, stride, padding, dilation):
    """im2col by numpy windows: [c * prod(kernel), n * prod(out)], rows in (c, kd, kh, kw) order."""
    nd = len(kernel)
    pad = [(0, 0), (0, 0)] + [(p, p) for p in padding]
    xp = np.pad(x, pad)
    span = [(k - 1) * d + 1 for k, d in zip(kernel, dilation)]
    win = np.lib.stride_tricks.sliding_window_view(xp, span, axis=tuple(range(2, 2 + nd)))
    idx = (slice(None), slice(None)) + tuple(slice(None, None, s) for s in stride) + tuple(slice(None, None, d) for d in dilation)
    win = win[idx]   # [n, c, out..., kernel...]
    n, c = x.shape[:2]
    out = win.shape[2:2 + nd]
    perm = (1,) + tuple(range(2 + nd, 2 + 2 * nd)) + (0,) + tuple(range(2, 2 + nd))
    return np.ascontiguousarray(win.transpose(perm)).reshape(c * int(np.prod(kernel)), n * int(np.prod(out))), out


@pytest.mark.parametrize("nd", [2, 3])
def test_conv_k_order_is_the_gemm_order(nd):
    """The conv oracle accumulates in the k order (c, [kd,] kh, kw): on random float32 data (where the order
    shows in the last bits) it is bit-identical to the GEMM oracle, whose fused-multiply-add order is pinned by
    test_oracle.py, applied to the im2col columns."""
    rng = np.random.default_rng(20 + nd)
    if nd == 2:
        xs, ws, s, p, d = (2, 5, 9, 8), (6, 5, 3, 2), (2, 1), (1, 1), (1, 2)
    else:
        xs, ws, s, p, d = (2, 4, 5, 6, 7), (6, 4, 3, 2, 3), (1, 2, 2), (1, 0, 1), (2, 1, 1)
    x = rng.standard_normal(xs).astype(np.float32)
    w = rng.standard_normal(ws).astype(np.float32)
    cols, out = _columns(x, ws[2:], s, p, d)
    prod = orc.gemm(w.reshape(ws[0], -1), cols, orc.F32)                       # [cout, n * prod(out)]
    want = prod.reshape((ws[0], xs[0]) + tuple(out)).swapaxes(0, 1)
    got = (orc.conv2d if nd == 2 else orc.conv3d)(x, w, orc.F32, stride=s, padding=p, dilation=d)
    assert np.array_equal(got, want)
    # the order matters on these data: summing the taps in reverse gives other bits somewhere
    rev = orc.gemm(w.reshape(ws[0], -1)[:, ::-1], cols[::-1], orc.F32)
    assert not np.array_equal(prod, rev)
