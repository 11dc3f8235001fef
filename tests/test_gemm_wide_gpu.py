"""float64 and integer products on the GPU (tvk_gemm's wide kernel, and
torch.mm/addmm/bmm/baddbmm/addmv on the vulkan device) against the oracle.
The bar is bit equality: float64 accumulates by fma in k order like the
oracle, and integer products wrap modulo 2^bits, which no summation order
changes."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
V = "vulkan"
WIDE = [(torch.float64, orc.F64), (torch.int64, orc.I64), (torch.int32, orc.I32), (torch.int16, orc.I16),
        (torch.int8, orc.I8), (torch.uint8, orc.U8)]


def rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.float64:
        return torch.randn(shape, generator=g, dtype=torch.float64)
    info = torch.iinfo(dtype)
    return torch.randint(info.min, info.max, shape, generator=g, dtype=torch.int64).to(dtype)


def equal(got: torch.Tensor, want: np.ndarray, what: str):
    g = got.detach().cpu().numpy()
    assert g.shape == want.shape, (what, g.shape, want.shape)
    if g.dtype == np.float64:
        bad = int((g.view(np.uint64) != want.view(np.uint64)).sum())
    else:
        bad = int((g != want).sum())
    assert bad == 0, f"{what}: {bad} of {g.size} elements differ from the oracle"


def device_view(t: torch.Tensor) -> torch.Tensor:
    base = t.as_strided((t.untyped_storage().nbytes() // t.element_size(),), (1,), 0).to(DEV)
    return base.as_strided(t.shape, t.stride(), t.storage_offset())


@pytest.mark.parametrize("dtype,odt", WIDE)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_wide_layouts_bit_exact(gpu, dtype, odt, ta, tb):
    M, N, K = 130, 97, 75
    a = rand((K, M), dtype, 1).t() if ta else rand((M, K), dtype, 1)
    b = rand((N, K), dtype, 2).t() if tb else rand((K, N), dtype, 3)
    c = torch.empty((M, N), dtype=dtype, device=DEV)
    gpu.gemm(device_view(a), device_view(b), c)
    torch.cuda.synchronize()
    equal(c, orc.gemm(a.numpy(), b.numpy(), odt), f"{dtype} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype,odt", WIDE)
def test_wide_batched_epilogue(gpu, dtype, odt):
    from torchvulkan_amd import _abi
    import ctypes as C

    a, b = rand((5, 64, 200), dtype, 4), rand((5, 200, 33), dtype, 5)
    bias = rand((5, 64, 33), dtype, 6)
    c = torch.empty((5, 64, 33), dtype=dtype, device=DEV)
    alpha, beta = (0.75, -1.25) if dtype == torch.float64 else (3.0, -2.0)
    for act in (orc.ACT_NONE, orc.ACT_RELU) + ((orc.ACT_GELU,) if dtype == torch.float64 else ()):
        d = _abi.make_gemm_desc(a.to(DEV), b.to(DEV), c, bias=bias.to(DEV), alpha=alpha, beta=beta, activation=act,
                                stream=torch.cuda.current_stream().cuda_stream)
        _abi.check(_abi.load().tvk_gemm(C.byref(d)))
        torch.cuda.synchronize()
        want = orc.gemm(a.numpy(), b.numpy(), odt, bias=bias.numpy(), alpha=alpha, beta=beta, act=act)
        if act == orc.ACT_GELU:
            # gelu's erf is the device library's, not the host's: float64 tolerance instead of bits
            g = c.cpu().numpy()
            assert np.abs(g - want).max() <= 1e-14 * (np.abs(want).max() + 1)
        else:
            equal(c, want, f"{dtype} act={act}")
        assert _abi.gemm_plan(a.to(DEV), b.to(DEV), c) == ("gemm_wide_f64" if dtype == torch.float64 else "gemm_wide_int")


def test_wide_k_zero_and_large_k(gpu):
    from torchvulkan_amd import _abi
    import ctypes as C

    s = torch.cuda.current_stream().cuda_stream
    a, b = torch.zeros((7, 0), dtype=torch.int32, device=DEV), torch.zeros((0, 9), dtype=torch.int32, device=DEV)
    bias = torch.arange(9, dtype=torch.int32)
    c = torch.full((7, 9), -1, dtype=torch.int32, device=DEV)
    d = _abi.make_gemm_desc(a, b, c, bias=bias.to(DEV), beta=2.0, stream=s)
    _abi.check(_abi.load().tvk_gemm(C.byref(d)))
    torch.cuda.synchronize()
    assert torch.equal(c.cpu(), (bias * 2).expand(7, 9))
    # a long K where float64 ordering shows
    x, y = rand((40, 4099), torch.float64, 7), rand((4099, 50), torch.float64, 8)
    z = torch.empty((40, 50), dtype=torch.float64, device=DEV)
    d = _abi.make_gemm_desc(x.to(DEV), y.to(DEV), z, stream=s)
    _abi.check(_abi.load().tvk_gemm(C.byref(d)))
    torch.cuda.synchronize()
    equal(z, orc.gemm(x.numpy(), y.numpy(), orc.F64), "float64 K 4099")


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


@pytest.mark.parametrize("dtype,odt", WIDE)
def test_wide_on_the_vulkan_device(gpu, strict, dtype, odt):
    import torchvulkan_amd  # noqa: F401

    a, b = rand((33, 45), dtype, 10), rand((45, 27), dtype, 11)
    bias = rand((27,), dtype, 12)
    equal(torch.mm(a.to(V), b.to(V)), orc.gemm(a.numpy(), b.numpy(), odt), f"{dtype} mm")
    alpha, beta = (0.5, 2.0) if dtype == torch.float64 else (3, 2)
    got = torch.addmm(bias.to(V), a.to(V), b.to(V), beta=beta, alpha=alpha)
    equal(got, orc.gemm(a.numpy(), b.numpy(), odt, bias=bias.numpy(), alpha=alpha, beta=beta), f"{dtype} addmm")
    x, y = rand((4, 10, 12), dtype, 13), rand((4, 12, 8), dtype, 14)
    equal(torch.bmm(x.to(V), y.to(V)), orc.gemm(x.numpy(), y.numpy(), odt), f"{dtype} bmm")
    inp = rand((4, 10, 8), dtype, 15)
    got = torch.baddbmm(inp.to(V), x.to(V), y.to(V), beta=beta, alpha=alpha)
    equal(got, orc.gemm(x.numpy(), y.numpy(), odt, bias=inp.numpy(), alpha=alpha, beta=beta), f"{dtype} baddbmm")
    v = rand((45,), dtype, 16)
    want = orc.gemm(v.numpy().reshape(1, 45), a.numpy().T, odt).reshape(33)
    equal(torch.mv(a.to(V), v.to(V)), want, f"{dtype} mv")
    if dtype != torch.float64:
        # the CPU computes integer products with the same wraparound
        assert torch.equal(torch.mm(a.to(V), b.to(V)).cpu(), torch.mm(a, b))


@pytest.mark.parametrize("dtype", [torch.float64, torch.int32, torch.int8, torch.uint8, torch.int64])
@pytest.mark.parametrize("cfg", [
    # (n, cin, h, w), (cout, cin/g, kh, kw), stride, padding, dilation, groups
    ((2, 6, 11, 9), (8, 6, 3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((3, 4, 10, 12), (6, 2, 3, 2), (2, 1), (0, 1), (1, 2), 2),
    ((1, 3, 7, 7), (5, 3, 1, 1), (2, 2), (0, 0), (1, 1), 1),
])
def test_wide_convolution_forward(gpu, strict, dtype, cfg):
    # im2col on the device + the wide GEMM; small integer values keep every sum exact, so the
    # float64 CPU convolution is the reference for the integer types too (the CPU has no integer conv)
    import torch.nn.functional as F
    import torchvulkan_amd  # noqa: F401

    xs, ws, st, pd, dl, g = cfg
    gen = torch.Generator().manual_seed(40)
    lo = 0 if dtype == torch.uint8 else -3
    x = torch.randint(lo, 4, xs, generator=gen).to(dtype)
    w = torch.randint(lo, 3, ws, generator=gen).to(dtype)
    b = torch.randint(lo, 4, (ws[0],), generator=gen).to(dtype)
    if dtype == torch.float64:
        x, w, b = x + torch.randn(xs, generator=gen, dtype=torch.float64), w * 0.37, b * 0.5
    got = F.conv2d(x.to(V), w.to(V), b.to(V), stride=st, padding=pd, dilation=dl, groups=g)
    want = F.conv2d(x.double(), w.double(), b.double(), stride=st, padding=pd, dilation=dl, groups=g)
    if dtype == torch.float64:
        assert ((got.cpu() - want).abs() <= 1e-12 * (want.abs() + 1)).all()
    else:
        assert torch.equal(got.cpu(), want.to(dtype))
    # transposed convolution (the input gradient of the forward one)
    wt = w.transpose(0, 1).contiguous() if g == 1 else None
    if wt is not None:
        got = F.conv_transpose2d(x.to(V), wt.to(V), stride=st, padding=pd, dilation=dl)
        want = F.conv_transpose2d(x.double(), wt.double(), stride=st, padding=pd, dilation=dl)
        if dtype == torch.float64:
            assert ((got.cpu() - want).abs() <= 1e-12 * (want.abs() + 1)).all()
        else:
            assert torch.equal(got.cpu(), want.to(dtype))


def test_float64_convolution_backward(gpu, strict):
    import torch.nn.functional as F
    import torchvulkan_amd  # noqa: F401

    gen = torch.Generator().manual_seed(41)
    x = torch.randn((2, 4, 9, 10), generator=gen, dtype=torch.float64)
    w = torch.randn((6, 2, 3, 3), generator=gen, dtype=torch.float64)
    b = torch.randn((6,), generator=gen, dtype=torch.float64)
    xv, wv, bv = (t.to(V).requires_grad_() for t in (x, w, b))
    xc, wc, bc = (t.clone().requires_grad_() for t in (x, w, b))
    y = F.conv2d(xv, wv, bv, stride=2, padding=1, groups=2)
    yc = F.conv2d(xc, wc, bc, stride=2, padding=1, groups=2)
    gy = torch.randn(tuple(yc.shape), generator=gen, dtype=torch.float64)
    y.backward(gy.to(V))
    yc.backward(gy)
    for got, want, name in ((xv.grad, xc.grad, "dx"), (wv.grad, wc.grad, "dw"), (bv.grad, bc.grad, "db")):
        assert got.shape == want.shape, name
        assert ((got.cpu() - want).abs() <= 1e-12 * (want.abs() + 1)).all(), name
