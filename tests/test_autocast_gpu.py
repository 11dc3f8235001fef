"""Automatic mixed precision on the vulkan device (the reference's
AutocastPrivateUse1 registration, src/api/registration.cpp:4-21).

Under torch.autocast("vulkan", float16 or bfloat16), float32 modules run their
products in the autocast dtype: nn.Linear and F.conv2d produce outputs of that
dtype, computed by the 16-bit MFMA kernels from the cast inputs, and the
gradients of the float32 parameters come back as float32. Strict mode is on,
so any CPU fallback on the way (the casts, the products, the backward) raises.

Parity: the oracle run on the inputs cast to the autocast dtype, within the
16-bit tolerance |got - ref| <= 5e-3 (|ref| + 1) (bfloat16 with the one-step
allowance that gemm_cases.py states).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.gemm_cases import ORC_DT, assert_close, decode, gen, oracle_mm, to_np

pytestmark = pytest.mark.gpu

V = "vulkan"


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


def _randn(shape, seed, std=1.0):
    return torch.randn(shape, generator=gen(seed)) * std


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_linear_under_autocast(gpu, strict, dt):
    import torchvulkan_amd  # noqa: F401

    lin = torch.nn.Linear(512, 384).to(V)
    x32 = _randn((256, 512), 1)
    dy = _randn((256, 384), 2).to(dt)
    xv = x32.to(V).requires_grad_()
    with torch.autocast("vulkan", dtype=dt):
        y = lin(xv)
    assert y.dtype == dt and y.device.type == "vulkan"
    y.backward(dy.to(V))
    # parameters stay float32, their gradients come back float32 through the cast's backward
    assert lin.weight.dtype == torch.float32 and lin.weight.grad.dtype == torch.float32
    assert xv.grad.dtype == torch.float32
    W = lin.weight.detach().cpu().to(dt)
    b = lin.bias.detach().cpu().to(dt)
    x = x32.to(dt)
    assert_close(y.detach().cpu().float().numpy(), oracle_mm(x, W.t(), dt, bias=b, beta=1.0), dt,
                 "autocast Linear forward")
    assert_close(xv.grad.cpu().numpy(), oracle_mm(dy, W, dt), dt, "autocast Linear grad input")
    assert_close(lin.weight.grad.cpu().numpy(), oracle_mm(dy.t(), x, dt), dt, "autocast Linear grad weight")
    # the product the backend issues for this forward is a 16-bit MFMA kernel
    dev = torch.device("cuda")
    c = torch.empty((256, 384), dtype=dt, device=dev)
    plan = gpu.gemm_plan(x.to(dev), W.to(dev).t(), c, bias=b.to(dev), beta=1.0)
    assert plan.startswith("gemm16"), plan


def test_conv2d_under_autocast(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    dt = torch.float16
    n, cin, cout, hw = 16, 32, 64, 16
    x32 = _randn((n, cin, hw, hw), 3)
    w32 = _randn((cout, cin, 3, 3), 4, std=(2.0 / (cin * 9)) ** 0.5)
    b32 = _randn((cout,), 5)
    xv, wv, bv = (t.to(V).requires_grad_() for t in (x32, w32, b32))
    with torch.autocast("vulkan", dtype=dt):
        y = F.conv2d(xv, wv, bv, stride=2, padding=1)
    assert y.dtype == dt
    dy = _randn(tuple(y.shape), 6).to(dt)
    y.backward(dy.to(V))
    assert wv.grad.dtype == torch.float32 and xv.grad.dtype == torch.float32
    x, w, b = x32.to(dt), w32.to(dt), b32.to(dt)
    od = ORC_DT[dt]
    oy = decode(orc.conv2d(to_np(x), to_np(w), od, bias=to_np(b), stride=(2, 2), padding=(1, 1)), dt)
    assert_close(y.detach().cpu().float().numpy(), oy, dt, "autocast conv2d forward")
    ogx = decode(orc.conv2d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, (2, 2), (1, 1), (1, 1), 1), dt)
    assert_close(xv.grad.cpu().numpy(), ogx, dt, "autocast conv2d grad input")
    ogw = decode(orc.conv2d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, (2, 2), (1, 1), (1, 1), 1, acc64=True), dt)
    assert_close(wv.grad.cpu().numpy(), ogw, dt, "autocast conv2d grad weight")


def test_autocast_policy_lists(gpu, strict):
    """Products in the lower-precision list run in the autocast dtype, a float32 bias included; autocast
    switched off inside the region gives float32 again."""
    import torchvulkan_amd  # noqa: F401

    a = _randn((64, 96), 7).to(V)
    b = _randn((96, 32), 8).to(V)
    with torch.autocast("vulkan", dtype=torch.float16):
        p = a @ b                       # lower-precision list
        assert p.dtype == torch.float16
        with torch.autocast("vulkan", enabled=False):
            q = a @ b                   # autocast off inside: float32 again
        assert q.dtype == torch.float32
        s = torch.addmm(q[0], a, b)     # float32 bias, operands: all cast
        assert s.dtype == torch.float16
    ref = (a.cpu().half().double() @ b.cpu().half().double()).numpy()
    assert_close(p.cpu().float().numpy(), ref, torch.float16, "autocast matmul vs float64")
    assert np.isfinite(s.cpu().float().numpy()).all()
