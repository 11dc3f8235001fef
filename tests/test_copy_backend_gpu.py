"""Copies and casts on the vulkan device run on the GPU (tvk_copy), with
TORCHVULKAN_STRICT=1 so that any CPU fallback would raise: .to(dtype),
.contiguous() of transposed and sliced views, channels_last, device -> host
of strided and expanded views, host -> device into strided views. Values are
compared with the same operations on CPU tensors (bit-exact)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

V = "vulkan"


@pytest.fixture()
def strict(gpu, monkeypatch):
    import torchvulkan_amd

    monkeypatch.setenv("TORCHVULKAN_STRICT", "1")
    return torchvulkan_amd


def same(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.cpu(), b.cpu()
    if a.dtype in (torch.float16, torch.bfloat16):
        a, b = a.view(torch.int16), b.view(torch.int16)
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b)


def test_dtype_casts_on_device(strict):
    g = torch.Generator().manual_seed(0)
    x = torch.randn((123, 77), generator=g) * 100
    xv = x.to(V)
    for dt in (torch.float16, torch.bfloat16, torch.float64, torch.int32, torch.int64, torch.uint8, torch.bool):
        src = x.abs().clamp(max=250) if dt == torch.uint8 else x   # above 255 is undefined (x86 wraps)
        assert same(src.to(V).to(dt), src.to(dt)), dt
    assert same(torch.arange(-50, 50).to(V).float(), torch.arange(-50, 50).float())
    assert same((x > 0).to(V).to(torch.float16), (x > 0).to(torch.float16))
    assert same(xv.half().float(), x.half().float())
    strict.synchronize()


def test_contiguous_of_views(strict):
    g = torch.Generator().manual_seed(1)
    x = torch.randn((64, 96), generator=g, dtype=torch.float32).half()
    xv = x.to(V)
    assert same(xv.t().contiguous(), x.t().contiguous())
    assert same(xv[:, ::2].clone(), x[:, ::2].clone())
    assert same(xv.t().to(torch.float32), x.t().to(torch.float32))
    y = torch.randn((3, 5, 7, 9), generator=g)
    yv = y.to(V)
    cl = yv.contiguous(memory_format=torch.channels_last)
    assert cl.is_contiguous(memory_format=torch.channels_last)
    assert same(cl, y.contiguous(memory_format=torch.channels_last))
    assert same(cl.contiguous(), y)


def test_device_to_host_views(strict):
    g = torch.Generator().manual_seed(2)
    x = torch.randn((40, 30), generator=g)
    xv = x.to(V)
    assert same(xv.t().cpu(), x.t())
    assert same(xv[1::3, ::2].cpu(), x[1::3, ::2])
    assert same(xv[:1].expand(5, 30).cpu(), x[:1].expand(5, 30))
    assert same(xv.t().to("cpu", torch.float16), x.t().to(torch.float16))


def test_host_to_device_strided_destination(strict):
    g = torch.Generator().manual_seed(3)
    dst = torch.zeros((20, 16), device=V)
    part = torch.randn((20, 8), generator=g)
    dst[:, ::2] = part
    ref = torch.zeros((20, 16))
    ref[:, ::2] = part
    assert same(dst, ref)
    dst.t()[3].copy_(torch.arange(20, dtype=torch.float64))   # a column, cast on the host side
    ref.t()[3].copy_(torch.arange(20, dtype=torch.float64))
    assert same(dst, ref)


def test_overlap_is_rejected_as_on_cpu(strict):
    x = torch.arange(10.0).to(V)
    with pytest.raises(RuntimeError, match="single memory location"):
        x[1:].copy_(x[:-1])


def test_fill_and_zero_on_device(strict):
    assert same(torch.zeros((7, 9), device=V), torch.zeros((7, 9)))
    assert same(torch.ones((5, 3), dtype=torch.float16, device=V), torch.ones((5, 3), dtype=torch.float16))
    assert same(torch.full((4, 4), -2.5, dtype=torch.bfloat16, device=V), torch.full((4, 4), -2.5, dtype=torch.bfloat16))
    x = torch.arange(12.0).view(3, 4).to(V)
    x[:, 1].fill_(7.0)
    ref = torch.arange(12.0).view(3, 4)
    ref[:, 1].fill_(7.0)
    assert same(x, ref)
    x.fill_(torch.tensor(3.0).to(V))
    assert same(x, torch.full((3, 4), 3.0))
    # the scalar converts exactly as on the CPU: a lone element takes inf, a larger fill raises
    assert same(torch.empty(1, dtype=torch.float16, device=V).fill_(1e10), torch.empty(1, dtype=torch.float16).fill_(1e10))
    with pytest.raises(RuntimeError, match="overflow"):
        torch.empty(3, dtype=torch.float16, device=V).fill_(1e10)
