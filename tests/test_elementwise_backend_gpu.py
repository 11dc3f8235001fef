"""sum and add/sub/mul on the vulkan device (TORCHVULKAN_STRICT=1: a CPU
fallback would raise), compared with CPU results: exactly where the
reference's rounding equals torch's (alpha == 1, integer inputs), with the
oracle's per-operation rounding otherwise, and an nn.Linear training step
(forward, two accumulating backwards, an in-place update) that stays on the
device end to end."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

V = "vulkan"


@pytest.fixture()
def strict(gpu, monkeypatch):
    import torchvulkan_amd

    monkeypatch.setenv("TORCHVULKAN_STRICT", "1")
    return torchvulkan_amd


def bits(t):
    t = t.cpu()
    return t.view(torch.int16) if t.dtype in (torch.float16, torch.bfloat16) else t


def test_sum_variants(strict):
    g = torch.Generator().manual_seed(0)
    x = torch.randint(-5, 6, (16, 8, 6, 6), generator=g).float()
    xv = x.to(V)
    assert torch.equal(xv.sum().cpu(), x.sum())
    assert torch.equal(xv.sum(0).cpu(), x.sum(0))
    assert torch.equal(xv.sum((0, 2, 3)).cpu(), x.sum((0, 2, 3)))
    assert torch.equal(xv.sum(-1, keepdim=True).cpu(), x.sum(-1, keepdim=True))
    assert torch.equal(xv.half().sum(1, dtype=torch.float32).cpu(), x.half().sum(1, dtype=torch.float32))
    i = torch.randint(-100, 100, (50, 7), generator=g, dtype=torch.int32)
    r = i.to(V).sum(0)
    assert r.dtype == torch.int64 and torch.equal(r.cpu(), i.sum(0))
    with pytest.raises(IndexError):
        xv.sum(7)
    with pytest.raises(RuntimeError, match="appears multiple times"):
        xv.sum((1, 1))
    y = torch.randn((300, 200), generator=g)
    torch.testing.assert_close(y.to(V).sum(0).cpu(), y.sum(0), rtol=1e-5, atol=1e-5)


def test_add_sub_mul(strict):
    g = torch.Generator().manual_seed(1)
    a, b = torch.randn((33, 17), generator=g), torch.randn((33, 17), generator=g)
    av, bv = a.to(V), b.to(V)
    assert torch.equal((av + bv).cpu(), a + b)
    assert torch.equal((av - bv).cpu(), a - b)
    assert torch.equal((av * bv).cpu(), a * b)
    assert torch.equal((av + 2.0).cpu(), a + 2.0)
    assert torch.equal((av * bv[0]).cpu(), a * b[0])              # broadcast
    for dt in (torch.float16, torch.bfloat16):
        ah, bh = a.to(dt), b.to(dt)
        assert torch.equal(bits(ah.to(V) + bh.to(V)), bits(ah + bh))
        got = torch.add(ah.to(V), bh.to(V), alpha=0.5)
        code = orc.F16 if dt == torch.float16 else orc.BF16
        want = orc.binary(bits(ah).numpy().view(np.uint16), bits(bh).numpy().view(np.uint16), code, orc.BIN_ADD, 0.5)
        assert (bits(got).numpy().view(np.uint16) == want).all()
    # promotion: half + float -> float
    r = a.half().to(V) + bv
    assert r.dtype == torch.float32 and torch.equal(r.cpu(), a.half() + b)
    c = av.clone()
    c.add_(bv, alpha=-0.25)
    want = orc.binary(a.numpy(), b.numpy(), orc.F32, orc.BIN_ADD, -0.25)
    assert (c.cpu().numpy() == want).all()
    out = torch.empty((0,), device=V)
    torch.sub(av, bv, out=out)
    assert out.shape == (33, 17) and torch.equal(out.cpu(), a - b)
    with pytest.raises(RuntimeError, match="doesn't match the broadcast shape"):
        av[0].add_(bv)
    with pytest.raises(RuntimeError, match="alpha must not be a floating point"):
        torch.add(torch.ones(3, dtype=torch.int32, device=V), torch.ones(3, dtype=torch.int32, device=V), alpha=0.5)
    ii = torch.arange(10, dtype=torch.int64)
    assert torch.equal((ii.to(V) * ii.to(V) - ii.to(V)).cpu(), ii * ii - ii)


def test_linear_training_step_stays_on_device(strict):
    torch.manual_seed(0)
    ref = torch.nn.Linear(64, 32)
    dev = torch.nn.Linear(64, 32).to(V)
    with torch.no_grad():
        dev.weight.copy_(ref.weight.to(V))
        dev.bias.copy_(ref.bias.to(V))
    g = torch.Generator().manual_seed(2)
    x1, x2 = torch.randn((16, 64), generator=g), torch.randn((16, 64), generator=g)
    for m, xs in ((ref, (x1, x2)), (dev, (x1.to(V), x2.to(V)))):
        for x in xs:                       # two backwards: the second accumulates into .grad
            (m(x) * m(x)).sum().backward()
        with torch.no_grad():
            for p in m.parameters():
                p.add_(p.grad, alpha=-0.01)
    for p_ref, p_dev in zip(ref.parameters(), dev.parameters()):
        torch.testing.assert_close(p_dev.detach().cpu(), p_ref.detach(), rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(p_dev.grad.cpu(), p_ref.grad, rtol=1e-4, atol=1e-4)
