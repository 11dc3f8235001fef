"""The vulkan device end to end on the GPU: torch ops on device="vulkan" reach
the gfx950 kernels through the PrivateUse1 registrations, with the reference's
semantics (results within the north_star tolerance of the oracle, CPU-identical
error messages, output shapes and contiguity, autograd through nn.Linear and
F.conv2d, strict mode, memory statistics)."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.gemm_cases import ORC_DT, assert_close, decode, gen, oracle_mm, randn, to_np

pytestmark = pytest.mark.gpu

V = "vulkan"


@pytest.fixture(scope="module")
def tv(gpu):
    import torchvulkan_amd

    assert torchvulkan_amd.is_available()
    return torchvulkan_amd


def host(t):
    return t.to("cpu")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_mm_addmm_bmm_baddbmm(tv, dtype):
    a, b = randn((300, 200), dtype, 1), randn((200, 260), dtype, 2)
    bias = randn((260,), dtype, 3)
    assert_close(decode(to_np(host(torch.mm(a.to(V), b.to(V)))), dtype), oracle_mm(a, b, dtype), dtype, "mm")
    got = torch.addmm(bias.to(V), a.to(V), b.to(V), beta=0.5, alpha=2.0)
    assert_close(decode(to_np(host(got)), dtype), oracle_mm(a, b, dtype, bias=bias, alpha=2.0, beta=0.5), dtype, "addmm")
    x, y = randn((6, 40, 30), dtype, 4), randn((6, 30, 50), dtype, 5)
    assert_close(decode(to_np(host(torch.bmm(x.to(V), y.to(V)))), dtype), oracle_mm(x, y, dtype), dtype, "bmm")
    inp = randn((6, 40, 50), dtype, 6)
    got = torch.baddbmm(inp.to(V), x.to(V), y.to(V), beta=1.0, alpha=0.5)
    assert_close(decode(to_np(host(got)), dtype), oracle_mm(x, y, dtype, bias=inp, alpha=0.5, beta=1.0), dtype, "baddbmm")


def test_transposed_views_and_out_variants(tv):
    dtype = torch.float16
    a = randn((64, 48), dtype, 10).to(V)
    b = randn((80, 48), dtype, 11).to(V)
    got = torch.mm(a, b.t())                       # k-contiguous B, no copy
    ref = oracle_mm(host(a), host(b).t(), dtype)
    assert got.is_contiguous() and got.shape == (64, 80)
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "mm(a, b.t())")
    out = torch.empty((1, 1), dtype=dtype, device=V)
    torch.mm(a, b.t(), out=out)
    assert out.shape == (64, 80)
    assert_close(decode(to_np(host(out)), dtype), ref, dtype, "mm.out")


def test_matmul_broadcast_and_vectors(tv):
    dtype = torch.float32
    x = randn((3, 5, 7), dtype, 20)
    w = randn((7, 4), dtype, 21)
    v = randn((7,), dtype, 22)
    got = torch.matmul(x.to(V), w.to(V))
    assert got.shape == (3, 5, 4)
    assert_close(host(got).numpy(), torch.matmul(x.double(), w.double()).numpy(), dtype, "matmul 3d@2d")
    got = torch.matmul(w.t().contiguous().to(V), v.to(V))
    assert got.shape == (4,)
    assert_close(host(got).numpy(), (w.t().double() @ v.double()).numpy(), dtype, "matvec")


def test_addmm_activation_and_addbmm(tv):
    dtype = torch.float16
    a, b, bias = randn((33, 40), dtype, 30), randn((40, 21), dtype, 31), randn((21,), dtype, 32)
    for gelu in (False, True):
        got = torch._addmm_activation(bias.to(V), a.to(V), b.to(V), use_gelu=gelu)
        ref = oracle_mm(a, b, dtype, bias=bias, beta=1.0, act=orc.ACT_GELU if gelu else orc.ACT_RELU)
        assert_close(decode(to_np(host(got)), dtype), ref, dtype, "_addmm_activation")
    b1, b2, inp = randn((5, 9, 12), dtype, 33), randn((5, 12, 7), dtype, 34), randn((9, 7), dtype, 35)
    got = torch.addbmm(inp.to(V), b1.to(V), b2.to(V))
    ref = torch.addbmm(inp.double(), b1.double(), b2.double()).numpy()
    assert_close(decode(to_np(host(got)), dtype), ref, dtype, "addbmm")


ERROR_CASES = {
    "mm 1d": lambda d: torch.mm(torch.zeros(3, device=d), torch.zeros(3, 3, device=d)),
    "mm 1d b": lambda d: torch.mm(torch.zeros(3, 3, device=d), torch.zeros(3, device=d)),
    "mm shape": lambda d: torch.mm(torch.zeros(2, 3, device=d), torch.zeros(4, 5, device=d)),
    "mm dtype": lambda d: torch.mm(torch.zeros(2, 3, device=d), torch.zeros(3, 2, dtype=torch.float16, device=d)),
    "addmm shape": lambda d: torch.addmm(torch.zeros(2, 5, device=d), torch.zeros(2, 3, device=d), torch.zeros(4, 5, device=d)),
    "addmm 1d": lambda d: torch.addmm(torch.zeros(2, 5, device=d), torch.zeros(3, device=d), torch.zeros(4, 5, device=d)),
    "bmm 2d": lambda d: torch.bmm(torch.zeros(2, 3, device=d), torch.zeros(1, 3, 2, device=d)),
    "bmm shape": lambda d: torch.bmm(torch.zeros(2, 3, 4, device=d), torch.zeros(2, 5, 2, device=d)),
    "bmm dtype": lambda d: torch.bmm(torch.zeros(2, 3, 4, device=d), torch.zeros(2, 4, 2, dtype=torch.float16, device=d)),
    "baddbmm dtype": lambda d: torch.baddbmm(torch.zeros(2, 3, 2, dtype=torch.float16, device=d),
                                             torch.zeros(2, 3, 4, device=d), torch.zeros(2, 4, 2, device=d)),
}


@pytest.mark.parametrize("case", list(ERROR_CASES))
def test_errors_match_cpu(tv, case):
    # the device rejects exactly what the CPU rejects, with the same message
    msgs = []
    for dev in ("cpu", V):
        with pytest.raises(RuntimeError) as e:
            ERROR_CASES[case](dev)
        msgs.append(str(e.value).splitlines()[0])
    assert msgs[0] == msgs[1]


def test_linear_forward_backward(tv):
    torch.manual_seed(0)
    lin = torch.nn.Linear(256, 128)
    x = torch.randn(64, 256)
    lin_v = torch.nn.Linear(256, 128).to(V)
    with torch.no_grad():
        lin_v.weight.copy_(lin.weight.to(V))
        lin_v.bias.copy_(lin.bias.to(V))
    y = lin(x)
    yv = lin_v(x.to(V))
    assert_close(host(yv).detach().numpy(), y.detach().numpy(), torch.float32, "linear fwd")
    g = torch.randn(64, 128)
    y.backward(g)
    yv.backward(g.to(V))
    assert_close(host(lin_v.weight.grad).numpy(), lin.weight.grad.numpy(), torch.float32, "dW")
    assert_close(host(lin_v.bias.grad).numpy(), lin.bias.grad.numpy(), torch.float32, "db")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_conv2d_forward_backward(tv, dtype):
    x = torch.randn((4, 8, 13, 11), generator=gen(40)).to(dtype)
    w = (torch.randn((16, 8, 3, 3), generator=gen(41)) * 0.2).to(dtype)
    b = torch.randn((16,), generator=gen(42)).to(dtype)
    xv = x.to(V).requires_grad_()
    wv = w.to(V).requires_grad_()
    y = F.conv2d(xv, wv, b.to(V), stride=2, padding=1)
    od = ORC_DT[dtype]
    ref = decode(orc.conv2d(to_np(x), to_np(w), od, bias=to_np(b), stride=(2, 2), padding=(1, 1)), dtype)
    assert_close(decode(to_np(host(y.detach())), dtype), ref, dtype, "conv2d fwd")
    dy = torch.randn(tuple(y.shape), generator=gen(43)).to(dtype)
    y.backward(dy.to(V))
    ref_dx = decode(orc.conv2d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, (2, 2), (1, 1)), dtype)
    ref_dw = decode(orc.conv2d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, (2, 2), (1, 1)), dtype)
    assert_close(decode(to_np(host(xv.grad)), dtype), ref_dx, dtype, "conv2d dgrad")
    assert_close(decode(to_np(host(wv.grad)), dtype), ref_dw, dtype, "conv2d wgrad")


def test_conv_transpose2d(tv):
    x = torch.randn((2, 6, 7, 5), generator=gen(50))
    w = torch.randn((6, 4, 3, 3), generator=gen(51)) * 0.3
    got = F.conv_transpose2d(x.to(V), w.to(V), stride=2, padding=1, output_padding=1)
    ref = F.conv_transpose2d(x.double(), w.double(), stride=2, padding=1, output_padding=1).numpy()
    assert got.shape == ref.shape
    assert_close(host(got).numpy(), ref, torch.float32, "conv_transpose2d")


def test_memory_statistics_and_strict_mode(tv):
    tv.synchronize()
    before = tv.memory_allocated()
    t = torch.empty((1024, 1024), dtype=torch.float32, device=V)
    assert tv.memory_allocated() >= before + t.numel() * 4
    assert tv.max_memory_allocated() >= tv.memory_allocated()
    free, total = tv.mem_get_info()
    assert 0 < free <= total
    del t
    tv.empty_cache()
    os.environ["TORCHVULKAN_STRICT"] = "1"
    try:
        with pytest.raises(RuntimeError, match="NOT IMPLEMENTED"):
            torch.sin(torch.zeros(4, device=V))
    finally:
        os.environ["TORCHVULKAN_STRICT"] = "0"
