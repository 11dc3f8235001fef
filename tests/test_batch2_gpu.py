"""Two batch dimensions (tvk_gemm_desc.batch_inner): [B, H, rows, cols]
operands whose B and H strides do not merge into one, such as the head-strided
q, k and v of a transformer layer ([B, L, H, D] underneath), run as one product
of batch B*H without a copy.

- Through the C ABI, on every kernel family the descriptor can reach: the
  LDS-ring tiles (fp16/bf16), the register-staged tiles, the sequential-order
  float32 kernel (bit-identical to the oracle), the M <= 16 streaming kernel,
  split-K, and the float64 wide kernel, with a bias broadcast over one batch
  dimension.
- Through torch.matmul on the vulkan device: the C3 attention products QK^T and
  PV on [B, H, L, D] head-strided views at the full batch (32 sequences x 8
  heads) against float64 and the oracle, with no copy on the way (the CPU
  profiler sees no aten::copy_ / clone), and with autograd (torch's composite
  takes over when a gradient is needed).

Tolerances: tests/gemm_cases.py.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from tests.gemm_cases import assert_bit_exact, assert_close, gen, oracle_mm

pytestmark = pytest.mark.gpu

DEV = "cuda"
V = "vulkan"


def _head_strided(B, L, H, D, dtype, seed, std=1.0):
    """[B, H, L, D] view of a [B, L, H, D] projection (the layout torch's attention meets)."""
    t = (torch.randn((B, L, H, D), generator=gen(seed)) * std).to(dtype)
    return t, t.permute(0, 2, 1, 3)


def _oracle4(a4, b4, dtype, bias4=None, beta=0.0, alpha=1.0):
    """The oracle per (b, h) matrix, stacked to [B, H, M, N]."""
    B, H = a4.shape[:2]
    out = []
    for i in range(B):
        row = []
        for j in range(H):
            bias = None if bias4 is None else bias4[i, j]
            row.append(oracle_mm(a4[i, j], b4[i, j], dtype, bias=bias, beta=beta, alpha=alpha))
        out.append(np.stack(row))
    return np.stack(out)


@pytest.fixture
def fresh_table():
    from torchvulkan_amd import _abi

    _abi.tune_reset()
    yield
    _abi.tune_reset()


@pytest.mark.parametrize("dtype,M,N,K", [
    (torch.float16, 256, 256, 64),     # QK^T of one layer's heads
    (torch.bfloat16, 256, 64, 256),    # PV
    (torch.float16, 72, 40, 56),       # K off the 32 grid
    (torch.float32, 96, 80, 48),       # sequential order: bit-exact
    (torch.float16, 8, 512, 1024),     # M <= 16 streaming kernel
    (torch.float16, 128, 128, 4096),   # split-K partials over the flat batch
], ids=["fp16-qk", "bf16-pv", "fp16-kodd", "fp32-seq", "fp16-skinny", "fp16-splitk"])
def test_abi_two_batch_dims_every_kernel(gpu, fresh_table, dtype, M, N, K):
    """Every candidate kernel of the product (recorded one at a time in the kernel-choice table) on
    [B, H, M, K] x [B, H, K, N] head-strided operands with a bias broadcast over B and the rows."""
    B, H = 3, 4
    # A: [B, M, H, K] underneath -> [B, H, M, K] view; B operand: [B, K, H, N] -> [B, H, K, N]
    a_base = torch.randn((B, M, H, K), generator=gen(1)).to(dtype)
    b_base = torch.randn((B, K, H, N), generator=gen(2)).to(dtype)
    bias = torch.randn((H, 1, N), generator=gen(3)).to(dtype)
    a4 = a_base.to(DEV).permute(0, 2, 1, 3)
    b4 = b_base.to(DEV).permute(0, 2, 1, 3)
    bias_d = bias.to(DEV)
    ref = _oracle4(a_base.permute(0, 2, 1, 3), b_base.permute(0, 2, 1, 3), dtype,
                   bias4=bias.expand(B, H, M, N), beta=0.5, alpha=2.0)
    kw = dict(bias=bias_d, beta=0.5, alpha=2.0)
    names = gpu.gemm_candidates(a4, b4, torch.empty((B, H, M, N), dtype=dtype, device=DEV), **kw)
    assert len(names) >= 2 or dtype == torch.float32, names
    for name in names:
        c4 = torch.full((B, H, M, N), float("nan"), dtype=dtype, device=DEV)
        gpu.tune_reset()
        gpu.gemm_choose(a4, b4, c4, name, **kw)
        print(f"{dtype} {M}x{N}x{K}: {name}", flush=True)
        gpu.gemm(a4, b4, c4, **kw)
        torch.cuda.synchronize()
        got = c4.cpu().float().numpy()
        if dtype == torch.float32:
            assert_bit_exact(got, ref, f"{name}, two batch dims")
        else:
            assert_close(got, ref, dtype, f"{name}, two batch dims")


def test_abi_two_batch_dims_float64(gpu):
    B, H, M, N, K = 2, 3, 33, 17, 29
    a_base = torch.randn((B, M, H, K), generator=gen(4), dtype=torch.float64)
    b_base = torch.randn((B, K, H, N), generator=gen(5), dtype=torch.float64)
    a4, b4 = a_base.to(DEV).permute(0, 2, 1, 3), b_base.to(DEV).permute(0, 2, 1, 3)
    c4 = torch.empty((B, H, M, N), dtype=torch.float64, device=DEV)
    assert gpu.gemm_plan(a4, b4, c4) == "gemm_wide_f64"
    gpu.gemm(a4, b4, c4)
    torch.cuda.synchronize()
    ref = torch.matmul(a_base.permute(0, 2, 1, 3), b_base.permute(0, 2, 1, 3))
    assert torch.allclose(c4.cpu(), ref, rtol=1e-13, atol=1e-13)


def test_abi_rejects_bad_inner_batch(gpu):
    a = torch.zeros((6, 8, 8), dtype=torch.float16, device=DEV)
    d = gpu.make_gemm_desc(a, a, a)
    d.batch_inner = 4   # does not divide 6
    assert gpu.load().tvk_gemm(gpu.C.byref(d)) == gpu.TVK_ERR_INVALID


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


def _copies(fn):
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CPU]) as prof:
        out = fn()
    names = [e.name for e in prof.events()]
    return out, [n for n in names if n in ("aten::copy_", "aten::clone", "aten::contiguous", "aten::_reshape_copy")]


def test_c3_matmul_head_strided_full_batch(gpu, strict):
    """QK^T and PV of the C3 config through torch.matmul on [B, H, L, D] views: one product each, no copies."""
    import torchvulkan_amd  # noqa: F401

    B, L, H, D = 32, 256, 8, 64
    f16 = torch.float16
    q, q4 = _head_strided(B, L, H, D, f16, 10)
    k, k4 = _head_strided(B, L, H, D, f16, 11)
    v, v4 = _head_strided(B, L, H, D, f16, 12)
    qv, kv, vv = (t.to(V).permute(0, 2, 1, 3) for t in (q, k, v))
    with torch.no_grad():
        s, cp1 = _copies(lambda: torch.matmul(qv, kv.transpose(-1, -2)))
        p = (torch.randn((B, H, L, L), generator=gen(13)) * 0.1).to(f16)
        pv = p.to(V)
        o, cp2 = _copies(lambda: torch.matmul(pv, vv))
    assert not cp1 and not cp2, (cp1, cp2)
    got_s, got_o = s.cpu().float().numpy(), o.cpu().float().numpy()
    ref_s = torch.matmul(q4.double(), k4.double().transpose(-1, -2)).numpy()
    ref_o = torch.matmul(p.double(), v4.double()).numpy()
    assert_close(got_s, ref_s, f16, "QK^T every head vs float64")
    assert_close(got_o, ref_o, f16, "PV every head vs float64")
    for b in (0, 17, 31):
        for h in (0, 5):
            assert_close(got_s[b, h], oracle_mm(q4[b, h], k4[b, h].transpose(0, 1), f16), f16, f"QK^T {b},{h} vs oracle")
            assert_close(got_o[b, h], oracle_mm(p[b, h], v4[b, h], f16), f16, f"PV {b},{h} vs oracle")


def test_matmul_broadcast_and_autograd(gpu, strict):
    """torch.matmul's other shapes on the device (1-D operands, broadcast batches), and its gradients."""
    import torchvulkan_amd  # noqa: F401

    f32 = torch.float32
    x = torch.randn((2, 3, 5, 7), generator=gen(20))
    w = torch.randn((7, 4), generator=gen(21))
    vec = torch.randn((7,), generator=gen(22))
    with torch.no_grad():
        for a, b in ((x, w), (x, vec), (vec, w), (vec, vec), (x[0, 0], w), (x, torch.randn((3, 7, 2), generator=gen(23)))):
            got = torch.matmul(a.to(V), b.to(V)).cpu()
            ref = torch.matmul(a.double(), b.double())
            assert got.shape == ref.shape, (a.shape, b.shape)
            assert torch.allclose(got.double(), ref, rtol=1e-5, atol=1e-5)
    # a head-strided product under autograd: the composite's reshape + bmm, gradients included
    q, q4 = _head_strided(2, 16, 4, 8, f32, 24)
    k, k4 = _head_strided(2, 16, 4, 8, f32, 25)
    qv = q.to(V).requires_grad_()
    kv = k.to(V).requires_grad_()
    s = torch.matmul(qv.permute(0, 2, 1, 3), kv.permute(0, 2, 3, 1))
    gs = torch.randn(tuple(s.shape), generator=gen(26))
    s.backward(gs.to(V))
    qd, kd = q.double().requires_grad_(), k.double().requires_grad_()
    torch.matmul(qd.permute(0, 2, 1, 3), kd.permute(0, 2, 3, 1)).backward(gs.double())
    assert torch.allclose(s.detach().cpu().double(), torch.matmul(q4.double(), k4.double().transpose(-1, -2)), rtol=1e-5, atol=1e-5)
    assert torch.allclose(qv.grad.cpu().double(), qd.grad, rtol=1e-5, atol=1e-5)
    assert torch.allclose(kv.grad.cpu().double(), kd.grad, rtol=1e-5, atol=1e-5)
