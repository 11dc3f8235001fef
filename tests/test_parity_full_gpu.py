"""Parity at the configs' full sizes.

- C4 ResNet layers (batch 128, float16): forward and grad input on EVERY image
  against torch's float64 convolution of the same float16 inputs (within the
  float16 tolerance), the oracle (the reference's rounding) on images spread
  across the batch, the last image (the batch's last tile) included, and the
  per-image channel sums of the forward against float64 sums.
- C3 head-strided QK^T and PV at the full batch of 32 sequences x 8 heads:
  every head against torch's float64 products, the oracle on a spread of heads.
- float16 autograd through the vulkan device at C2 and C4 shapes: nn.Linear
  (256 x 4096 -> 4096) and F.conv2d (64 -> 64, 3x3, batch 128) forward and
  backward against the oracle (and, for the bias gradient, a float64 sum).
- The C3 layer's backward products at full size (8192 tokens), as nn.Linear's
  backward forms them: dX = dY.W and dW = dY^T.X for every projection, every
  element against float64, rows spread over every 128-row tile against the
  oracle.
- The C2 10-output layer's backward: dX with K = 10, dW on the M <= 16
  streaming kernel, every element against the oracle; and the same layer
  under autograd with loss sum() (a gradient with stride 0 in both dims).

Tolerances are the ones gemm_cases.py states: |got - ref| <= 5e-3 (|ref| + 1)
for float16. Against float64 the float16 result also carries its own
rounding, which the same bound covers (one float16 step is 2^-11 relative).
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

DEV = "cuda"
V = "vulkan"
F16 = torch.float16

C4 = [
    # name, cin, cout, k, stride, pad, spatial
    ("stem_3_64", 3, 64, 3, 1, 1, 32),
    ("3x3_64_64", 64, 64, 3, 1, 1, 32),
    ("3x3_64_128_s2", 64, 128, 3, 2, 1, 32),
    ("3x3_128_256_s2", 128, 256, 3, 2, 1, 16),
    ("1x1_64_128_s2", 64, 128, 1, 2, 0, 32),
    ("1x1_128_256_s2", 128, 256, 1, 2, 0, 16),
]
SPREAD = [0, 37, 64, 101, 127]   # images checked against the oracle (127: the last tile)


def _rand(shape, seed, std=1.0):
    return (torch.randn(shape, generator=gen(seed)) * std).to(F16)


@pytest.mark.parametrize("layer", C4, ids=[c[0] for c in C4])
def test_c4_full_batch(gpu, layer):
    _, cin, cout, k, s, p, hw = layer
    n = 128
    x = _rand((n, cin, hw, hw), 70)
    w = _rand((cout, cin, k, k), 71, std=(2.0 / (cin * k * k)) ** 0.5)
    bias = _rand((cout,), 72)
    y = gpu.conv2d_fwd(x.to(DEV), w.to(DEV), bias.to(DEV), s, p, 1, 1)
    dy = _rand(tuple(y.shape), 73)
    gx = gpu.conv2d_dgrad(dy.to(DEV), w.to(DEV), x.shape, s, p, 1, 1)
    torch.cuda.synchronize()
    got_y, got_gx = y.cpu().float().numpy(), gx.cpu().float().numpy()
    # every image: float64 mathematics of the same float16 inputs
    ref_y = F.conv2d(x.double(), w.double(), bias.double(), stride=s, padding=p).numpy()
    ref_gx = torch.nn.grad.conv2d_input(x.shape, w.double(), dy.double(), stride=s, padding=p).numpy()
    assert_close(got_y, ref_y, F16, "fwd, every image vs float64")
    assert_close(got_gx, ref_gx, F16, "dgrad, every image vs float64")
    # per-image channel sums: a tile written to the wrong image or left unwritten moves a whole sum
    sums = got_y.astype(np.float64).sum(axis=(2, 3))
    ref_sums = ref_y.sum(axis=(2, 3))
    assert np.abs(sums - ref_sums).max() <= 5e-3 * (np.abs(ref_y).sum(axis=(2, 3)).max() + hw * hw)
    # spread images: the oracle's own rounding
    idx = torch.tensor(SPREAD)
    od = ORC_DT[F16]
    oy = decode(orc.conv2d(to_np(x[idx]), to_np(w), od, bias=to_np(bias), stride=(s, s), padding=(p, p)), F16)
    ogx = decode(orc.conv2d_dgrad(to_np(dy[idx]), to_np(w), (len(SPREAD),) + tuple(x.shape[1:]), od, (s, s), (p, p),
                                  (1, 1), 1), F16)
    assert_close(got_y[SPREAD], oy, F16, "fwd, spread images vs oracle")
    assert_close(got_gx[SPREAD], ogx, F16, "dgrad, spread images vs oracle")


def _device_view(t: torch.Tensor) -> torch.Tensor:
    base = t.as_strided((t.untyped_storage().nbytes() // t.element_size(),), (1,), 0).to(DEV)
    return base.as_strided(t.shape, t.stride(), t.storage_offset())


def test_c3_head_strided_full_batch(gpu):
    B, L, H, D = 32, 256, 8, 64
    q = _rand((B * L, H * D), 80)
    k = _rand((B * L, H * D), 81)
    v = _rand((B * L, H * D), 82)
    # [B*H, L, D] views of the [B*L, H*D] projections (no copies)
    q4 = q.view(B, L, H, D).permute(0, 2, 1, 3)   # [B, H, L, D]
    k4 = k.view(B, L, H, D).permute(0, 2, 3, 1)   # [B, H, D, L]
    v4 = v.view(B, L, H, D).permute(0, 2, 1, 3)
    s_ = torch.empty((B, H, L, L), dtype=F16, device=DEV)
    o_ = torch.empty((B, H, L, D), dtype=F16, device=DEV)
    qd, kd, vd = _device_view(q4), _device_view(k4), _device_view(v4)
    for b in range(B):   # one strided batched product per sequence: [H, L, D] x [H, D, L]
        gpu.gemm(qd[b], kd[b], s_[b])
    pm = _rand((B, H, L, L), 83, std=0.1)
    pd = pm.to(DEV)
    for b in range(B):
        gpu.gemm(pd[b], vd[b], o_[b])
    torch.cuda.synchronize()
    got_s, got_o = s_.cpu().float().numpy(), o_.cpu().float().numpy()
    ref_s = torch.matmul(q4.double(), k4.double()).numpy()
    ref_o = torch.matmul(pm.double(), v4.double()).numpy()
    assert_close(got_s, ref_s, F16, "QK^T, every head of every sequence vs float64")
    assert_close(got_o, ref_o, F16, "PV, every head of every sequence vs float64")
    for b in (0, 13, 31):
        assert_close(got_s[b], oracle_mm(q4[b], k4[b], F16), F16, f"QK^T sequence {b} vs oracle")
        assert_close(got_o[b], oracle_mm(pm[b], v4[b], F16), F16, f"PV sequence {b} vs oracle")


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


def test_c2_linear_autograd_fp16(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    torch.manual_seed(0)
    lin = torch.nn.Linear(4096, 4096).to(F16)
    x = _rand((256, 4096), 90)
    dy = _rand((256, 4096), 91)
    lv = torch.nn.Linear(4096, 4096).to(F16).to(V)
    with torch.no_grad():
        lv.weight.copy_(lin.weight.to(V))
        lv.bias.copy_(lin.bias.to(V))
    xv = x.to(V).requires_grad_()
    y = lv(xv)
    y.backward(dy.to(V))
    W, b = lin.weight.detach(), lin.bias.detach()
    assert_close(y.detach().cpu().float().numpy(), oracle_mm(x, W.t(), F16, bias=b, beta=1.0), F16, "Linear forward")
    assert_close(xv.grad.cpu().float().numpy(), oracle_mm(dy, W, F16), F16, "Linear grad input")
    assert_close(lv.weight.grad.cpu().float().numpy(), oracle_mm(dy.t(), x, F16), F16, "Linear grad weight")
    db = dy.double().sum(0).numpy()
    assert_close(lv.bias.grad.cpu().float().numpy(), db, F16, "Linear grad bias vs float64 sum")


def test_c4_conv_autograd_fp16(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    n, cin, cout, hw = 128, 64, 64, 32
    x = _rand((n, cin, hw, hw), 92)
    w = _rand((cout, cin, 3, 3), 93, std=(2.0 / (cin * 9)) ** 0.5)
    bias = _rand((cout,), 94)
    dy = _rand((n, cout, hw, hw), 95)
    xv, wv, bv = (t.to(V).requires_grad_() for t in (x, w, bias))
    y = F.conv2d(xv, wv, bv, stride=1, padding=1)
    y.backward(dy.to(V))
    idx = torch.tensor(SPREAD)
    od = ORC_DT[F16]
    oy = decode(orc.conv2d(to_np(x[idx]), to_np(w), od, bias=to_np(bias), stride=(1, 1), padding=(1, 1)), F16)
    assert_close(y.detach().cpu()[idx].float().numpy(), oy, F16, "conv2d forward vs oracle")
    ogx = decode(orc.conv2d_dgrad(to_np(dy[idx]), to_np(w), (len(SPREAD), cin, hw, hw), od, (1, 1), (1, 1), (1, 1), 1), F16)
    assert_close(xv.grad.cpu()[idx].float().numpy(), ogx, F16, "conv2d grad input vs oracle")
    ogw = decode(orc.conv2d_wgrad(to_np(x), to_np(dy), (cout, cin, 3, 3), od, (1, 1), (1, 1), (1, 1), 1, acc64=True), F16)
    assert_close(wv.grad.cpu().float().numpy(), ogw, F16, "conv2d grad weight vs oracle")
    db = dy.double().sum((0, 2, 3)).numpy()
    assert_close(bv.grad.cpu().float().numpy(), db, F16, "conv2d grad bias vs float64 sum")


C3_LINEARS = [(512, 512), (512, 256), (512, 3072), (1536, 512), (512, 96)]   # (in, out): q, kv, gate_up, down, head


@pytest.mark.parametrize("fin,fout", C3_LINEARS, ids=[f"{a}to{b}" for a, b in C3_LINEARS])
def test_c3_backward_products_full(gpu, fin, fout):
    T = 8192
    dy = _rand((T, fout), 100 + fout)
    x = _rand((T, fin), 200 + fin)
    w = _rand((fout, fin), 300 + fin + fout, std=0.02)
    dyd, wd, xd = dy.to(DEV), w.to(DEV), x.to(DEV)
    dx = torch.empty((T, fin), dtype=F16, device=DEV)
    dw = torch.empty((fout, fin), dtype=F16, device=DEV)
    gpu.gemm(dyd, wd, dx)            # dX = dY . W: B [out, in] row-major (n-contiguous), K = out
    gpu.gemm(dyd.t(), xd, dw)        # dW = dY^T . X: A an m-contiguous view, K = 8192 tokens
    torch.cuda.synchronize()
    plans = (gpu.gemm_plan(dyd, wd, dx), gpu.gemm_plan(dyd.t(), xd, dw))
    got_dx, got_dw = dx.cpu().float().numpy(), dw.cpu().float().numpy()
    assert_close(got_dx, (dy.double() @ w.double()).numpy(), F16, f"dX {plans[0]} vs float64")
    assert_close(got_dw, (dy.double().t() @ x.double()).numpy(), F16, f"dW {plans[1]} vs float64")
    rows = np.r_[0:T:97, T - 1]        # at least one row of every 128-row tile, and the last
    assert_close(got_dx[rows], oracle_mm(dy[rows], w, F16), F16, f"dX {plans[0]} vs oracle")
    wrows = np.r_[0:fout:7, fout - 1]
    assert_close(got_dw[wrows], oracle_mm(dy.t()[wrows], x, F16), F16, f"dW {plans[1]} vs oracle")


def test_c2_last_layer_backward(gpu):
    g = torch.Generator().manual_seed(120)
    dy = torch.randn((256, 10), generator=g).to(F16)
    w = (torch.randn((10, 4096), generator=g) * 0.02).to(F16)
    x = torch.rand((256, 4096), generator=g).to(F16)
    dyd, wd, xd = dy.to(DEV), w.to(DEV), x.to(DEV)
    dx = torch.empty((256, 4096), dtype=F16, device=DEV)
    dw = torch.empty((10, 4096), dtype=F16, device=DEV)
    gpu.gemm(dyd, wd, dx)            # K = 10: one partial k step
    gpu.gemm(dyd.t(), xd, dw)        # M = 10: the streaming kernel
    torch.cuda.synchronize()
    assert gpu.gemm_plan(dyd.t(), xd, dw).startswith("gemm16_skinny"), gpu.gemm_plan(dyd.t(), xd, dw)
    assert_close(dx.cpu().float().numpy(), oracle_mm(dy, w, F16), F16, "dX, K = 10")
    assert_close(dw.cpu().float().numpy(), oracle_mm(dy.t(), x, F16), F16, "dW, M = 10")


def test_c2_last_layer_autograd_sum_loss(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    torch.manual_seed(1)
    lin = torch.nn.Linear(4096, 10).to(F16)
    x = torch.rand((256, 4096), generator=gen(121)).to(F16)
    lv = torch.nn.Linear(4096, 10).to(F16).to(V)
    with torch.no_grad():
        lv.weight.copy_(lin.weight.to(V))
        lv.bias.copy_(lin.bias.to(V))
    xv = x.to(V).requires_grad_()
    y = lv(xv)
    y.sum().backward()               # the gradient reaches the products as ones expanded with stride 0
    W, b = lin.weight.detach(), lin.bias.detach()
    ones = torch.ones((256, 10), dtype=F16)
    assert_close(y.detach().cpu().float().numpy(), oracle_mm(x, W.t(), F16, bias=b, beta=1.0), F16, "forward")
    assert_close(xv.grad.cpu().float().numpy(), oracle_mm(ones, W, F16), F16, "grad input")
    assert_close(lv.weight.grad.cpu().float().numpy(), oracle_mm(ones.t(), x, F16), F16, "grad weight")
    assert torch.equal(lv.bias.grad.cpu(), torch.full((10,), 256.0, dtype=F16)), "grad bias"

