"""A transformer layer trained through the vulkan device: the products, the
fused causal GQA attention (forward and backward), the residual adds, the
element-wise product and the float32 loss sum all run on the device under
TORCHVULKAN_STRICT=1 (any CPU fallback raises), and the loss and every weight
gradient match the same layer computed by torch on the CPU in float64 from the
same float16 parameters.

Layer (the C3 config's, at 2 sequences of 128 tokens): q, k, v projections
(8 query and 2 key/value heads of 64), causal attention with enable_gqa, out
projection + residual, gate * up (SwiGLU without its SiLU, which is not on the
path), down projection + residual; loss = sum(float32).

Tolerance: float16 storage of every intermediate (the float64 reference keeps
none) gives relative errors of a few float16 steps per stage; each gradient is
held to 3e-2 of its largest magnitude, which a dropped term, a transposed
product or a wrong head mapping exceeds by far.
"""
from __future__ import annotations

import os

import pytest
import torch
import torch.nn.functional as F

from tests.gemm_cases import gen

pytestmark = pytest.mark.gpu

V = "vulkan"
Bs, Ls, DM, HQ, HKV, DH, FF = 2, 128, 512, 8, 2, 64, 1536


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


def _layer(x, w, sdpa):
    q = F.linear(x, w["q"]).view(Bs, Ls, HQ, DH).transpose(1, 2)
    k = F.linear(x, w["k"]).view(Bs, Ls, HKV, DH).transpose(1, 2)
    v = F.linear(x, w["v"]).view(Bs, Ls, HKV, DH).transpose(1, 2)
    a = sdpa(q, k, v)
    h = x + F.linear(a.transpose(1, 2).reshape(Bs * Ls, HQ * DH), w["o"])
    y = h + F.linear(F.linear(h, w["gate"]) * F.linear(h, w["up"]), w["down"])
    return y.float().sum()


def test_transformer_layer_autograd_on_device(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    shapes = {"q": (HQ * DH, DM), "k": (HKV * DH, DM), "v": (HKV * DH, DM), "o": (DM, HQ * DH),
              "gate": (FF, DM), "up": (FF, DM), "down": (DM, FF)}
    w16 = {n: (torch.randn(s, generator=gen(40 + i)) * 0.02).to(torch.float16) for i, (n, s) in enumerate(shapes.items())}
    x16 = torch.randn((Bs * Ls, DM), generator=gen(60)).to(torch.float16)

    wv = {n: t.to(V).requires_grad_() for n, t in w16.items()}
    loss = _layer(x16.to(V), wv, lambda q, k, v: F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True))
    loss.backward()

    wr = {n: t.double().requires_grad_() for n, t in w16.items()}

    def ref_sdpa(q, k, v):
        rep = HQ // HKV
        k, v = k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)
        s = (q @ k.transpose(-1, -2)) / DH ** 0.5
        mask = torch.ones((Ls, Ls), dtype=torch.bool).triu(1)
        return torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1) @ v

    ref = _layer(x16.double(), wr, ref_sdpa)
    ref.backward()
    got, want = float(loss.detach().cpu()), float(ref.detach())
    assert abs(got - want) <= 3e-2 * max(1.0, abs(want)), (got, want)
    for n in shapes:
        g = wv[n].grad.cpu().double()
        r = wr[n].grad
        scale = float(r.abs().max())
        err = float((g - r).abs().max())
        assert err <= 3e-2 * scale, f"grad {n}: max error {err:.3e} against max |grad| {scale:.3e}"
