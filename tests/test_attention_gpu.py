"""tvk_attention_fwd / tvk_attention_bwd on the GPU through the C ABI against
the float64 attention oracle, at the north_star tolerance for float16/bfloat16
(5e-3*(|ref|+1) on out and on dq, dk, dv; lse within 1e-3*(|lse|+1)). For
bfloat16 the GEMM tests' rule applies: one bfloat16 step (2^-7 relative) is
larger than that bound above |ref| ~ 0.7, so an element may sit one step away,
on at most 1% of the elements. Also
F.scaled_dot_product_attention on the vulkan device (forward and backward)
against torch's CPU math attention in float64."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.gemm_cases import assert_close
from torchvulkan_amd import _abi

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def f64(t):
    return t.detach().cpu().double().numpy()


def check(q, k, v, bias=None, causal=False, scale=None, what=""):
    out, lse = _abi.attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), None if bias is None else bias.to(DEV), causal, scale)
    torch.cuda.synchronize()
    ro, rl = orc.attention(f64(q), f64(k), f64(v), None if bias is None else f64(bias), causal, scale)
    go, gl = f64(out), lse.cpu().double().numpy()
    assert_close(go, ro, q.dtype, f"{what}: out")
    fin = np.isfinite(rl)
    assert (np.isinf(gl) == ~fin).all(), f"{what}: +inf lse rows differ"
    lerr = np.abs(gl[fin] - rl[fin]) / (1e-3 * (np.abs(rl[fin]) + 1))
    assert lerr.size == 0 or lerr.max() <= 1.0, f"{what}: lse off by {lerr.max():.2f}x tolerance"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_transformer_shape(gpu, dtype, causal):
    # the C3 attention at a reduced batch: 8 query heads over 2 kv heads, head_dim 64, seq 256
    q, k, v = rand((2, 8, 256, 64), dtype, 1), rand((2, 2, 256, 64), dtype, 2), rand((2, 2, 256, 64), dtype, 3)
    check(q, k, v, causal=causal, what=f"{dtype} causal={causal}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ragged_lengths_and_head_dim_128(gpu, dtype):
    q, k, v = rand((1, 4, 100, 128), dtype, 4), rand((1, 4, 301, 128), dtype, 5), rand((1, 4, 301, 128), dtype, 6)
    check(q, k, v, what="L 100 S 301 D 128")
    check(q, k, v, causal=True, what="causal L 100 S 301")
    q2 = rand((1, 2, 300, 64), dtype, 7)
    k2, v2 = rand((1, 2, 70, 64), dtype, 8), rand((1, 2, 70, 64), dtype, 9)
    check(q2, k2, v2, causal=True, scale=0.2, what="causal L 300 > S 70")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_wide_grid_two_query_columns_per_wave(gpu, dtype, causal):
    # batch*heads*ceil(L/128) >= 2048 selects 128-query workgroups (two 16-query
    # columns per wave); the oracle checks a few (batch, head) slices
    B, Hq, Hk, L, D = 16, 16, 4, 1024, 64
    q, k, v = rand((B, Hq, L, D), dtype, 60), rand((B, Hk, L, D), dtype, 61), rand((B, Hk, L, D), dtype, 62)
    out, lse = _abi.attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), None, causal)
    torch.cuda.synchronize()
    out, lse = f64(out), lse.cpu().double().numpy()
    for b, h in ((0, 0), (5, 9), (15, 15)):
        hk = h // (Hq // Hk)
        ro, rl = orc.attention(f64(q[b:b + 1, h:h + 1]), f64(k[b:b + 1, hk:hk + 1]), f64(v[b:b + 1, hk:hk + 1]),
                               None, causal)
        assert_close(out[b:b + 1, h:h + 1], ro, dtype, f"b {b} h {h}: out")
        assert (np.abs(lse[b:b + 1, h:h + 1] - rl) <= 1e-3 * (np.abs(rl) + 1)).all(), f"b {b} h {h}: lse"


@pytest.mark.parametrize("causal", [False, True])
def test_negative_and_zero_scale(gpu, causal):
    dtype = torch.float16
    q, k, v = rand((2, 4, 130, 64), dtype, 63), rand((2, 4, 130, 64), dtype, 64), rand((2, 4, 130, 64), dtype, 65)
    check(q, k, v, causal=causal, scale=-0.3, what=f"scale -0.3 causal={causal}")
    check(q, k, v, causal=causal, scale=0.0, what=f"scale 0 causal={causal}")


def test_bias_broadcast_and_masked_rows(gpu):
    dtype = torch.float16
    q, k, v = rand((2, 4, 64, 64), dtype, 10), rand((2, 4, 96, 64), dtype, 11), rand((2, 4, 96, 64), dtype, 12)
    bias = rand((1, 4, 64, 96), dtype, 13)
    check(q, k, v, bias=bias, what="bias broadcast over batch")
    mask = torch.zeros((2, 1, 64, 96), dtype=dtype)
    mask[:, :, 5] = float("-inf")            # row 5 attends to nothing: out 0, lse +inf
    mask[:, :, 9, 1:] = float("-inf")        # row 9 attends to key 0 only
    check(q, k, v, bias=mask, what="masked rows")


def test_head_strided_views(gpu):
    # q, k, v as [B, L, H, D] underneath (the projection output split into heads)
    dtype = torch.float16
    x = rand((2, 128, 8, 64), dtype, 14).to(DEV)
    kv = rand((2, 128, 2, 64), dtype, 15).to(DEV)
    q, k, v = x.transpose(1, 2), kv.transpose(1, 2), (kv * 0.5).transpose(1, 2)
    check(q.cpu(), k.cpu(), v.cpu(), what="dense reference")
    out, lse = _abi.attention_fwd(q, k, v, None, True)
    torch.cuda.synchronize()
    ro, _ = orc.attention(f64(q), f64(k), f64(v), None, True)
    assert (np.abs(f64(out) - ro) <= 5e-3 * (np.abs(ro) + 1)).all()


def test_rejects_unsupported(gpu):
    q = torch.zeros((1, 1, 8, 520), dtype=torch.float16, device=DEV)
    with pytest.raises(_abi.TvkUnsupported):
        _abi.attention_fwd(q, q, q)
    q64 = torch.zeros((1, 1, 8, 64), dtype=torch.float64, device=DEV)
    with pytest.raises(_abi.TvkUnsupported):
        _abi.attention_fwd(q64, q64, q64)


# The general kernels: float32, head dims other than 64/128 (query/key and value dims may
# differ), several 64-column chunks of the head dim, GQA, ragged and causal lengths, bias.
GENERAL_CASES = [
    # dtype, B, Hq, Hk, L, S, D, Dv, causal, bias
    (torch.float32, 2, 4, 2, 77, 130, 64, 64, False, False),
    (torch.float32, 1, 2, 2, 100, 100, 64, 64, True, True),
    (torch.float16, 1, 4, 1, 129, 65, 80, 80, False, True),
    (torch.float16, 2, 2, 2, 64, 200, 96, 48, True, False),
    (torch.bfloat16, 1, 2, 1, 50, 70, 32, 32, False, False),
    (torch.float16, 1, 2, 2, 40, 90, 200, 320, False, False),
    (torch.float32, 1, 1, 1, 33, 47, 512, 512, True, False),
]


def general_inputs(case, seed):
    dt, B, Hq, Hk, L, S, D, Dv, causal, with_bias = case
    q, k, v = rand((B, Hq, L, D), dt, seed), rand((B, Hk, S, D), dt, seed + 1), rand((B, Hk, S, Dv), dt, seed + 2)
    bias = rand((B, Hq, L, S), dt, seed + 3) if with_bias else None
    return q, k, v, bias, causal


@pytest.mark.parametrize("case", range(len(GENERAL_CASES)))
def test_general_forward(gpu, case):
    q, k, v, bias, causal = general_inputs(GENERAL_CASES[case], 100 + 10 * case)
    check(q, k, v, bias, causal, what=f"general case {case}")


@pytest.mark.parametrize("case", range(len(GENERAL_CASES)))
def test_general_backward(gpu, case):
    q, k, v, bias, causal = general_inputs(GENERAL_CASES[case], 200 + 10 * case)
    check_bwd(q, k, v, bias, causal, what=f"general case {case}")


def test_general_strided_views_float32(gpu):
    # projections split into heads ([B, L, H, D] underneath) and a head dim with stride 2
    x = rand((2, 96, 4, 128), torch.float32, 300).to(DEV)
    kv = rand((2, 80, 2, 64), torch.float32, 301).to(DEV)
    q, k, v = x.transpose(1, 2)[..., ::2], kv.transpose(1, 2), (kv * 0.5).transpose(1, 2)
    assert q.stride(3) == 2
    out, lse = _abi.attention_fwd(q, k, v, None, True)
    torch.cuda.synchronize()
    ro, rl = orc.attention(f64(q), f64(k), f64(v), None, True)
    assert_close(f64(out), ro, torch.float32, "strided float32 out")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_score_gradient(gpu, dtype):
    q, k, v = rand((2, 4, 70, 64), dtype, 400), rand((2, 2, 90, 64), dtype, 401), rand((2, 2, 90, 64), dtype, 402)
    bias = rand((2, 4, 70, 90), dtype, 403)
    bias[1, 2, 5] = float("-inf")         # a row that attends to nothing
    dev = [t.to(DEV) for t in (q, k, v)]
    out, lse = _abi.attention_fwd(*dev, bias.to(DEV), True)
    dout = rand(out.shape, dtype, 404)
    dq, dk, dv, ds = _abi.attention_bwd(*dev, out, lse, dout.to(DEV), bias.to(DEV), True, dscores=True)
    torch.cuda.synchronize()
    rdt = {torch.float16: orc.F16, torch.bfloat16: orc.BF16}.get(dtype)
    *ref, ref_ds = orc.attention_bwd(f64(q), f64(k), f64(v), f64(dout), f64(bias), True, None, out=f64(out),
                                     round_to=rdt, return_ds=True)
    for got, want, name in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert_close(f64(got), want, dtype, f"{dtype} {name} with the score gradient")
    # dS is float32 from float32 P and dP: held to the dtype's bound, masked entries exactly 0
    assert_close(f64(ds), ref_ds, dtype, f"{dtype} dS")
    assert (f64(ds)[:, :, np.arange(70)[:, None] < np.arange(90)[None, :]] == 0).all()


def test_sdpa_on_vulkan_device(gpu):
    import torchvulkan_amd  # noqa: F401

    V = "vulkan"
    dtype = torch.float16
    q, k, v = rand((2, 8, 128, 64), dtype, 20), rand((2, 2, 128, 64), dtype, 21), rand((2, 2, 128, 64), dtype, 22)
    qv, kv_, vv = (t.to(V).requires_grad_() for t in (q, k, v))
    out = F.scaled_dot_product_attention(qv, kv_, vv, is_causal=True, enable_gqa=True)
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    ref = F.scaled_dot_product_attention(q64, k64, v64, is_causal=True, enable_gqa=True)
    assert out.shape == ref.shape and out.dtype == dtype
    assert ((out.detach().cpu().double() - ref.detach()).abs() <= 5e-3 * (ref.detach().abs() + 1)).all()
    g = rand(out.shape, dtype, 23)
    out.backward(g.to(V))
    ref.backward(g.double())
    for got, want, name in ((qv.grad, q64.grad, "dq"), (kv_.grad, k64.grad, "dk"), (vv.grad, v64.grad, "dv")):
        assert got.shape == want.shape, name
        assert ((got.cpu().double() - want).abs() <= 5e-3 * (want.abs() + 1)).all(), name


def test_sdpa_training_step_strict(gpu, monkeypatch):
    # forward and backward both on the device kernels: strict mode would raise on any CPU fallback
    import torchvulkan_amd  # noqa: F401

    monkeypatch.setenv("TORCHVULKAN_STRICT", "1")
    V = "vulkan"
    q, k, v = (rand((1, 4, 64, 64), torch.float16, 50 + i).to(V).requires_grad_() for i in range(3))
    out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    out.backward(torch.ones_like(out))
    assert q.grad is not None and k.grad is not None and v.grad is not None


def check_bwd(q, k, v, bias=None, causal=False, scale=None, what=""):
    dev = [t.to(DEV) for t in (q, k, v)]
    db = None if bias is None else bias.to(DEV)
    out, lse = _abi.attention_fwd(*dev, db, causal, scale)
    dout = rand(out.shape, q.dtype, 99)
    dq, dk, dv = _abi.attention_bwd(*dev, out, lse, dout.to(DEV), db, causal, scale)
    torch.cuda.synchronize()
    # delta from the stored (dtype-rounded) forward output, and P, dS rounded to the dtype
    # before their products: the reference's cooperative-matrix backward
    rdt = {torch.float16: orc.F16, torch.bfloat16: orc.BF16}.get(q.dtype)
    ref = orc.attention_bwd(f64(q), f64(k), f64(v), f64(dout), None if bias is None else f64(bias), causal, scale,
                            out=f64(out), round_to=rdt)
    for got, want, name in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert_close(f64(got), want, q.dtype, f"{what} {name}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_transformer_shape(gpu, dtype, causal):
    q, k, v = rand((2, 8, 256, 64), dtype, 31), rand((2, 2, 256, 64), dtype, 32), rand((2, 2, 256, 64), dtype, 33)
    check_bwd(q, k, v, causal=causal, what=f"{dtype} causal={causal}")


def test_backward_ragged_bias_d128(gpu):
    dtype = torch.float16
    q, k, v = rand((1, 4, 100, 128), dtype, 34), rand((1, 2, 150, 128), dtype, 35), rand((1, 2, 150, 128), dtype, 36)
    check_bwd(q, k, v, what="ragged D128")
    check_bwd(q, k, v, causal=True, what="ragged causal")
    bias = rand((1, 4, 100, 150), dtype, 37)
    bias[0, :, 7] = float("-inf")        # a row that attends to nothing
    check_bwd(q, k, v, bias=bias, what="bias with an empty row")
    q2 = rand((1, 2, 200, 64), dtype, 38)
    k2, v2 = rand((1, 2, 40, 64), dtype, 39), rand((1, 2, 40, 64), dtype, 40)
    check_bwd(q2, k2, v2, causal=True, what="causal L 200 > S 40")


@pytest.mark.parametrize("causal", [False, True])
def test_backward_odd_tiles_mha(gpu, causal):
    # one head per kv head, 3 query tiles (the two dK/dV wave groups take 2 and 1),
    # batch*heads = 3 (not a multiple of the 8 XCDs), keys past the queries
    dtype = torch.float16
    q = rand((1, 3, 130, 64), dtype, 41)
    k, v = rand((1, 3, 190, 64), dtype, 42), rand((1, 3, 190, 64), dtype, 43)
    check_bwd(q, k, v, causal=causal, what=f"MHA L 130 S 190 causal={causal}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_backward_wide_grid(gpu, dtype):
    # batch*heads*ceil(L/128) >= 2048: dQ with two query columns per wave; the
    # oracle checks two (batch, kv head) slices with all four of their query heads
    B, Hq, Hk, L, D = 16, 16, 4, 1024, 64
    q, k, v = rand((B, Hq, L, D), dtype, 44), rand((B, Hk, L, D), dtype, 45), rand((B, Hk, L, D), dtype, 46)
    dq_, dk_, dv_ = (t.to(DEV) for t in (q, k, v))
    out, lse = _abi.attention_fwd(dq_, dk_, dv_, None, True)
    dout = rand(out.shape, dtype, 47)
    gq, gk, gv = _abi.attention_bwd(dq_, dk_, dv_, out, lse, dout.to(DEV), None, True)
    torch.cuda.synchronize()
    rdt = orc.F16 if dtype == torch.float16 else orc.BF16
    for b, hk in ((0, 0), (11, 3)):
        hs = slice(4 * hk, 4 * hk + 4)
        ref = orc.attention_bwd(f64(q[b:b + 1, hs]), f64(k[b:b + 1, hk:hk + 1]), f64(v[b:b + 1, hk:hk + 1]),
                                f64(dout[b:b + 1, hs]), None, True, None, out=f64(out[b:b + 1, hs]), round_to=rdt)
        for got, want, name in zip((gq[b:b + 1, hs], gk[b:b + 1, hk:hk + 1], gv[b:b + 1, hk:hk + 1]), ref,
                                   ("dq", "dk", "dv")):
            assert_close(f64(got), want, dtype, f"b {b} kv head {hk} {name}")


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.float16, 80)])
def test_sdpa_general_on_vulkan_with_bias_gradient(gpu, monkeypatch, dtype, D):
    # float32 and head dim 80 run on the device (strict mode raises on any CPU fallback),
    # and the gradient of a broadcast float mask comes back through the score gradient
    import torchvulkan_amd  # noqa: F401

    monkeypatch.setenv("TORCHVULKAN_STRICT", "1")
    V = "vulkan"
    q, k, v = rand((2, 4, 48, D), dtype, 500), rand((2, 4, 60, D), dtype, 501), rand((2, 4, 60, D), dtype, 502)
    mask = rand((1, 4, 48, 60), dtype, 503)
    qv, kv_, vv, mv = (t.to(V).requires_grad_() for t in (q, k, v, mask))
    out = F.scaled_dot_product_attention(qv, kv_, vv, attn_mask=mv)
    q64, k64, v64, m64 = (t.double().requires_grad_() for t in (q, k, v, mask))
    ref = F.scaled_dot_product_attention(q64, k64, v64, attn_mask=m64)
    assert_close(f64(out), ref.detach().numpy(), dtype, "sdpa out")
    g = rand(out.shape, dtype, 504)
    out.backward(g.to(V))
    ref.backward(g.double())
    tol = 1e-5 if dtype == torch.float32 else 5e-3
    for got, want, name in ((qv.grad, q64.grad, "dq"), (kv_.grad, k64.grad, "dk"), (vv.grad, v64.grad, "dv"),
                            (mv.grad, m64.grad, "dmask")):
        assert got.shape == want.shape, name
        err = (got.cpu().double() - want).abs() / (tol * (want.abs() + 1))
        assert err.max().item() <= 1.0, f"{name}: {err.max().item():.2f}x tolerance"
