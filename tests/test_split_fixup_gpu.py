"""Split-K with the reduction in the same launch on the M <= 16 streaming
kernel (the last workgroup of each column strip sums the strip's float32
partial planes in split order): tvk_gemm takes it, and tvk_gemm_noalloc keeps
the separate reduction launch, so the two entry points must agree bit for
bit. Calls run several times in a row (a strip counter left nonzero by one
launch would leave strips of the next one unwritten), on two streams, over
batches, into a strided output (element stores instead of 8-byte ones), with
bias and GELU epilogues and for odd M."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gemm_cases import randn
from torchvulkan_amd import _abi

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def two_launch(a, b, c, bias=None, beta=0.0, act=_abi.TVK_ACT_NONE) -> None:
    _abi.gemm_noalloc(a, b, c, bias=bias, beta=beta, activation=act)


# (M, N, K, batch, dtype, bias, activation, expected kernel)
CASES = [
    (16, 14336, 4096, 1, torch.float16, False, _abi.TVK_ACT_NONE, "gemm16_skinny_ring_splitk"),
    (16, 14336, 4096, 1, torch.bfloat16, True, _abi.TVK_ACT_GELU, "gemm16_skinny_ring_splitk"),
    (1, 4096, 4096, 1, torch.float16, True, _abi.TVK_ACT_RELU, "gemm16_skinny_ring_splitk"),
    (5, 4096, 4096, 3, torch.bfloat16, True, _abi.TVK_ACT_NONE, "gemm16_skinny_ring_splitk"),
]


def operands(M, N, K, batch, dtype, with_bias, seed):
    a = randn((batch, M, K), dtype, 3 * seed).to(DEV)
    b = randn((batch, K, N), dtype, 3 * seed + 1).to(DEV)
    bias = randn((N,), dtype, 3 * seed + 2).to(DEV) if with_bias else None
    if batch == 1:
        a, b = a[0], b[0]
    return a, b, bias


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}b{c[3]}-{str(c[4])[6:]}-act{c[6]}")
def test_fused_matches_two_launch(case):
    M, N, K, batch, dtype, with_bias, act, kern = case
    shape = (M, N) if batch == 1 else (batch, M, N)
    for seed in (1, 2, 3):
        a, b, bias = operands(M, N, K, batch, dtype, with_bias, seed)
        beta = 1.0 if with_bias else 0.0
        want = torch.empty(shape, dtype=dtype, device=DEV)
        two_launch(a, b, want, bias, beta, act)
        got = torch.full(shape, float("nan"), dtype=dtype, device=DEV)
        assert _abi.gemm_plan(a, b, got, bias=bias, beta=beta, activation=act) == kern
        _abi.gemm(a, b, got, bias=bias, beta=beta, activation=act)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), f"seed {seed}: fused split-K differs from the two-launch reduction"


def test_fused_two_streams_and_strided_output():
    M, N, K = 16, 14336, 4096
    a, b, bias = operands(M, N, K, 1, torch.float16, True, 7)
    want = torch.empty((M, N), dtype=torch.float16, device=DEV)
    two_launch(a, b, want, bias, 1.0)
    # a column-major output: finish4 takes its element stores
    got_t = torch.full((N, M), float("nan"), dtype=torch.float16, device=DEV).t()
    _abi.gemm(a, b, got_t, bias=bias, beta=1.0)
    # the same product on two more streams, back to back (each stream has its own tile counters)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)]
    torch.cuda.synchronize()   # operands and outputs ready before the side streams read them
    for s, o in zip((s1, s2, s1, s2), outs):
        _abi.gemm(a, b, o, bias=bias, beta=1.0, stream=s.cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(bits(got_t), bits(want))
    for i, o in enumerate(outs):
        assert np.array_equal(bits(o), bits(want)), f"call {i} on a side stream differs"


def test_fused_after_cached_split_reduction_on_one_stream():
    """A two-launch split-K product on the 128x128 ring (its reduction reads the partials with ordinary cached
    loads, from the stream's pool buffer) alternates on one stream with the fused skinny product, which writes its
    partials through to the same pool buffer and reads them back at system scope. Any stale L2 line left by the
    cached reads would change the fused result's bits."""
    s = torch.cuda.Stream()
    ring_a = randn((256, 4096), torch.float16, 60).to(DEV)
    ring_b = randn((4096, 2048), torch.float16, 61).to(DEV)
    ring_c = torch.empty((256, 2048), dtype=torch.float16, device=DEV)
    assert _abi.gemm_plan(ring_a, ring_b, ring_c) == "gemm16_dma_128x128_splitk"
    M, N, K = 16, 14336, 4096
    ops = [operands(M, N, K, 1, torch.float16, True, 70 + i) for i in range(3)]
    wants = []
    for a, b, bias in ops:
        w = torch.empty((M, N), dtype=torch.float16, device=DEV)
        two_launch(a, b, w, bias, 1.0)
        wants.append(w)
    ring_want = torch.empty_like(ring_c)
    _abi.gemm_noalloc(ring_a, ring_b, ring_want)
    torch.cuda.synchronize()
    for it in range(6):
        a, b, bias = ops[it % 3]
        _abi.gemm(ring_a, ring_b, ring_c, stream=s.cuda_stream)            # partials through the pool, cached reads
        got = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
        torch.cuda.synchronize()
        _abi.gemm(a, b, got, bias=bias, beta=1.0, stream=s.cuda_stream)   # fused, same stream, same pool buffer
        torch.cuda.synchronize()
        assert np.array_equal(bits(ring_c), bits(ring_want)), f"iteration {it}: ring split-K differs"
        assert np.array_equal(bits(got), bits(wants[it % 3])), f"iteration {it}: fused split-K differs"
