"""tvk_gemm_noalloc through the C ABI: the allocation-free variant of tvk_gemm
(scratch in the library's fixed 32 MiB per-device array) gives tvk_gemm's
results bit for bit on products that use scratch (split-K partials, repacked
operands, the streaming kernel's partials) and on one that uses none, on two
calls in a row with the second smaller (the array keeps the first call's
contents), allocates no device memory (checked against an emptied scratch
pool, where tvk_gemm's lease of the same product does allocate), and rejects a product whose scratch
exceeds the array before queuing anything."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from tests.gemm_cases import randn
from torchvulkan_amd import _abi

pytestmark = pytest.mark.gpu

DEV = "cuda"


def noalloc(a, b, c, **kw) -> int:
    """Status of one tvk_gemm_noalloc call (the raw C ABI), on torch's current stream."""
    d = _abi.make_gemm_desc(a, b, c, kw.get("bias"), kw.get("alpha", 1.0), kw.get("beta", 0.0),
                            kw.get("act", _abi.TVK_ACT_NONE), torch.cuda.current_stream().cuda_stream, False)
    return _abi.load().tvk_gemm_noalloc(C.byref(d))


def reserved() -> int:
    v = C.c_size_t(0)
    assert _abi.load().tvk_memory_reserved(torch.cuda.current_device(), C.byref(v)) == _abi.TVK_OK
    return v.value


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return (t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)).numpy()


# (M, N, K, dtype, transposed B, batch, bias, expected kernel): a split-K product,
# an operand repack, the streaming kernel's split partials, batches, and float32 (no scratch)
CASES = [
    ((256, 4096, 4096, torch.float16, True, 1, True), "gemm16_dma_128x128_splitk"),
    ((1000, 3000, 777, torch.float16, False, 1, False), "gemm16_dma_128x128"),
    ((16, 14336, 4096, torch.bfloat16, False, 1, False), "gemm16_skinny_ring_splitk"),
    ((512, 512, 8192, torch.bfloat16, True, 2, True), "gemm16_dma_128x128_splitk"),
    ((300, 260, 200, torch.float32, False, 1, True), "gemm_seq_mfma_64x64"),
]
SMALLER = {
    0: (128, 2048, 4096),
    1: (500, 1000, 333),
    2: (8, 4096, 2048),
    3: (256, 256, 4096),
    4: (64, 64, 64),
}


def operands(M, N, K, dtype, bt, batch, with_bias, seed):
    a = randn((batch, M, K), dtype, seed).to(DEV)
    b = randn((batch, N, K), dtype, seed + 1).to(DEV).transpose(1, 2) if bt else randn((batch, K, N), dtype, seed + 1).to(DEV)
    bias = randn((N,), dtype, seed + 2).to(DEV) if with_bias else None
    if batch == 1:
        a, b = a[0], b[0]
    return a, b, bias


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_tvk_gemm_twice(gpu, case):
    (M, N, K, dtype, bt, batch, with_bias), kernel = CASES[case]
    torch.cuda.synchronize()
    for step, (m, n, k) in enumerate(((M, N, K), SMALLER[case])):
        print(f"case {case} step {step}: {m}x{n}x{k} {dtype} batch {batch}", flush=True)
        a, b, bias = operands(m, n, k, dtype, bt, batch, with_bias, 10 * case + step)
        shape = (batch, m, n) if batch > 1 else (m, n)
        c_ref = torch.empty(shape, dtype=dtype, device=DEV)
        c = torch.full(shape, float("nan"), dtype=dtype, device=DEV)
        kw = dict(bias=bias, alpha=0.5, beta=2.0 if with_bias else 0.0)
        if step == 0:
            assert _abi.gemm_plan(a, b, c, **kw) == kernel
        torch.cuda.synchronize()
        # drop every idle scratch-pool buffer and cached block first: a lease from the pool would
        # then have to allocate a new buffer, which the reserved bytes would show
        assert _abi.load().tvk_empty_cache(torch.cuda.current_device()) == _abi.TVK_OK
        held0 = reserved()
        assert noalloc(a, b, c, **kw) == _abi.TVK_OK, _abi.load().tvk_last_error()
        torch.cuda.synchronize()
        # no device memory was taken: the library's reserved bytes (allocator blocks and the
        # scratch pool's buffers) are unchanged
        assert reserved() == held0
        # the check has teeth: tvk_gemm of a product that needs scratch leases a pool buffer,
        # which the emptied pool must allocate
        if step == 0 and not kernel.startswith("gemm_seq_mfma"):
            _abi.gemm(a, b, torch.empty_like(c), **kw)
            torch.cuda.synchronize()
            assert reserved() > held0
        _abi.gemm(a, b, c_ref, **kw)
        torch.cuda.synchronize()
        assert np.array_equal(bits(c), bits(c_ref)), f"case {case} step {step}: differs from tvk_gemm"


def test_noalloc_rejects_scratch_beyond_the_array(gpu):
    # rows of 4097 float16 elements miss the 16-byte layout: A [8192, 4097] is repacked into
    # 8192 x 4104 x 2 bytes = 64.1 MiB of scratch, twice the array
    a, b, _ = operands(8192, 1024, 4097, torch.float16, False, 1, False, 90)
    c = torch.zeros((8192, 1024), dtype=torch.float16, device=DEV)
    st = noalloc(a, b, c)
    assert st == _abi.TVK_ERR_INVALID
    assert b"bytes of scratch" in _abi.load().tvk_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(c).item() == 0      # nothing was queued
