"""Pins the CPU oracle (oracle/gemm_oracle.c) before anything is compared to it.

Each check is chosen so that a plausible mistake in the oracle fails it:
conversions against numpy/torch's correctly rounded ones, exact integer
products (any summation order gives the same bits), the error bound every
order satisfies, an exact-rational restatement of the sequential order on
tiny inputs, and the epilogue special cases of the reference
(src/api/ops/matmul.cpp:259,284-288; src/shaders/helpers/gemm_simd.slang:67-99).
"""
from fractions import Fraction
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.build()


# ---------------------------------------------------------------------------
# conversions
# ---------------------------------------------------------------------------

def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    # wide exponent range: subnormals, normals, overflow to inf
    x = (rng.standard_normal(200_000) * np.exp2(rng.integers(-30, 18, 200_000))).astype(np.float32)
    # exact midpoints between neighbouring halves (ties to even)
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.float32([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, np.inf, -np.inf])])
    got = orc.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert orc.f32_to_f16_bits(np.float32([np.nan]))[0] & 0x7e00 == 0x7e00


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200_000) * np.exp2(rng.integers(-130, 120, 200_000))).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, np.inf, -np.inf, 3.3895314e38])])
    got = orc.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(orc.bf16_bits_to_f32(got), torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------------------
# GEMM values
# ---------------------------------------------------------------------------

def _encode(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == orc.F32:
        return x
    if dtype == orc.F16:
        return x.astype(np.float16).view(np.uint16)
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", [orc.F32, orc.F16, orc.BF16])
@pytest.mark.parametrize("fma", [True, False])
def test_integer_products_are_exact(dtype, fma):
    # |sum| <= 64*16 = 1024: exact in float32 partials and in every output type
    rng = np.random.default_rng(2)
    a = rng.integers(-4, 5, (37, 64)).astype(np.float32)
    b = rng.integers(-4, 5, (64, 29)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    got = orc.to_f32(orc.gemm(_encode(a, dtype), _encode(b, dtype), dtype, fma=fma), dtype)
    assert np.array_equal(got, want)
    # transposed and sliced operand views give the same values
    at = np.ascontiguousarray(_encode(a, dtype).T).T
    bt = np.ascontiguousarray(_encode(b, dtype).T).T
    got_t = orc.to_f32(orc.gemm(at, bt, dtype, fma=fma), dtype)
    assert np.array_equal(got_t, want)


def test_batched_broadcast_exact():
    rng = np.random.default_rng(3)
    a = rng.integers(-3, 4, (5, 8, 16)).astype(np.float32)
    b = rng.integers(-3, 4, (16, 7)).astype(np.float32)  # broadcast over the batch
    got = orc.gemm(a, b, orc.F32)
    want = np.einsum("bmk,kn->bmn", a.astype(np.int64), b.astype(np.int64)).astype(np.float32)
    assert got.shape == (5, 8, 7)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("K", [1, 17, 300, 1024])
def test_f32_error_bound(K):
    # every summation order satisfies |c - exact| <= gamma_K * sum|a||b|
    rng = np.random.default_rng(K)
    a = rng.standard_normal((19, K)).astype(np.float32)
    b = rng.standard_normal((K, 23)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound_scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    u = 2.0 ** -24
    gamma = (K + 1) * u / (1 - (K + 1) * u)
    for fma in (True, False):
        got = orc.gemm(a, b, orc.F32, fma=fma).astype(np.float64)
        assert np.all(np.abs(got - exact) <= gamma * bound_scale + 1e-30)


def _round_f32(q: Fraction) -> Fraction:
    """Rounds an exact rational to float32, nearest even (normal and subnormal)."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    scale = max(e, -126) - 23
    x = q / (Fraction(2) ** scale)
    n = math.floor(x)
    r = x - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * Fraction(2) ** scale


def test_sequential_order_exact_rational():
    # operands of very different magnitudes make the order and the fused form visible
    rng = np.random.default_rng(4)
    K = 9
    a = (rng.standard_normal((3, K)) * np.exp2(rng.integers(-20, 20, (3, K)))).astype(np.float32)
    b = (rng.standard_normal((K, 4)) * np.exp2(rng.integers(-20, 20, (K, 4)))).astype(np.float32)
    for fma in (True, False):
        got = orc.gemm(a, b, orc.F32, fma=fma)
        differs_from_reverse = False
        for i in range(3):
            for j in range(4):
                acc = Fraction(0)
                rev = Fraction(0)
                for k in range(K):
                    p = Fraction(float(a[i, k])) * Fraction(float(b[k, j]))
                    acc = _round_f32(acc + p) if fma else _round_f32(acc + _round_f32(p))
                for k in reversed(range(K)):
                    p = Fraction(float(a[i, k])) * Fraction(float(b[k, j]))
                    rev = _round_f32(rev + p) if fma else _round_f32(rev + _round_f32(p))
                assert Fraction(float(got[i, j])) == acc, (fma, i, j)
                differs_from_reverse |= acc != rev
        assert differs_from_reverse  # the inputs do distinguish the order


# ---------------------------------------------------------------------------
# epilogue
# ---------------------------------------------------------------------------

def test_alpha_beta_bias_against_torch():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((33, 40)).astype(np.float32)
    b = rng.standard_normal((40, 21)).astype(np.float32)
    bias = rng.standard_normal(21).astype(np.float32)
    got = orc.gemm(a, b, orc.F32, bias=bias, alpha=0.5, beta=1.25)
    want = torch.addmm(torch.from_numpy(bias).double(), torch.from_numpy(a).double(), torch.from_numpy(b).double(),
                       beta=1.25, alpha=0.5).numpy()
    assert np.all(np.abs(got - want) <= 1e-5 * (np.abs(want) + 1))


def test_beta_zero_ignores_nan_bias():
    a = np.ones((4, 3), np.float32)
    b = np.ones((3, 5), np.float32)
    bias = np.full((4, 5), np.nan, np.float32)
    got = orc.gemm(a, b, orc.F32, bias=bias, beta=0.0)
    assert np.array_equal(got, np.full((4, 5), 3.0, np.float32))


def test_k_zero_gives_beta_bias():
    a = np.zeros((4, 0), np.float32)
    b = np.zeros((0, 5), np.float32)
    bias = np.arange(5, dtype=np.float32)
    assert np.array_equal(orc.gemm(a, b, orc.F32, bias=bias, beta=2.0), np.broadcast_to(2.0 * bias, (4, 5)))
    assert np.array_equal(orc.gemm(a, b, orc.F32), np.zeros((4, 5), np.float32))


def test_relu_and_gelu():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((16, 32)).astype(np.float32)
    b = rng.standard_normal((32, 16)).astype(np.float32)
    plain = orc.gemm(a, b, orc.F32)
    relu = orc.gemm(a, b, orc.F32, act=orc.ACT_RELU)
    assert np.array_equal(relu, np.maximum(plain, 0))
    gelu = orc.gemm(a, b, orc.F32, act=orc.ACT_GELU)
    want = torch.nn.functional.gelu(torch.from_numpy(plain).double()).numpy()
    assert np.all(np.abs(gelu - want) <= 1e-6 * (np.abs(want) + 1))
