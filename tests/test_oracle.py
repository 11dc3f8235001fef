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


# ---------------------------------------------------------------------------
# float64 and integer products (oracle_gemm_wide_rows)
# ---------------------------------------------------------------------------

INT_TYPES = [(orc.I64, np.int64), (orc.I32, np.int32), (orc.I16, np.int16), (orc.I8, np.int8), (orc.U8, np.uint8)]


@pytest.mark.parametrize("dt,npt", INT_TYPES)
def test_integer_products_wrap_like_numpy(dt, npt):
    # numpy's integer matmul accumulates in the type and wraps: the reference's accumulate type
    rng = np.random.default_rng(10 + dt)
    info = np.iinfo(npt)
    a = rng.integers(info.min, info.max, (3, 17, 29), endpoint=True, dtype=npt)
    b = rng.integers(info.min, info.max, (3, 29, 11), endpoint=True, dtype=npt)
    got = orc.gemm(a, b, dt)
    assert got.dtype == npt
    assert np.array_equal(got, np.matmul(a, b))
    # transposed views, broadcast B, bias with integer alpha and beta
    bt = np.ascontiguousarray(b[0].T).T
    bias = rng.integers(info.min, info.max, (11,), endpoint=True, dtype=npt)
    got = orc.gemm(a[1], bt, dt, bias=bias, alpha=3.0, beta=-2.0)
    with np.errstate(over="ignore"):
        want = (np.matmul(a[1], bt) * npt(3) + bias * (npt(-2) if info.min < 0 else npt(-2 % (info.max + 1)))).astype(npt)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt,npt", INT_TYPES)
def test_integer_products_brute_force_modular(dt, npt):
    # Python integers reduced modulo 2^bits at the end: a different route to the same bits
    rng = np.random.default_rng(20 + dt)
    info = np.iinfo(npt)
    bits = info.bits
    a = rng.integers(info.min, info.max, (4, 9), endpoint=True, dtype=npt)
    b = rng.integers(info.min, info.max, (9, 5), endpoint=True, dtype=npt)
    bias = rng.integers(info.min, info.max, (4, 5), endpoint=True, dtype=npt)
    got = orc.gemm(a, b, dt, bias=bias, alpha=5.0, beta=7.0, act=orc.ACT_RELU)
    for i in range(4):
        for j in range(5):
            v = 5 * sum(int(a[i, k]) * int(b[k, j]) for k in range(9)) + 7 * int(bias[i, j])
            v %= 1 << bits
            if info.min < 0 and v >= 1 << (bits - 1):
                v -= 1 << bits
            if v < 0:
                v = 0
            assert int(got[i, j]) == v, (i, j)


def test_float64_sequential_fma_order():
    # exact-rational fma recurrence per output (fma = the exact a*b + acc, rounded once);
    # the inputs span many magnitudes so that other orders land on other doubles
    rng = np.random.default_rng(30)
    M, N, K = 5, 6, 40
    a = rng.standard_normal((M, K)) * np.exp2(rng.integers(-30, 30, (M, K)))
    b = rng.standard_normal((K, N)) * np.exp2(rng.integers(-30, 30, (K, N)))
    bias = rng.standard_normal((N,))
    got = orc.gemm(a, b, orc.F64, bias=bias, alpha=0.3, beta=-1.7)
    differs = 0
    for i in range(M):
        for j in range(N):
            acc = 0.0
            for k in range(K):
                acc = float(Fraction(a[i, k]) * Fraction(b[k, j]) + Fraction(acc))
            v = float(Fraction(acc) * Fraction(0.3))
            t = float(Fraction(bias[j]) * Fraction(-1.7))
            v = float(Fraction(v) + Fraction(t))
            assert got[i, j] == v, (i, j)
            differs += float(np.dot(a[i], b[:, j])) * 0.3 + bias[j] * -1.7 != v
    assert differs > 0   # the order is visible on these inputs


def test_float64_integer_valued_exact_and_activations():
    rng = np.random.default_rng(31)
    a = rng.integers(-8, 9, (2, 33, 70)).astype(np.float64)
    b = rng.integers(-8, 9, (2, 70, 21)).astype(np.float64)
    assert np.array_equal(orc.gemm(a, b, orc.F64), a @ b)
    x = rng.standard_normal((9, 13))
    y = rng.standard_normal((13, 7))
    r = orc.gemm(x, y, orc.F64)
    assert np.array_equal(orc.gemm(x, y, orc.F64, act=orc.ACT_RELU), np.maximum(r, 0.0))
    g = torch.nn.functional.gelu(torch.from_numpy(r)).numpy()
    np.testing.assert_allclose(orc.gemm(x, y, orc.F64, act=orc.ACT_GELU), g, rtol=1e-15, atol=1e-15)


def test_wide_k_zero_and_beta_zero():
    a = np.zeros((3, 0))
    b = np.zeros((0, 4))
    bias = np.arange(4, dtype=np.float64)
    assert np.array_equal(orc.gemm(a, b, orc.F64, bias=bias, beta=2.0), np.tile(bias * 2.0, (3, 1)))
    nanb = np.full((4,), np.nan)
    x = np.ones((3, 5))
    assert np.array_equal(orc.gemm(x, np.ones((5, 4)), orc.F64, bias=nanb, beta=0.0), np.full((3, 4), 5.0))
    ai = np.ones((3, 0), dtype=np.int32)
    bi = np.ones((0, 4), dtype=np.int32)
    assert np.array_equal(orc.gemm(ai, bi, orc.I32, bias=np.int32([1, 2, 3, 4]), beta=3.0),
                          np.tile(np.int32([3, 6, 9, 12]), (3, 1)))
