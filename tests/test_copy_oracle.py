"""Pins the cast oracle (oracle/copy_oracle.c, the reference's castValue rules)
against independent conversions: numpy's float64 -> float16 (one correctly
rounded step), numpy/torch float and integer conversions, exact integer
arithmetic, and hand-built rounding cases where one and two roundings differ.
Plausible mistakes (going through float32 for half(double), the wrong
tie rule, bool casts that keep the value, integer saturation instead of wrap)
each fail at least one test."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc

FLOATS = [orc.F32, orc.F16, orc.BF16, orc.F64]
INTS = [orc.I64, orc.I32, orc.I16, orc.I8, orc.U8]
NP_INT = {orc.I64: np.int64, orc.I32: np.int32, orc.I16: np.int16, orc.I8: np.int8, orc.U8: np.uint8}


def as_value(bits: np.ndarray, dt: int) -> np.ndarray:
    """Element values (float64 for floats) of an oracle storage array."""
    if dt == orc.F16:
        return bits.view(np.float16).astype(np.float64)
    if dt == orc.BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bits.astype(np.float64)


def from_value(x: np.ndarray, dt: int) -> np.ndarray:
    """Storage array of float values that are exact in dt."""
    if dt == orc.F16:
        return x.astype(np.float16).view(np.uint16)
    if dt == orc.BF16:
        return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return x.astype(orc.STORAGE[dt])


def random_doubles(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    mant = rng.uniform(1.0, 2.0, n)
    exp = rng.integers(-30, 20, n)
    sign = rng.choice([-1.0, 1.0], n)
    return sign * np.ldexp(mant, exp)


def test_f64_to_f16_is_one_rounding():
    x = random_doubles(200_000, 0)
    # every half midpoint and its neighbours one double ulp either side
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    ties = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, np.inf), -mids])
    x = np.concatenate([x, ties, [0.0, -0.0, 65504.0, 65519.999, 65520.0, 2.0**-25, 2.0**-24, 1e-300]])
    got = orc.cast(x, orc.F64, orc.F16)
    want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_f64_to_f16_differs_from_two_roundings():
    # 1 + 2^-11 + 2^-40 is just above the midpoint of 1 and 1 + 2^-10; through
    # float32 it lands on the midpoint and ties to 1.0 (torch CPU's route)
    d = np.array([1.0 + 2.0**-11 + 2.0**-40, -(1.0 + 2.0**-11 + 2.0**-40)])
    got = orc.cast(d, orc.F64, orc.F16).view(np.float16)
    assert got[0] == np.float16(1.0 + 2.0**-10) and got[1] == -np.float16(1.0 + 2.0**-10)
    two_step = torch.from_numpy(d).to(torch.float16).numpy()
    assert two_step[0] == np.float16(1.0), "the case must separate one and two roundings"


def test_f64_to_bf16_goes_through_float32():
    # BFloat16(float(v)): a double just above a bf16 midpoint that float32 rounds onto the midpoint
    d = np.array([1.0 + 2.0**-8 + 2.0**-40])
    got = orc.cast(d, orc.F64, orc.BF16)
    assert as_value(got, orc.BF16)[0] == 1.0
    want = torch.from_numpy(d).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_float_to_float_matches_numpy_and_torch():
    x = np.concatenate([random_doubles(50_000, 1).astype(np.float32), [0, -0.0, np.inf, -np.inf, 3e38, 1e-40]])
    x = x.astype(np.float32)
    np.testing.assert_array_equal(orc.cast(x, orc.F32, orc.F16), x.astype(np.float16).view(np.uint16))
    bf = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.cast(x, orc.F32, orc.BF16), bf)
    np.testing.assert_array_equal(orc.cast(x, orc.F32, orc.F64), x.astype(np.float64))
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(h.view(np.float16))
    np.testing.assert_array_equal(orc.cast(h, orc.F16, orc.F32)[finite], h.view(np.float16).astype(np.float32)[finite])
    np.testing.assert_array_equal(orc.cast(h, orc.BF16, orc.F64), as_value(h, orc.BF16))
    # half <-> bfloat16 through float: one rounding from the exact float value
    np.testing.assert_array_equal(orc.cast(h[finite], orc.F16, orc.BF16),
                                  orc.cast(h.view(np.float16).astype(np.float32)[finite], orc.F32, orc.BF16))


def test_nan_stays_nan():
    x = np.array([np.nan, -np.nan], dtype=np.float32)
    for dt in (orc.F16, orc.BF16, orc.F64):
        assert np.isnan(as_value(orc.cast(x, orc.F32, dt), dt)).all()


@pytest.mark.parametrize("sdt", INTS)
def test_int_to_float(sdt):
    info = np.iinfo(NP_INT[sdt])
    rng = np.random.default_rng(sdt)
    v = rng.integers(info.min, info.max, 20_000, dtype=np.int64, endpoint=True).astype(NP_INT[sdt])
    v = np.concatenate([v, np.array([info.min, info.max, 0, 1], dtype=NP_INT[sdt])])
    np.testing.assert_array_equal(orc.cast(v, sdt, orc.F32), v.astype(np.float32))
    np.testing.assert_array_equal(orc.cast(v, sdt, orc.F64), v.astype(np.float64))
    np.testing.assert_array_equal(orc.cast(v, sdt, orc.F16), v.astype(np.float64).astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(orc.cast(v, sdt, orc.BF16), from_value(v.astype(np.float32), orc.BF16))


def test_int64_to_float32_rounds_to_nearest_even():
    v = np.array([2**24 + 1, 2**24 + 3, 2**53 + 1, -(2**24 + 1), 2**63 - 1], dtype=np.int64)
    np.testing.assert_array_equal(orc.cast(v, orc.I64, orc.F32), np.array([2**24, 2**24 + 4, 2**53, -(2**24), 2.0**63],
                                                                           dtype=np.float32))


@pytest.mark.parametrize("ddt", INTS)
def test_float_to_int_truncates_in_range(ddt):
    info = np.iinfo(NP_INT[ddt])
    rng = np.random.default_rng(ddt + 10)
    lo, hi = max(info.min, -2**40), min(info.max, 2**40)
    x = rng.uniform(lo, hi, 20_000)
    x = np.concatenate([x, [-0.9, 0.9, -0.0, 2.5, -2.5]])
    x = x[(x > info.min - 1) & (x < info.max + 1)]
    np.testing.assert_array_equal(orc.cast(x, orc.F64, ddt), np.trunc(x).astype(NP_INT[ddt]))
    x32 = x.astype(np.float32)
    x32 = x32[(x32 > info.min - 1) & (x32 < info.max + 1) & (np.abs(x32) < 2**31)]
    np.testing.assert_array_equal(orc.cast(x32, orc.F32, ddt), np.trunc(x32).astype(np.int64).astype(NP_INT[ddt]))


def test_float_to_int_out_of_range_saturates_nan_is_zero():
    x = np.array([1e30, -1e30, np.nan, 300.0, -5.0], dtype=np.float64)
    assert list(orc.cast(x, orc.F64, orc.I32)) == [2**31 - 1, -2**31, 0, 300, -5]
    assert list(orc.cast(x, orc.F64, orc.I8)) == [127, -128, 0, 127, -5]
    assert list(orc.cast(x, orc.F64, orc.U8)) == [255, 0, 0, 255, 0]
    assert list(orc.cast(x, orc.F64, orc.I64)) == [2**63 - 1, -2**63, 0, 300, -5]


@pytest.mark.parametrize("sdt", INTS)
@pytest.mark.parametrize("ddt", INTS)
def test_int_to_int_wraps(sdt, ddt):
    info = np.iinfo(NP_INT[sdt])
    v = np.random.default_rng(sdt * 16 + ddt).integers(info.min, info.max, 5000, dtype=np.int64,
                                                         endpoint=True).astype(NP_INT[sdt])
    np.testing.assert_array_equal(orc.cast(v, sdt, ddt), v.astype(NP_INT[ddt]))


@pytest.mark.parametrize("dt", FLOATS + INTS)
def test_bool_casts(dt):
    if dt in FLOATS:
        vals = from_value(np.array([0.0, -0.0, 1.0, -2.5, 1e-30 if dt != orc.F16 else 2.0**-24, np.inf]), dt)
        want = np.array([0, 0, 1, 1, 1, 1], dtype=np.uint8)
        nan = from_value(np.array([np.nan]), dt)
        assert orc.cast(nan, dt, orc.BOOL)[0] == 1, "NaN != 0"
    else:
        vals = np.array([0, 1, 2, 255 if dt == orc.U8 else -1, 100], dtype=NP_INT[dt])
        want = (vals != 0).astype(np.uint8)
    np.testing.assert_array_equal(orc.cast(vals, dt, orc.BOOL), want)
    b = np.array([0, 1], dtype=np.uint8)
    np.testing.assert_array_equal(as_value(orc.cast(b, orc.BOOL, dt), dt), [0.0, 1.0])
    # a bool byte other than 1 still reads as true
    assert as_value(orc.cast(np.array([2], dtype=np.uint8), orc.BOOL, dt), dt)[0] == 1.0
