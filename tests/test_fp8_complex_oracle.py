"""Pins of the oracle's float8 conversions, division, complex product and
emulated _scaled_mm (CPU only).

float8 conversion is c10's (the reference converts through it), so torch's
own CPU conversion is the reference here: every code decoded, and encoding on
a sweep of every rounding boundary of both formats (each midpoint between
neighbouring codes, the codes themselves, one and two float32 steps either
side, overflow and NaN) plus random float32 bit patterns. The complex product
and _scaled_mm restatements are pinned exactly on integer-valued data (every
product and sum exact, so any ordering agrees and a dropped term or wrong
sign shows) and to float tolerance against torch's CPU kernels otherwise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc

F8 = [(orc.F8E4M3FN, torch.float8_e4m3fn), (orc.F8E5M2, torch.float8_e5m2)]


def boundary_sweep(tdt) -> np.ndarray:
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(tdt).float().numpy()
    fin = np.unique(np.abs(vals[np.isfinite(vals)])).astype(np.float32)
    mids = ((fin[:-1].astype(np.float64) + fin[1:]) / 2).astype(np.float32)
    extra = np.array([448, 464, 480, 496, 57344, 61440, 65536, 1e30, np.inf, np.nan, 0.0, 1e-40, 1e-45,
                      2.0 ** -10, 2.0 ** -17, 2.0 ** -18], np.float32)
    base = np.concatenate([fin, mids, extra])
    pts = [base]
    up, dn = base, base
    for _ in range(2):
        up = np.nextafter(up, np.float32(np.inf))
        dn = np.nextafter(dn, np.float32(0))
        pts += [up, dn]
    x = np.concatenate(pts).astype(np.float32)
    return np.concatenate([x, -x])


def random_bits(n: int, seed: int) -> np.ndarray:
    g = np.random.default_rng(seed)
    return g.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("odt,tdt", F8)
def test_f8_decode_every_code_matches_torch(odt, tdt):
    codes = np.arange(256, dtype=np.uint8)
    got = orc.cast(codes, odt, orc.F32).view(np.uint32)
    want = torch.from_numpy(codes).view(tdt).float().numpy().view(np.uint32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("odt,tdt", F8)
def test_f8_encode_matches_torch(odt, tdt):
    x = np.concatenate([boundary_sweep(tdt), random_bits(1 << 20, 7)])
    got = orc.cast(x, orc.F32, odt)
    want = torch.from_numpy(x).to(tdt).view(torch.uint8).numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


@pytest.mark.parametrize("odt,tdt", F8)
def test_f8_to_and_from_other_types_match_torch(odt, tdt):
    g = np.random.default_rng(3)
    # float64 / float16 / bfloat16 / integers -> float8 (through float32, as the CPU does)
    x64 = np.concatenate([g.standard_normal(4096) * 300, boundary_sweep(tdt).astype(np.float64)])
    assert np.array_equal(orc.cast(x64, orc.F64, odt), torch.from_numpy(x64).to(tdt).view(torch.uint8).numpy())
    h = torch.from_numpy(g.standard_normal(4096).astype(np.float32) * 200).half()
    got = orc.cast(h.view(torch.int16).numpy().view(np.uint16), orc.F16, odt)
    assert np.array_equal(got, h.to(tdt).view(torch.uint8).numpy())
    bf = torch.from_numpy(g.standard_normal(4096).astype(np.float32) * 200).bfloat16()
    got = orc.cast(bf.view(torch.int16).numpy().view(np.uint16), orc.BF16, odt)
    assert np.array_equal(got, bf.to(tdt).view(torch.uint8).numpy())
    ints = np.arange(-600, 600, dtype=np.int32)
    assert np.array_equal(orc.cast(ints, orc.I32, odt), torch.from_numpy(ints).to(tdt).view(torch.uint8).numpy())
    # float8 -> the other types, for every finite code (NaN and infinity to an
    # integer are undefined on the CPU)
    # (NaN payloads of wider results are not compared: the CPU's route through
    # float32 and each rounding may requiet them)
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(tdt)
    assert np.array_equal(orc.cast(codes, odt, orc.F64), t.double().numpy(), equal_nan=True)
    assert np.array_equal(orc.to_f32(orc.cast(codes, odt, orc.F16), orc.F16), t.half().float().numpy(), equal_nan=True)
    assert np.array_equal(orc.to_f32(orc.cast(codes, odt, orc.BF16), orc.BF16), t.bfloat16().float().numpy(),
                          equal_nan=True)
    assert np.array_equal(orc.cast(codes, odt, orc.BOOL), t.bool().numpy().view(np.uint8))
    fin = np.isfinite(t.float().numpy())
    assert np.array_equal(orc.cast(codes, odt, orc.I32)[fin], t.int().numpy()[fin])


def test_f8_between_formats_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    for (sa, ta), (sb, tb) in ((F8[0], F8[1]), (F8[1], F8[0])):
        want = torch.from_numpy(codes).view(ta).to(tb).view(torch.uint8).numpy()
        assert np.array_equal(orc.cast(codes, sa, sb), want)


@pytest.mark.parametrize("dt,tdt", [(orc.F32, torch.float32), (orc.F64, torch.float64), (orc.F16, torch.float16),
                                    (orc.BF16, torch.bfloat16)])
def test_binary_div_matches_torch(dt, tdt):
    g = np.random.default_rng(5)
    a = torch.from_numpy(g.standard_normal(20000) * 10).to(tdt)
    b = torch.from_numpy(g.standard_normal(20000)).to(tdt)
    b[:7] = torch.tensor([0.0, -0.0, float("inf"), float("nan"), 1e-30, 3.0, -7.0]).to(tdt)
    store = lambda t: t.view(torch.int16).numpy().view(np.uint16) if t.element_size() == 2 else t.numpy()
    got = orc.binary(store(a), store(b), dt, orc.BIN_DIV)
    want = store(a / b)
    gv = got.view(np.uint64 if dt == orc.F64 else np.uint32 if dt == orc.F32 else np.uint16)
    wv = want.view(gv.dtype)
    nan = np.isnan((a / b).float().numpy())
    assert np.array_equal(gv[~nan], wv[~nan])
    assert np.isnan(orc.to_f32(got, dt) if dt in (orc.F16, orc.BF16) else got)[nan].all()
    with pytest.raises(ValueError):
        orc.binary(np.arange(4, dtype=np.int32), np.arange(1, 5, dtype=np.int32), orc.I32, orc.BIN_DIV)


def _cint(g, shape, dt):
    return (g.integers(-8, 9, shape) + 1j * g.integers(-8, 9, shape)).astype(dt)


@pytest.mark.parametrize("dt", [np.complex64, np.complex128])
def test_complex_gemm_exact_on_integers(dt):
    g = np.random.default_rng(11)
    a, b, c = _cint(g, (3, 13, 24), dt), _cint(g, (3, 24, 7), dt), _cint(g, (7,), dt)
    for alpha, beta in ((1.0, 0.0), (2 - 1j, 0.0), (1.0, 1.0), (-3 + 2j, 0.5 + 4j)):
        got = orc.complex_gemm(a, b, c, alpha=alpha, beta=beta)
        want = torch.baddbmm(torch.from_numpy(c).expand(3, 13, 7), torch.from_numpy(a), torch.from_numpy(b),
                             beta=beta, alpha=alpha).numpy()
        assert got.dtype == dt and np.array_equal(got, want), (alpha, beta)
    # conjugates: the product of the conjugated operand's parts
    got = orc.complex_gemm(np.conj(a), b)
    assert np.array_equal(got, torch.bmm(torch.from_numpy(a).conj().resolve_conj(), torch.from_numpy(b)).numpy())


@pytest.mark.parametrize("dt,tol", [(np.complex64, 2e-6), (np.complex128, 1e-14)])
def test_complex_gemm_close_to_torch(dt, tol):
    g = np.random.default_rng(12)
    a = (g.standard_normal((40, 300)) + 1j * g.standard_normal((40, 300))).astype(dt)
    b = (g.standard_normal((300, 33)) + 1j * g.standard_normal((300, 33))).astype(dt)
    c = (g.standard_normal((40, 33)) + 1j * g.standard_normal((40, 33))).astype(dt)
    got = orc.complex_gemm(a, b, c, alpha=0.3 + 0.7j, beta=-1.1j)
    want = torch.addmm(torch.from_numpy(c), torch.from_numpy(a), torch.from_numpy(b), beta=-1.1j, alpha=0.3 + 0.7j).numpy()
    assert np.abs(got - want).max() <= tol * np.abs(want).max()


def _f8_codes(vals: np.ndarray, tdt) -> np.ndarray:
    return torch.from_numpy(vals.astype(np.float32)).to(tdt).view(torch.uint8).numpy()


def test_scaled_mm_exact_on_integers():
    g = np.random.default_rng(13)
    a = _f8_codes(g.integers(-6, 7, (16, 64)), torch.float8_e4m3fn)
    b = _f8_codes(g.integers(-6, 7, (64, 24)), torch.float8_e5m2)
    ta = torch.from_numpy(a).view(torch.float8_e4m3fn)
    tb = torch.from_numpy(b).view(torch.float8_e5m2)
    for out_dt, tout in ((orc.F32, torch.float32), (orc.BF16, torch.bfloat16)):
        got = orc.scaled_mm(a, orc.F8E4M3FN, b, orc.F8E5M2, 0.5, 2.0, out_dt)
        want = torch._scaled_mm(ta, tb, torch.tensor(0.5), torch.tensor(2.0), out_dtype=tout)
        want = want.numpy() if out_dt == orc.F32 else want.view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want)
    # a float8 result with scale_result: 1/4 applied before the rounding
    got = orc.scaled_mm(a, orc.F8E4M3FN, b, orc.F8E5M2, 0.5, 2.0, orc.F8E4M3FN, scale_result=4.0)
    want = torch._scaled_mm(ta, tb, torch.tensor(0.5), torch.tensor(2.0), scale_result=torch.tensor(4.0),
                            out_dtype=torch.float8_e4m3fn)
    assert np.array_equal(got, want.view(torch.uint8).numpy())


def test_scaled_mm_rowwise_and_bias_against_float64():
    # the CPU has no row-wise _scaled_mm: the float64 product of the decoded, scaled operands
    g = np.random.default_rng(14)
    a = _f8_codes(g.standard_normal((32, 128)) * 3, torch.float8_e4m3fn)
    b = _f8_codes(g.standard_normal((128, 48)) * 3, torch.float8_e4m3fn)
    sa = g.random((32, 1)).astype(np.float32) + 0.5
    sb = g.random((1, 48)).astype(np.float32) + 0.5
    bias = g.standard_normal(48).astype(np.float32)
    got = orc.scaled_mm(a, orc.F8E4M3FN, b, orc.F8E4M3FN, sa, sb, orc.F32, bias=bias)
    fa = torch.from_numpy(a).view(torch.float8_e4m3fn).double().numpy() * sa
    fb = torch.from_numpy(b).view(torch.float8_e4m3fn).double().numpy() * sb
    want = fa @ fb + bias
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
