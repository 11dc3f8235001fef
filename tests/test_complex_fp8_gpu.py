"""float8 casts (tvk_copy), division (tvk_binary), complex products and the
emulated _scaled_mm on the GPU, against the oracle. The bar is bit equality:
the float8 conversions are exact functions of their input, complex64 parts
multiply on the float32 kernel (sequential k order, as the oracle) and
complex128 parts on the float64 one, and every combining step is one IEEE
operation in the real type on both sides."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
V = "vulkan"
F8 = [(orc.F8E4M3FN, torch.float8_e4m3fn), (orc.F8E5M2, torch.float8_e5m2)]


@pytest.fixture
def strict():
    old = os.environ.get("TORCHVULKAN_STRICT")
    os.environ["TORCHVULKAN_STRICT"] = "1"
    yield
    if old is None:
        del os.environ["TORCHVULKAN_STRICT"]
    else:
        os.environ["TORCHVULKAN_STRICT"] = old


def sweep(tdt) -> np.ndarray:
    """Every rounding boundary of the format (midpoints, codes, +-1 and 2
    float32 steps, overflow, NaN), both signs, then random bit patterns."""
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(tdt).float().numpy()
    fin = np.unique(np.abs(vals[np.isfinite(vals)])).astype(np.float32)
    mids = ((fin[:-1].astype(np.float64) + fin[1:]) / 2).astype(np.float32)
    extra = np.array([448, 464, 480, 57344, 61440, 65536, 1e30, np.inf, np.nan, 0, 1e-40, 1e-45], np.float32)
    base = np.concatenate([fin, mids, extra])
    pts, up, dn = [base], base, base
    for _ in range(2):
        up, dn = np.nextafter(up, np.float32(np.inf)), np.nextafter(dn, np.float32(0))
        pts += [up, dn]
    x = np.concatenate(pts).astype(np.float32)
    g = np.random.default_rng(21)
    rnd = g.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([x, -x, rnd])


@pytest.mark.parametrize("odt,tdt", F8)
def test_f8_encode_bit_exact(gpu, odt, tdt):
    x = sweep(tdt)
    src = torch.from_numpy(x).to(DEV)
    dst = torch.empty(x.shape, dtype=tdt, device=DEV)
    gpu.copy(src, dst)
    torch.cuda.synchronize()
    got = dst.view(torch.uint8).cpu().numpy()
    want = orc.cast(x, orc.F32, odt)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    # and from the other float types and integers (through float32)
    g = np.random.default_rng(22)
    for sdt, tsrc in ((orc.F64, torch.float64), (orc.F16, torch.float16), (orc.BF16, torch.bfloat16),
                      (orc.I32, torch.int32)):
        t = torch.from_numpy(g.standard_normal(50000) * 300).to(tsrc)
        d = torch.empty(t.shape, dtype=tdt, device=DEV)
        gpu.copy(t.to(DEV), d)
        torch.cuda.synchronize()
        s = t.numpy() if t.element_size() != 2 else t.view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(d.view(torch.uint8).cpu().numpy(), orc.cast(s, sdt, odt)), tsrc


@pytest.mark.parametrize("odt,tdt", F8)
def test_f8_decode_bit_exact(gpu, odt, tdt):
    codes = np.tile(np.arange(256, dtype=np.uint8), 33)
    src = torch.from_numpy(codes).view(tdt).to(DEV)
    nan = np.isnan(torch.from_numpy(codes).view(tdt).float().numpy())
    for ddt, tout, bits in ((orc.F32, torch.float32, torch.int32), (orc.F64, torch.float64, torch.int64),
                            (orc.F16, torch.float16, torch.int16), (orc.BF16, torch.bfloat16, torch.int16),
                            (orc.BOOL, torch.bool, torch.uint8), (orc.F8E4M3FN, torch.float8_e4m3fn, torch.uint8),
                            (orc.F8E5M2, torch.float8_e5m2, torch.uint8)):
        dst = torch.empty(codes.shape, dtype=tout, device=DEV)
        gpu.copy(src, dst)
        torch.cuda.synchronize()
        got = dst.view(bits).cpu().numpy()
        # a same-dtype copy moves the stored bytes (every NaN code kept)
        want = codes if ddt == odt else orc.cast(codes, odt, ddt).view(got.dtype)
        # NaN payloads are compared where they are defined: float32 (the
        # decoded value itself) and the float8 codes
        keep = np.ones(codes.shape, bool) if ddt in (orc.F32, orc.F8E4M3FN, orc.F8E5M2, orc.BOOL) else ~nan
        assert np.array_equal(got[keep], want[keep]), tout
        if not keep.all():
            assert torch.isnan(dst.float().cpu()[torch.from_numpy(nan)]).all(), tout
    # integers: finite codes only (NaN and infinity to an integer have no defined value)
    fin = np.isfinite(torch.from_numpy(codes).view(tdt).float().numpy())
    dst = torch.empty(codes.shape, dtype=torch.int32, device=DEV)
    gpu.copy(src, dst)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy()[fin], orc.cast(codes, odt, orc.I32)[fin])


@pytest.mark.parametrize("odt,tdt", F8)
def test_f8_strided_and_transposed_copies(gpu, odt, tdt):
    g = np.random.default_rng(23)
    codes = g.integers(0, 256, (300, 260), dtype=np.uint8)
    src = torch.from_numpy(codes).view(tdt).to(DEV)
    dst = torch.empty((260, 300), dtype=tdt, device=DEV)
    gpu.copy(src.t(), dst)                                 # same-dtype transpose: raw bytes
    f = torch.empty((260, 300), dtype=torch.float32, device=DEV)
    gpu.copy(src.t(), f)                                   # decode through the transpose kernel
    back = torch.empty((150, 130), dtype=tdt, device=DEV)
    gpu.copy(f[::2, ::2].t(), back)                        # strided encode
    torch.cuda.synchronize()
    assert np.array_equal(dst.view(torch.uint8).cpu().numpy(), codes.T)
    assert np.array_equal(f.cpu().numpy().view(np.uint32), orc.cast(codes.T, odt, orc.F32).view(np.uint32))
    want = orc.cast(orc.cast(codes.T, odt, orc.F32)[::2, ::2].T, orc.F32, odt)
    assert np.array_equal(back.view(torch.uint8).cpu().numpy(), want)


@pytest.mark.parametrize("tdt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_f8_on_the_vulkan_device(gpu, strict, tdt):
    import torchvulkan_amd  # noqa: F401

    x = torch.from_numpy(sweep(tdt)[:200000])
    assert torch.equal(x.to(V).to(tdt).view(torch.uint8).cpu(), x.to(tdt).view(torch.uint8))
    codes = torch.arange(256, dtype=torch.uint8).view(tdt)
    assert torch.equal(codes.to(V).float().cpu().view(torch.int32), codes.float().view(torch.int32))
    assert torch.equal(codes.to(V).to(torch.float8_e5m2 if tdt == torch.float8_e4m3fn else torch.float8_e4m3fn)
                       .view(torch.uint8).cpu(),
                       codes.to(torch.float8_e5m2 if tdt == torch.float8_e4m3fn else torch.float8_e4m3fn).view(torch.uint8))
    t = torch.empty((17, 5), dtype=tdt, device=V)
    t.fill_(-3.3)
    assert torch.equal(t.view(torch.uint8).cpu(), torch.full((17, 5), -3.3).to(tdt).view(torch.uint8))


@pytest.mark.parametrize("dt,tdt", [(orc.F32, torch.float32), (orc.F64, torch.float64), (orc.F16, torch.float16),
                                    (orc.BF16, torch.bfloat16)])
def test_binary_div_bit_exact(gpu, dt, tdt):
    g = np.random.default_rng(24)
    a = torch.from_numpy(g.standard_normal((300, 200)) * 10).to(tdt)
    b = torch.from_numpy(g.standard_normal((200,))).to(tdt)
    b[:6] = torch.tensor([0.0, -0.0, float("inf"), 1e-30, 3.0, -7.0]).to(tdt)
    out = torch.empty((300, 200), dtype=tdt, device=DEV)
    gpu.binary(a.to(DEV), b.to(DEV), out, gpu.TVK_BIN_DIV)
    torch.cuda.synchronize()
    store = lambda t: t.view(torch.int16).numpy().view(np.uint16) if t.element_size() == 2 else t.numpy()
    want = orc.binary(store(a), store(b), dt, orc.BIN_DIV)
    got = store(out.cpu())
    if dt == orc.F64:
        assert np.array_equal(got, want, equal_nan=True)
    elif dt == orc.F32:
        assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    else:
        f = orc.to_f32(want, dt)
        assert np.array_equal(got[~np.isnan(f)], want[~np.isnan(f)])
    with pytest.raises(gpu.TvkUnsupported):
        o = torch.empty(4, dtype=torch.int32, device=DEV)
        gpu.binary(torch.ones(4, dtype=torch.int32, device=DEV), torch.ones(4, dtype=torch.int32, device=DEV), o,
                   gpu.TVK_BIN_DIV)


def crand(g, shape, dt):
    return (g.standard_normal(shape) + 1j * g.standard_normal(shape)).astype(dt)


def bits_equal(got: torch.Tensor, want: np.ndarray, what: str):
    g = got.detach().cpu().numpy()
    assert g.shape == want.shape and g.dtype == want.dtype, (what, g.shape, want.shape, g.dtype, want.dtype)
    w = np.ascontiguousarray(want)
    iv = np.uint64 if g.dtype == np.complex128 else np.uint32
    bad = int((np.ascontiguousarray(g).view(iv) != w.view(iv)).sum())
    assert bad == 0, f"{what}: {bad} of {2 * g.size} parts differ from the oracle"


@pytest.mark.parametrize("cdt,tdt", [(np.complex64, torch.complex64), (np.complex128, torch.complex128)])
def test_complex_products_bit_exact(gpu, strict, cdt, tdt):
    import torchvulkan_amd  # noqa: F401

    g = np.random.default_rng(25)
    a, b = crand(g, (37, 90), cdt), crand(g, (90, 45), cdt)
    c = crand(g, (37, 45), cdt)
    av, bv, cv = (torch.from_numpy(t).to(V) for t in (a, b, c))
    bits_equal(torch.mm(av, bv), orc.complex_gemm(a, b), "mm")
    bits_equal(av @ bv, orc.complex_gemm(a, b), "matmul")
    for alpha, beta in ((1, 1), (0.5 - 2j, 1.5 + 0.25j), (2, 0)):
        bits_equal(torch.addmm(cv, av, bv, beta=beta, alpha=alpha), orc.complex_gemm(a, b, c, alpha=alpha, beta=beta),
                   f"addmm {alpha} {beta}")
    # conjugate, transposed and adjoint views: no copy is materialised on the way in
    bits_equal(torch.mm(av.conj(), bv), orc.complex_gemm(np.conj(a), b), "mm conj")
    bt = crand(g, (45, 90), cdt)
    bits_equal(torch.mm(av, torch.from_numpy(bt).to(V).mH), orc.complex_gemm(a, np.conj(bt).T), "mm adjoint")
    bits_equal(torch.mm(av, torch.from_numpy(bt).to(V).t()), orc.complex_gemm(a, bt.T), "mm transposed")
    # batched, broadcast bias
    x, y, z = crand(g, (4, 20, 33), cdt), crand(g, (4, 33, 18), cdt), crand(g, (18,), cdt)
    xv, yv, zv = (torch.from_numpy(t).to(V) for t in (x, y, z))
    bits_equal(torch.bmm(xv, yv), orc.complex_gemm(x, y), "bmm")
    zb = np.broadcast_to(z, (4, 20, 18))
    bits_equal(torch.baddbmm(zv.expand(4, 20, 18), xv, yv, beta=-1j, alpha=3),
               orc.complex_gemm(x, y, zb, alpha=3, beta=-1j), "baddbmm")
    # matrix-vector, and K = 0
    v = crand(g, (90,), cdt)
    bits_equal(torch.mv(av, torch.from_numpy(v).to(V)), orc.complex_gemm(v[None, :], a.T)[0], "mv")
    e = torch.mm(torch.empty((5, 0), dtype=tdt, device=V), torch.empty((0, 7), dtype=tdt, device=V))
    assert torch.equal(e.cpu(), torch.zeros((5, 7), dtype=tdt))
    # out= and in-place forms land in the given tensor
    out = torch.empty((37, 45), dtype=tdt, device=V)
    torch.mm(av, bv, out=out)
    bits_equal(out, orc.complex_gemm(a, b), "mm.out")


def test_conjugate_and_negative_views(gpu, strict):
    # copies of views with a pending conjugation or negation resolve them on the
    # device (the generic math-bit fallback would recurse through _copy_from)
    import torchvulkan_amd  # noqa: F401

    g = np.random.default_rng(28)
    a = crand(g, (33, 20), np.complex64)
    av = torch.from_numpy(a).to(V)
    assert np.array_equal(av.conj().cpu().numpy(), np.conj(a))
    assert np.array_equal(torch._neg_view(av).cpu().numpy(), -a)
    w = torch.empty_like(av)
    w.copy_(av.conj())
    assert np.array_equal(w.cpu().numpy(), np.conj(a))
    c = av.conj().clone()
    assert not c.is_conj() and np.array_equal(c.cpu().numpy(), np.conj(a))
    w.conj().copy_(av)                       # writing through a conjugate view stores conj(values)
    assert np.array_equal(w.cpu().numpy(), np.conj(a))
    r = torch.from_numpy(g.standard_normal((5, 7)).astype(np.float32))
    assert np.array_equal(torch._neg_view(r.to(V)).cpu().numpy(), -r.numpy())
    v = crand(g, (20,), np.complex64)
    got = torch.mv(av.conj(), torch.from_numpy(v).to(V))   # mv resolves the view first, then the product
    bits_equal(got, orc.complex_gemm(v[None, :], np.conj(a).T)[0], "mv of a conjugate")


def test_complex32_product(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    g = np.random.default_rng(26)
    a, b = crand(g, (24, 40), np.complex64), crand(g, (40, 16), np.complex64)
    ah, bh = torch.from_numpy(a).to(torch.complex32), torch.from_numpy(b).to(torch.complex32)
    got = torch.mm(ah.to(V), bh.to(V))
    assert got.dtype == torch.complex32
    # the parts widened to float32, multiplied there, rounded once to float16
    want = orc.complex_gemm(ah.to(torch.complex64).numpy(), bh.to(torch.complex64).numpy())
    want16 = torch.from_numpy(want).to(torch.complex32)
    assert torch.equal(torch.view_as_real(got.cpu()).view(torch.int16), torch.view_as_real(want16).view(torch.int16))


@pytest.mark.parametrize("fa,fb", [(orc.F8E4M3FN, orc.F8E4M3FN), (orc.F8E4M3FN, orc.F8E5M2)])
def test_scaled_mm_bit_exact(gpu, strict, fa, fb):
    import torchvulkan_amd  # noqa: F401

    tdt = {orc.F8E4M3FN: torch.float8_e4m3fn, orc.F8E5M2: torch.float8_e5m2}
    g = np.random.default_rng(27)
    M, K, N = 48, 256, 40
    a = torch.from_numpy(g.standard_normal((M, K)).astype(np.float32) * 3).to(tdt[fa])
    b = torch.from_numpy(g.standard_normal((N, K)).astype(np.float32) * 3).to(tdt[fb]).t()   # column-major, as callers pass it
    ac, bc = a.view(torch.uint8).numpy(), b.contiguous().view(torch.uint8).numpy()
    av, bv = a.to(V), b.to(V)   # b keeps its column-major strides on the device
    sa, sb = torch.tensor(0.75), torch.tensor(1.5)
    cases = [
        dict(out_dtype=torch.float32, od=orc.F32),
        dict(out_dtype=torch.bfloat16, od=orc.BF16),
        dict(out_dtype=torch.float16, od=orc.F16),
        dict(out_dtype=torch.float8_e4m3fn, od=orc.F8E4M3FN, scale_result=torch.tensor(8.0)),
    ]
    for c in cases:
        kw = {k: v for k, v in c.items() if k != "od"}
        if "scale_result" in kw:
            kw["scale_result"] = kw["scale_result"].to(V)
        got = torch._scaled_mm(av, bv, sa.to(V), sb.to(V), **kw)
        want = orc.scaled_mm(ac, fa, bc, fb, 0.75, 1.5, c["od"],
                             scale_result=8.0 if "scale_result" in c else None)
        gb = got.cpu()
        gb = gb.numpy() if gb.dtype == torch.float32 else gb.view(torch.uint8 if gb.element_size() == 1 else torch.int16) \
            .numpy().view(np.uint8 if gb.element_size() == 1 else np.uint16)
        assert np.array_equal(gb.view(want.dtype), want), c["out_dtype"]
    # row-wise scales and a bfloat16 bias
    sa2 = torch.from_numpy(g.random((M, 1)).astype(np.float32) + 0.5)
    sb2 = torch.from_numpy(g.random((1, N)).astype(np.float32) + 0.5)
    bias = torch.from_numpy(g.standard_normal(N).astype(np.float32)).bfloat16()
    got = torch._scaled_mm(av, bv, sa2.to(V), sb2.to(V), bias=bias.to(V), out_dtype=torch.float32)
    want = orc.scaled_mm(ac, fa, bc, fb, sa2.numpy(), sb2.numpy(), orc.F32,
                         bias=bias.view(torch.int16).numpy().view(np.uint16), bias_dt=orc.BF16)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # the default output dtype is the first operand's
    assert torch._scaled_mm(av, bv, sa.to(V), sb.to(V)).dtype == tdt[fa]


def test_scaled_mm_errors_match_cpu(gpu, strict):
    import torchvulkan_amd  # noqa: F401

    a = torch.randn(8, 16).to(torch.float8_e4m3fn)
    b = torch.randn(16, 8).to(torch.float8_e4m3fn)
    bad = [
        (a.float(), b, torch.tensor(1.0), torch.tensor(1.0)),           # not float8
        (a, b[:8], torch.tensor(1.0), torch.tensor(1.0)),               # shapes
        (a, b, torch.ones(3), torch.tensor(1.0)),                        # scaling configuration
        (a, b, torch.tensor(1.0, dtype=torch.float64), torch.tensor(1.0)),
    ]
    for args in bad:
        with pytest.raises((RuntimeError, ValueError)):
            torch._scaled_mm(*(t.to(V) for t in args))
