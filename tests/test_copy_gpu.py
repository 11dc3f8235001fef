"""tvk_copy on the GPU through the C ABI: every dtype pair against the cast
oracle (bit-exact; NaN payloads aside), and strided copies (transposes,
NCHW <-> NHWC, slices, expanded sources, strided destinations, many
dimensions, empty and one-element shapes) against torch's CPU copy_, which
defines the index semantics the reference's TensorIterator follows."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from torchvulkan_amd import _abi

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TORCH_OF = {orc.F32: torch.float32, orc.F16: torch.float16, orc.BF16: torch.bfloat16, orc.F64: torch.float64,
            orc.I64: torch.int64, orc.I32: torch.int32, orc.I16: torch.int16, orc.I8: torch.int8,
            orc.U8: torch.uint8, orc.BOOL: torch.bool}
ALL = list(TORCH_OF)
FLOATS = {orc.F32, orc.F16, orc.BF16, orc.F64}
RAW = {torch.float16: torch.int16, torch.bfloat16: torch.int16}


def storage_np(t: torch.Tensor) -> np.ndarray:
    """CPU numpy view in the oracle's storage convention (raw uint16 for 16-bit floats, uint8 for bool)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in RAW:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.bool:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def source_values(dt: int, n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    td = TORCH_OF[dt]
    if dt in FLOATS:
        x = torch.randn(n, generator=g, dtype=torch.float64) * torch.exp2(torch.randint(-20, 20, (n,), generator=g).double())
        x[:16] = torch.tensor([0.0, -0.0, 1.0, -1.0, 0.5, 2.5, -2.5, 255.5, 65504.0, 65520.0, 1e30, -1e30,
                               float("inf"), -float("inf"), float("nan"), 1e-30], dtype=torch.float64)
        return x.to(td)
    if dt == orc.BOOL:
        return torch.randint(0, 2, (n,), generator=g).bool()
    info = torch.iinfo(td)
    x = torch.randint(info.min, info.max, (n,), generator=g, dtype=torch.int64)
    x[:4] = torch.tensor([info.min, info.max, 0, 1])
    return x.to(td)


def run_copy(src: torch.Tensor, dst: torch.Tensor) -> str:
    plan = _abi.copy_plan(src, dst)
    _abi.copy(src, dst)
    torch.cuda.synchronize()
    return plan


def assert_bits_equal(got: np.ndarray, want: np.ndarray, ddt: int, what: str):
    if ddt in FLOATS:
        g = got.view(np.float16) if ddt == orc.F16 else got
        w = want.view(np.float16) if ddt == orc.F16 else want
        if ddt == orc.BF16:
            g = (got.astype(np.uint32) << 16).view(np.float32)
            w = (want.astype(np.uint32) << 16).view(np.float32)
        nan_g, nan_w = np.isnan(g), np.isnan(w)
        assert (nan_g == nan_w).all(), f"{what}: NaN positions differ"
        got, want = got[~nan_g], want[~nan_w]
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{what}: {bad.size} elements differ, first at {bad[0]}: got {got[bad[0]]} want {want[bad[0]]}"


@pytest.mark.parametrize("sdt", ALL)
def test_contiguous_cast_all_pairs(gpu, sdt):
    n = 4099   # a ragged tail after the 8-element groups
    src_cpu = source_values(sdt, n + 1, sdt)
    for ddt in ALL:
        for off in (0, 1):   # 1: bases off the vector alignment
            src = src_cpu.to(DEV)[off:off + n]
            dst = torch.empty(n, dtype=TORCH_OF[ddt], device=DEV)
            plan = run_copy(src, dst)
            assert plan == ("memcpy" if sdt == ddt and sdt != orc.BOOL else "cast_contig")
            want = orc.cast(storage_np(src_cpu[off:off + n]), sdt, ddt)
            assert_bits_equal(storage_np(dst), want, ddt, f"{TORCH_OF[sdt]}->{TORCH_OF[ddt]} off {off}")


def check_like_torch(src: torch.Tensor, dst: torch.Tensor, plan: str | None = None):
    """Copies device src into device dst and compares with torch's CPU copy_ of the same views."""
    ref_dst = dst.detach().cpu()
    before = dst.detach().cpu().clone()
    ref_dst.copy_(src.detach().cpu())
    got_plan = run_copy(src, dst)
    if plan is not None:
        assert got_plan == plan, f"plan {got_plan}, expected {plan}"
    assert torch.equal(storage_view(dst.detach().cpu()), storage_view(ref_dst)), "values differ from torch's copy_"
    return before


def storage_view(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype in RAW else t


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.float16, torch.uint8])
def test_transpose_2d_and_batched(gpu, dtype):
    g = torch.Generator().manual_seed(3)
    a = (torch.randn((300, 517), generator=g) * 50).to(dtype).to(DEV)
    dst = torch.empty((517, 300), dtype=dtype, device=DEV)
    check_like_torch(a.t(), dst, "transpose")
    b = (torch.randn((5, 70, 130), generator=g) * 50).to(dtype).to(DEV)
    dst = torch.empty((5, 130, 70), dtype=dtype, device=DEV)
    check_like_torch(b.transpose(1, 2), dst, "transpose")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_nchw_nhwc_round_trip(gpu, dtype):
    g = torch.Generator().manual_seed(4)
    x = torch.randn((4, 33, 9, 11), generator=g).to(dtype).to(DEV)
    cl = torch.empty_like(x, memory_format=torch.channels_last)
    check_like_torch(x, cl, "transpose")
    back = torch.empty_like(x)
    check_like_torch(cl, back, "transpose")
    assert torch.equal(storage_view(back.cpu()), storage_view(x.cpu()))


def test_slices_expands_and_strided_destinations(gpu):
    g = torch.Generator().manual_seed(5)
    x = torch.randn((64, 90), generator=g).to(DEV)
    check_like_torch(x[::2, 1::3], torch.empty((32, 30), device=DEV), "strided")
    row = torch.randn((1, 300), generator=g).to(DEV)
    check_like_torch(row.expand(200, 300), torch.empty((200, 300), device=DEV))
    scalar = torch.tensor(2.5).to(DEV)
    check_like_torch(scalar.expand(7, 9), torch.empty((7, 9), device=DEV))
    big = torch.zeros((40, 100), device=DEV)
    check_like_torch(torch.randn((40, 50), generator=g).to(DEV), big[:, ::2])
    assert (big.cpu()[:, 1::2] == 0).all(), "elements outside the strided view changed"
    # a column of a row-major matrix into a contiguous vector, and back
    check_like_torch(x[:, 7], torch.empty(64, device=DEV))
    check_like_torch(torch.randn(64, generator=g).to(DEV), x[:, 7])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64, torch.uint8, torch.int64])
def test_rows_permute_outer_dimensions(gpu, dtype):
    """Same-dtype copies whose innermost dimension is contiguous on both sides in whole 16-byte vectors
    take the rows kernel (a permute of the outer dimensions, an expanded row, a sliced batch, a strided
    destination), bit-exact against torch's CPU copy_; runs that are not whole vectors, and casts, do
    not."""
    g = torch.Generator().manual_seed(21)
    x = (torch.randn((4, 33, 8, 64), generator=g) * 50).to(dtype).to(DEV)
    check_like_torch(x.transpose(1, 2), torch.empty((4, 8, 33, 64), dtype=dtype, device=DEV), "rows")
    check_like_torch(x.permute(2, 0, 1, 3), torch.empty((8, 4, 33, 64), dtype=dtype, device=DEV), "rows")
    check_like_torch(x[::2].transpose(1, 2), torch.empty((2, 8, 33, 64), dtype=dtype, device=DEV), "rows")
    row = (torch.randn((1, 128), generator=g) * 50).to(dtype).to(DEV)
    check_like_torch(row.expand(300, 128), torch.empty((300, 128), dtype=dtype, device=DEV), "rows")
    big = torch.zeros((33, 4, 8, 2, 64), dtype=dtype, device=DEV)
    check_like_torch(x.permute(1, 0, 2, 3), big[:, :, :, 0, :], "rows")
    assert (big[:, :, :, 1, :].cpu() == 0).all(), "wrote outside the view"
    y = (torch.randn((4, 33, 8, 3), generator=g) * 50).to(dtype).to(DEV)   # 3-element runs
    check_like_torch(y.transpose(1, 2), torch.empty((4, 8, 33, 3), dtype=dtype, device=DEV), "strided")
    if dtype != torch.float32:
        check_like_torch(x.transpose(1, 2), torch.empty((4, 8, 33, 64), dtype=torch.float32, device=DEV))


@pytest.mark.parametrize("sdt", ALL)
def test_broadcast_scalar_all_pairs(gpu, sdt):
    """An expanded scalar (stride 0 everywhere) into a dense destination: the broadcast kernel, every dtype
    pair bit-exact against the cast oracle, with destinations starting off 16-byte alignment and lengths
    that leave a head and a tail outside the 16-byte stores."""
    vals = source_values(sdt, 16, 40 + sdt)
    for i in (2, 5, 14):
        src_cpu = vals[i:i + 1].reshape(())
        src = src_cpu.to(DEV)
        for ddt in ALL:
            want = orc.cast(storage_np(src_cpu.reshape(1)), sdt, ddt)[0]
            for n, off in ((37, 0), (37, 3), (4099, 1), (3 * 1024 * 1024 + 5, 0)):
                if n > 4099 and i != 2:
                    continue
                buf = torch.zeros(n + off + 2, dtype=TORCH_OF[ddt], device=DEV)
                dst = buf[off:off + n].view(n // 1, 1) if n % 2 else buf[off:off + n].view(n // 2, 2)
                assert run_copy(src.expand(dst.shape), dst) == "broadcast"
                got = storage_np(buf)
                assert_bits_equal(got[off:off + n], np.full(n, want, dtype=got.dtype), ddt,
                                  f"{TORCH_OF[sdt]}->{TORCH_OF[ddt]} n={n} off={off}")
                assert (got[:off] == 0).all() and (got[off + n:] == 0).all(), "wrote outside the destination"


def test_many_dims_empty_and_single(gpu):
    g = torch.Generator().manual_seed(6)
    x = torch.randn((2, 3, 2, 3, 2, 3, 2, 3), generator=g).to(DEV)
    p = x.permute(7, 0, 5, 2, 3, 1, 6, 4)
    check_like_torch(p, torch.empty(p.shape, device=DEV))
    e = torch.empty((0, 5), device=DEV)
    assert run_copy(torch.empty((0, 5), device=DEV), e) == "none"
    one = torch.empty((1, 1, 1), dtype=torch.float16, device=DEV)
    src = torch.tensor([[[3.25]]], dtype=torch.float64).to(DEV)
    run_copy(src, one)
    assert one.item() == 3.25


@pytest.mark.parametrize("sdt,ddt", [(orc.F32, orc.F16), (orc.F16, orc.F32), (orc.F64, orc.BF16),
                                     (orc.I64, orc.F32), (orc.F32, orc.I32), (orc.BF16, orc.BOOL)])
def test_strided_casts(gpu, sdt, ddt):
    src_flat = source_values(sdt, 130 * 77, 20 + sdt)
    src_cpu = src_flat.view(130, 77)
    src = src_cpu.to(DEV)
    for view_fn, shape, plan in [(lambda t: t.t(), (77, 130), "transpose"), (lambda t: t[1::2, ::3], (65, 26), "strided")]:
        dst = torch.empty(shape, dtype=TORCH_OF[ddt], device=DEV)
        assert run_copy(view_fn(src), dst) == plan
        want = orc.cast(storage_np(view_fn(src_cpu)), sdt, ddt)
        assert_bits_equal(storage_np(dst).reshape(-1), want.reshape(-1), ddt, f"{TORCH_OF[sdt]}->{TORCH_OF[ddt]} {plan}")


def test_large_round_trip(gpu):
    # 2^26 half values (every pattern 1024 times) -> float32 -> half is the identity on non-NaN patterns
    pat = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).repeat(1024).to(DEV)
    h = pat.view(torch.float16)
    f = torch.empty(h.shape, dtype=torch.float32, device=DEV)
    h2 = torch.empty_like(h)
    run_copy(h, f)
    run_copy(f, h2)
    keep = ~torch.isnan(h)
    assert torch.equal(h2.view(torch.int16)[keep], pat[keep])
    # and a strided half of it through the transpose kernel
    m = h.view(4096, 16384)
    t = torch.empty((16384, 4096), dtype=torch.float16, device=DEV)
    assert run_copy(m.t(), t) == "transpose"
    assert torch.equal(t.view(torch.int16).cpu(), m.t().contiguous().view(torch.int16).cpu())


def test_rejects_bad_descriptors(gpu):
    lib = _abi.load()
    assert lib.tvk_copy(None) == _abi.TVK_ERR_INVALID
    d = _abi.make_copy_desc(torch.zeros(4, device=DEV), torch.zeros(4, device=DEV))
    d.src_dtype = 42
    assert lib.tvk_copy(d) == _abi.TVK_ERR_UNSUPPORTED
    d = _abi.make_copy_desc(torch.zeros(4, device=DEV), torch.zeros(4, device=DEV))
    d.dst_strides[0] = 0
    assert lib.tvk_copy(d) == _abi.TVK_ERR_INVALID
    assert b"overlapping" in lib.tvk_last_error()


@pytest.mark.parametrize("dtype,value", [(torch.float32, -1.5), (torch.float16, 65504.0), (torch.bfloat16, 3.0),
                                         (torch.float64, 1e-300), (torch.int64, -(2**40)), (torch.int8, -7),
                                         (torch.bool, True), (torch.uint8, 200)])
def test_fill(gpu, dtype, value):
    base = torch.zeros(1000, dtype=dtype, device=DEV)
    for lo, hi in ((0, 1000), (1, 1000), (3, 997), (5, 6)):   # heads and tails off the 16-byte grid
        _abi.fill(base[lo:hi], value)
        torch.cuda.synchronize()
        ref = torch.zeros(1000, dtype=dtype)
        ref[lo:hi] = value
        assert torch.equal(storage_view(base.cpu()), storage_view(ref)), (lo, hi)
        base.zero_()
    m = torch.zeros((30, 40), dtype=dtype, device=DEV)
    _abi.fill(m[::3, 1::2], value)
    torch.cuda.synchronize()
    ref = torch.zeros((30, 40), dtype=dtype)
    ref[::3, 1::2] = value
    assert torch.equal(storage_view(m.cpu()), storage_view(ref))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64, torch.uint8, torch.bfloat16])
def test_transpose_aligned_vector_path(gpu, dtype):
    # 16-byte aligned rows on both sides: the vectorized tile kernel, including chunks cut by the matrix edge
    g = torch.Generator().manual_seed(30)
    big = (torch.randn((200, 144), generator=g) * 50).to(dtype).to(DEV)
    for cols in (144, 132, 129):
        src = big[:, :cols]
        dst = torch.empty((cols, 200), dtype=dtype, device=DEV)
        check_like_torch(src.t(), dst, "transpose")
    x = torch.randn((4, 32, 8, 16), generator=g).to(dtype).to(DEV)
    cl = torch.empty_like(x, memory_format=torch.channels_last)
    check_like_torch(x, cl, "transpose")
    back = torch.empty_like(x)
    check_like_torch(cl, back, "transpose")
    # several 64 x 256 tiles with edge blocks on both sides (16-bit: the register-transposing kernel), batched
    for shape in ((520, 776), (3, 264, 136), (1000, 8)):
        src = (torch.randn(shape, generator=g) * 50).to(dtype).to(DEV)
        dst = torch.empty(shape[:-2] + (shape[-1], shape[-2]), dtype=dtype, device=DEV)
        check_like_torch(src.transpose(-1, -2), dst, "transpose")


@pytest.mark.parametrize("sdt,ddt", [(orc.F32, orc.F16), (orc.F16, orc.F32), (orc.BF16, orc.F32), (orc.F32, orc.BF16)])
def test_transpose_cast_vector_path(gpu, sdt, ddt):
    src_cpu = source_values(sdt, 96 * 256, 40 + sdt).view(96, 256)
    src = src_cpu.to(DEV)
    dst = torch.empty((256, 96), dtype=TORCH_OF[ddt], device=DEV)
    assert run_copy(src.t(), dst) == "transpose"
    want = orc.cast(storage_np(src_cpu.t()), sdt, ddt)
    assert_bits_equal(storage_np(dst).reshape(-1), want.reshape(-1), ddt, "vector transpose cast")
