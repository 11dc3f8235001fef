"""CPU checks of the C ABI: the library loads, exports every entry point that
include/tvk_hip.h declares, and rejects bad descriptors with the documented
status codes. No compute is launched (there is no GPU here)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from torchvulkan_amd import _abi

ROOT = Path(__file__).resolve().parent.parent


def declared_entry_points() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tvk_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = _abi.load()
    names = declared_entry_points()
    assert "tvk_gemm" in names and "tvk_malloc" in names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(_abi._ALL_ENTRY_POINTS) <= names


def test_device_count_without_gpu_is_not_an_error():
    assert _abi.device_count() >= 0


def test_gemm_rejects_null_desc():
    lib = _abi.load()
    assert lib.tvk_gemm(None) == _abi.TVK_ERR_INVALID
    assert b"desc is NULL" in lib.tvk_last_error()


def _desc(**kw):
    d = _abi.GemmDesc()
    d.dtype, d.batch, d.M, d.N, d.K = _abi.TVK_F16, 1, 4, 4, 4
    d.a, d.b, d.c = 16, 16, 16   # never dereferenced by validation
    d.a_stride = _abi.I64x3(0, 4, 1)
    d.b_stride = _abi.I64x3(0, 4, 1)
    d.c_stride = _abi.I64x3(0, 4, 1)
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("field,value,status", [
    ("dtype", 9, _abi.TVK_ERR_UNSUPPORTED),   # BOOL: every other dtype has a kernel
    ("activation", 9, _abi.TVK_ERR_INVALID),
    ("M", -1, _abi.TVK_ERR_INVALID),
    ("K", 1 << 40, _abi.TVK_ERR_UNSUPPORTED),
    ("c", None, _abi.TVK_ERR_INVALID),
])
def test_gemm_validation_codes(field, value, status):
    lib = _abi.load()
    d = _desc(**{field: value})
    assert lib.tvk_gemm(C.byref(d)) == status
    assert lib.tvk_last_error()


@pytest.mark.parametrize("a_stride,b_stride,dtype,M,N,K,want", [
    ((0, 8192, 1), (0, 8192, 1), _abi.TVK_F16, 8192, 8192, 8192, "gemm16_dma_256x256"),
    ((0, 1, 8192), (0, 1, 8192), _abi.TVK_BF16, 8192, 8192, 4096, "gemm16_dma_256x256"),
    ((0, 8200, 1), (0, 8192, 1), _abi.TVK_F16, 8192, 8192, 8200, "gemm16_mfma_256x256_w8"),   # K % 32 != 0
    ((0, 8193, 1), (0, 8192, 1), _abi.TVK_F16, 8192, 8192, 8192, "gemm16_dma_256x256"),   # rows not 16 B aligned: A repacked
    ((0, 777, 1), (0, 3000, 1), _abi.TVK_F16, 1000, 3000, 777, "gemm16_dma_128x128"),       # C5 ragged, A repacked (rows padded to 32 with zeros)
    ((0, 1000, 1), (0, 1000, 1), _abi.TVK_F16, 1000, 1000, 1000, "gemm16_mfma_64x64"),    # 64 tiles of 128^2
    ((0, 4096, 1), (0, 1, 4096), _abi.TVK_F16, 256, 4096, 4096, "gemm16_dma_128x128_splitk"),
    ((0, 1, 512), (0, 512, 1), _abi.TVK_BF16, 512, 512, 8192, "gemm16_dma_128x128_splitk"),
    ((0, 4096, 1), (0, 1, 4096), _abi.TVK_F16, 256, 10, 4096, "gemm16_dma_128x128_splitk"),   # 10 columns
    ((0, 5000, 1), (0, 320, 1), _abi.TVK_F16, 384, 320, 5000, "gemm16_mfma_128x128_splitk"),    # K % 32 != 0
    ((0, 512, 1), (0, 1, 512), _abi.TVK_F16, 4096, 1024, 512, "gemm16_dma_128x128"),      # both k-contiguous, short K
    ((0, 512, 1), (0, 1024, 1), _abi.TVK_F16, 4096, 1024, 512, "gemm16_dma_128x128"),
    ((0, 512, 1), (0, 1024, 1), _abi.TVK_F16, 1024, 1024, 512, "gemm16_mfma_64x64"),      # 64 tiles of 128^2
    ((0, 512, 1), (0, 1, 512), _abi.TVK_F16, 8192, 3072, 512, "gemm16_dma_128x256"),     # 384 tiles of 256^2: 1.5 rounds
    ((0, 3072, 1), (0, 512, 1), _abi.TVK_F16, 8192, 512, 3072, "gemm16_dma_128x128"),
    ((0, 1024, 1), (0, 4096, 1), _abi.TVK_F16, 1024, 4096, 1024, "gemm16_dma_128x128"),   # K < 2048: no split
    ((0, 1, 768), (0, 768, 1), _abi.TVK_F16, 768, 768, 4096, "gemm16_dma_128x128_splitk"),
    ((0, 512, 1), (0, 512, 1), _abi.TVK_BF16, 8192, 512, 512, "gemm16_dma_128x128"),
    ((0, 4096, 1), (0, 14336, 1), _abi.TVK_F16, 16, 14336, 4096, "gemm16_skinny_ring_splitk"),
    ((0, 96, 1), (0, 32768, 1), _abi.TVK_F16, 16, 32768, 96, "gemm16_skinny_ring"),
    ((0, 2000, 1), (0, 1000, 1), _abi.TVK_F16, 7, 1000, 2000, "gemm16_skinny_bn"),
    ((0, 4096, 1), (0, 1, 4096), _abi.TVK_BF16, 8, 4096, 4096, "gemm16_skinny_bk"),
    ((0, 3, 5), (0, 4, 1), _abi.TVK_F16, 8, 4, 4, "gemm_generic"),
    ((0, 1024, 1), (0, 1024, 1), _abi.TVK_F32, 1024, 1024, 1024, "gemm_seq_mfma_64x64"),
    ((0, 2048, 1), (0, 2048, 1), _abi.TVK_F32, 2048, 2048, 2048, "gemm_seq_mfma_64x64"),
    ((0, 4096, 1), (0, 4096, 1), _abi.TVK_F32, 4096, 4096, 4096, "gemm_seq_mfma_128x128"),
    ((0, 4, 1), (0, 4, 1), _abi.TVK_BF16, 4, 4, 0, "gemm_k0_fill"),
])
def test_gemm_plan_without_gpu(a_stride, b_stride, dtype, M, N, K, want):
    lib = _abi.load()
    d = _desc(a_stride=_abi.I64x3(*a_stride), b_stride=_abi.I64x3(*b_stride), dtype=dtype, M=M, N=N, K=K)
    buf = C.create_string_buffer(64)
    assert lib.tvk_gemm_plan(C.byref(d), buf, 64) == _abi.TVK_OK
    assert buf.value.decode() == want


@pytest.mark.parametrize("a_stride,b_stride,M,N,K,want", [
    # A spans 4 GiB: tvk_gemm runs it in row blocks below 2 GiB, each on the tiled kernels
    ((0, 2048, 1), (0, 256, 1), 1 << 20, 256, 2048, "gemm16_dma_256x256"),
    # just below the boundary: one block
    ((0, 2048, 1), (0, 256, 1), 524032, 256, 2048, "gemm16_dma_256x256"),
    # B spans 4 GiB along N with K rows: column blocks
    ((0, 2048, 1), (0, 1, 2048), 512, 1 << 20, 2048, "gemm16_dma_256x256"),
    # a single k row of B spans 4 GiB (n-contiguous, k stride 2^20): no block fits, the generic kernel
    ((0, 2048, 1), (0, 1 << 20, 1), 512, 1 << 20, 2048, "gemm_generic"),
])
def test_gemm_plan_past_2gib_operands(a_stride, b_stride, M, N, K, want):
    lib = _abi.load()
    d = _desc(a_stride=_abi.I64x3(*a_stride), b_stride=_abi.I64x3(*b_stride), M=M, N=N, K=K)
    d.a, d.b, d.c = 1 << 12, 1 << 12, 1 << 12
    buf = C.create_string_buffer(64)
    assert lib.tvk_gemm_plan(C.byref(d), buf, 64) == _abi.TVK_OK
    assert buf.value.decode() == want


def test_free_rejects_foreign_pointer():
    lib = _abi.load()
    assert lib.tvk_free(C.c_void_p(0x1234)) == _abi.TVK_ERR_INVALID
    assert lib.tvk_free(None) == _abi.TVK_OK


def _convnd(**kw):
    import torch

    d = _abi.make_convnd_desc((2, 4, 5, 6, 7), (8, 4, 3, 3, 3), torch.float16, stride=1, padding=1)
    d.x = d.weight = d.y = 16   # never dereferenced by validation
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("field,value,status", [
    ("spatial_dims", 4, _abi.TVK_ERR_UNSUPPORTED),
    ("spatial_dims", 0, _abi.TVK_ERR_UNSUPPORTED),
    ("dtype", 3, _abi.TVK_ERR_UNSUPPORTED),   # float64 convolutions run as im2col + GEMM in the backend
    ("groups", 3, _abi.TVK_ERR_INVALID),
    ("c_in", 0, _abi.TVK_ERR_INVALID),
])
def test_convnd_validation(field, value, status):
    lib = _abi.load()
    d = _convnd(**{field: value})
    for fn in (lib.tvk_conv_fwd, lib.tvk_conv_dgrad, lib.tvk_conv_wgrad):
        assert fn(C.byref(d)) == status, (field, value, lib.tvk_last_error())


def test_convnd_rejects_wrong_output_size():
    lib = _abi.load()
    d = _convnd()
    d.out_size[1] = 99
    assert lib.tvk_conv_fwd(C.byref(d)) == _abi.TVK_ERR_INVALID
    assert b"out_size[1]" in lib.tvk_last_error()
    assert lib.tvk_conv_fwd(None) == _abi.TVK_ERR_INVALID


@pytest.mark.parametrize("mode,missing", [(0, "x"), (0, "weight"), (1, "y"), (1, "weight"), (2, "x"), (2, "y")])
def test_conv_rejects_null_inputs(mode, missing):
    # a direction's inputs must be given: checked before any launch (no GPU needed)
    lib = _abi.load()
    fn = (lib.tvk_conv_fwd, lib.tvk_conv_dgrad, lib.tvk_conv_wgrad)[mode]
    for d in (_convnd(), _conv2(**{})):
        setattr(d, missing, None)
        assert fn(C.byref(d)) == _abi.TVK_ERR_INVALID
        assert b"input pointer is NULL" in lib.tvk_last_error()


def _conv2(**kw):
    import torch

    d = _abi.make_convnd_desc((8, 64, 32, 32), (64, 64, 3, 3), torch.float16, stride=1, padding=1)
    d.x = d.weight = d.y = 256   # 16-byte aligned, never dereferenced here
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_conv_candidates_without_gpu():
    import torch

    lib = _abi.load()
    d = _conv2()
    for mode in (_abi.TVK_CONV_FWD, _abi.TVK_CONV_DGRAD, _abi.TVK_CONV_WGRAD):
        names = _abi.conv_candidates(d, mode)
        # the 3x3 stride-1 layer: the halo kernels first, the implicit GEMM (every problem) last
        assert names[0] == "conv_halo" and names[-1] == "conv_implicit_gemm" and len(names) >= 2, names
    f32 = _abi.make_convnd_desc((8, 64, 32, 32), (64, 64, 3, 3), torch.float32, stride=1, padding=1)
    f32.x = f32.weight = f32.y = 256
    assert _abi.conv_candidates(f32, _abi.TVK_CONV_FWD) == ["conv_implicit_gemm"]
    exact = _conv2(flags=_abi.TVK_GEMM_EXACT)
    assert _abi.conv_candidates(exact, _abi.TVK_CONV_WGRAD) == ["conv_implicit_gemm"]
    assert _abi.conv_candidates(_convnd(), _abi.TVK_CONV_FWD) == ["conv_implicit_gemm"]   # 3-D
    buf = C.create_string_buffer(64)
    assert lib.tvk_conv_candidates(C.byref(d), 3, buf, 64) == _abi.TVK_ERR_INVALID
    assert lib.tvk_conv_candidates(C.byref(d), 0, buf, 4) == _abi.TVK_ERR_INVALID   # names do not fit
    assert lib.tvk_conv_choose(C.byref(d), 0, b"no_such_family", 0) == _abi.TVK_ERR_INVALID


def test_strict_allocation_switch():
    # the reference's TORCHVULKAN_STRICT_ALLOCATION (src/vulkan/vulkan_context.cpp:248), switchable for the process
    lib = _abi.load()
    v = C.c_int(-1)
    assert lib.tvk_get_strict_allocation(C.byref(v)) == _abi.TVK_OK
    old = v.value
    try:
        for on in (1, 0):
            assert lib.tvk_set_strict_allocation(on) == _abi.TVK_OK
            assert lib.tvk_get_strict_allocation(C.byref(v)) == _abi.TVK_OK and v.value == on
    finally:
        lib.tvk_set_strict_allocation(old)
    assert lib.tvk_host_free(C.c_void_p(16)) == _abi.TVK_ERR_INVALID   # not a tvk_host_malloc block
    p = C.c_int(7)
    assert lib.tvk_host_pointer_pinned(C.c_void_p(16), C.byref(p)) == _abi.TVK_OK and p.value == 0


def test_copy_plans_without_gpu():
    """tvk_copy_plan names the kernel a copy would take (no launch): dense same-dtype and cast copies,
    a transpose, an expanded scalar into a dense destination (the broadcast fill), a permute of outer
    dimensions with whole 16-byte rows (the rows kernel), and an expanded row of 28 bytes (strided)."""
    import torch

    x = torch.zeros((64, 48), dtype=torch.float16)
    assert _abi.copy_plan(x, torch.empty((64, 48), dtype=torch.float16)) == "memcpy"
    assert _abi.copy_plan(x, torch.empty((64, 48), dtype=torch.float32)) == "cast_contig"
    assert _abi.copy_plan(x.t(), torch.empty((48, 64), dtype=torch.float16)) == "transpose"
    s = torch.tensor(1.5, dtype=torch.float32)
    for dt in (torch.float16, torch.float32, torch.bfloat16, torch.int64, torch.bool, torch.uint8):
        assert _abi.copy_plan(s.expand(300, 7), torch.empty((300, 7), dtype=dt)) == "broadcast", dt
    wide = torch.empty((300, 8), dtype=torch.float16)
    assert _abi.copy_plan(s.expand(300, 7), wide[:, :7]) == "strided"      # destination not dense
    row = torch.zeros((1, 7), dtype=torch.float32)
    assert _abi.copy_plan(row.expand(300, 7), torch.empty((300, 7))) == "strided"   # 28-byte runs
    y = torch.zeros((4, 33, 8, 64), dtype=torch.float16)
    assert _abi.copy_plan(y.transpose(1, 2), torch.empty((4, 8, 33, 64), dtype=torch.float16)) == "rows"
    assert _abi.copy_plan(y.transpose(1, 2), torch.empty((4, 8, 33, 64), dtype=torch.float32)) != "rows"
    assert _abi.copy_plan(s.expand(0, 7), torch.empty((0, 7))) == "none"
