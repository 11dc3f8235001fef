"""CPU checks of the GEMM kernel-choice table (no kernel runs): the candidate
sets, recording a choice for a shape class, and the tuning file's rules after
the reference's tuner (src/vulkan/autotuner.cpp:56-121): a later line wins,
lines of another format are skipped, a recorded kernel that does not apply to
a product is ignored, TORCHVULKAN_PIPELINE_CACHE=0 keeps nothing on disk and
TORCHVULKAN_CACHE_DIR moves the file (src/vulkan/cache.cpp:181-202)."""
import ctypes as C

import pytest

from torchvulkan_amd import _abi


def _desc(M, N, K, dtype=_abi.TVK_F16, batch=1, a_stride=None, b_stride=None, flags=0):
    d = _abi.GemmDesc()
    d.dtype, d.batch, d.M, d.N, d.K, d.flags = dtype, batch, M, N, K, flags
    d.a, d.b, d.c = 256, 256, 256   # never dereferenced without a launch
    d.a_stride = _abi.I64x3(*(a_stride or (M * K, K, 1)))
    d.b_stride = _abi.I64x3(*(b_stride or (K * N, N, 1)))
    d.c_stride = _abi.I64x3(M * N, N, 1)
    return d


def candidates(d):
    buf = C.create_string_buffer(4096)
    assert _abi.load().tvk_gemm_candidates(C.byref(d), buf, 4096) == _abi.TVK_OK, _abi.load().tvk_last_error()
    return buf.value.decode().split("\n")


def plan(d):
    buf = C.create_string_buffer(128)
    assert _abi.load().tvk_gemm_plan(C.byref(d), buf, 128) == _abi.TVK_OK
    return buf.value.decode()


def choose(d, kernel, persist=0):
    return _abi.load().tvk_gemm_choose(C.byref(d), kernel.encode(), persist)


@pytest.fixture(autouse=True)
def fresh_table(tmp_path, monkeypatch):
    monkeypatch.setenv("TORCHVULKAN_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("TORCHVULKAN_PIPELINE_CACHE", raising=False)
    _abi.tune_reset()
    yield tmp_path
    _abi.tune_reset()


def test_candidate_sets():
    big = candidates(_desc(8192, 8192, 8192))
    assert big[0] == "gemm16_dma_256x256" == plan(_desc(8192, 8192, 8192))
    assert {"gemm16_mfma_128x128", "gemm16_dma_128x128", "gemm16_mfma_256x256_w8", "gemm16_mfma_256x256",
            "gemm16_mfma_128x128_splitk:2"} <= set(big)
    assert len(big) == len(set(big))
    # split-K partials are capped at 512 MB: 16 chunks of an 8192^2 float32 output are not offered
    assert "gemm16_mfma_128x128_splitk:4" not in big
    assert "gemm16_mfma_128x128_splitk:16" in candidates(_desc(1024, 1024, 8192))
    # float32 (and exact mode): only the sequential-order kernels
    assert candidates(_desc(1024, 1024, 1024, _abi.TVK_F32)) == [
        "gemm_seq_mfma_64x64", "gemm_seq_mfma_128x128", "gemm_seq_mfma_64x128"]
    assert set(candidates(_desc(512, 512, 512, flags=_abi.TVK_GEMM_EXACT))) == {
        "gemm_seq_mfma_128x128", "gemm_seq_mfma_64x128", "gemm_seq_mfma_64x64"}
    # M <= 16: the streaming kernel first, the tiled kernels after it
    sk = candidates(_desc(16, 14336, 4096))
    assert sk[0] == "gemm16_skinny_ring_splitk" and "gemm16_mfma_128x128" in sk
    assert not any(n.startswith("gemm16_mfma_256") for n in sk)
    # K not a multiple of the LDS ring's k step: no ring kernels
    assert not any("dma" in n for n in candidates(_desc(1024, 1024, 1000)))
    # no alternatives: K == 0, and operands no tiled kernel reads
    assert candidates(_desc(4, 4, 0)) == ["gemm_k0_fill"]
    assert candidates(_desc(8, 4, 4, a_stride=(0, 3, 5))) == ["gemm_generic"]


def test_choice_covers_the_shape_class():
    d = _desc(8192, 8192, 8192)
    assert choose(d, "gemm16_mfma_128x128") == _abi.TVK_OK
    assert plan(d) == "gemm16_mfma_128x128"
    # same class: ceil(log2) of every dimension and the same layout facts
    assert plan(_desc(8000, 8000, 8000)) == "gemm16_mfma_128x128"
    # other classes keep the shape's own kernel
    assert plan(_desc(4096, 8192, 8192)) == "gemm16_dma_256x256"
    assert plan(_desc(8192, 8192, 8192, _abi.TVK_BF16)) == "gemm16_dma_256x256"
    assert choose(d, "gemm16_mfma_128x128_splitk:2") == _abi.TVK_OK
    assert plan(d) == "gemm16_mfma_128x128_splitk"
    _abi.tune_reset()
    assert plan(d) == "gemm16_dma_256x256"


def test_rejects_kernels_that_do_not_compute_the_product():
    lib = _abi.load()
    assert choose(_desc(1024, 1024, 1024, _abi.TVK_F32), "gemm16_dma_128x128") == _abi.TVK_ERR_INVALID
    assert b"does not compute this product" in lib.tvk_last_error()
    assert choose(_desc(64, 64, 64), "no_such_kernel") == _abi.TVK_ERR_INVALID
    assert choose(_desc(64, 64, 0), "gemm_k0_fill") == _abi.TVK_ERR_INVALID
    buf = C.create_string_buffer(8)
    assert lib.tvk_gemm_candidates(C.byref(_desc(8192, 8192, 8192)), buf, 8) == _abi.TVK_ERR_INVALID


def test_recorded_kernel_outside_the_product_is_ignored():
    # M = 128 and M = 100 share a class; the 256-row tiles are candidates only from M >= 128
    assert choose(_desc(128, 128, 4096), "gemm16_mfma_256x256_w8") == _abi.TVK_OK
    assert plan(_desc(128, 128, 4096)) == "gemm16_mfma_256x256_w8"
    assert "gemm16_mfma_256x256_w8" not in candidates(_desc(100, 128, 4096))
    assert plan(_desc(100, 128, 4096)) == plan(_desc(100, 128, 4096)) != "gemm16_mfma_256x256_w8"


def test_tuning_file_persists_and_later_lines_win(fresh_table):
    path = _abi.tune_path()
    assert path.startswith(str(fresh_table)) and path.endswith(".txt")
    d = _desc(2048, 2048, 2048)
    assert choose(d, "gemm16_mfma_256x256", persist=1) == _abi.TVK_OK
    assert choose(d, "gemm16_dma_128x128", persist=1) == _abi.TVK_OK
    lines = open(path).read().splitlines()
    assert len(lines) == 2 and all(l.split()[:2] == ["tvk1", "gemm"] for l in lines)
    assert lines[1].split()[3] == "gemm16_dma_128x128"
    _abi.tune_reset()
    assert plan(d) == "gemm16_dma_128x128"      # read back from the file
    # a line of another format is skipped; a memory-only choice leaves the file alone
    key = lines[0].split()[2]
    with open(path, "a") as f:
        f.write(f"tvk0 gemm {key} gemm16_mfma_256x256\n")
    _abi.tune_reset()
    assert plan(d) == "gemm16_dma_128x128"
    assert choose(d, "gemm16_mfma_128x128", persist=0) == _abi.TVK_OK
    assert len(open(path).read().splitlines()) == 3


def test_persistence_off(monkeypatch, fresh_table):
    monkeypatch.setenv("TORCHVULKAN_PIPELINE_CACHE", "0")
    _abi.tune_reset()
    assert _abi.tune_path() == ""
    d = _desc(2048, 2048, 2048)
    assert choose(d, "gemm16_mfma_256x256", persist=1) == _abi.TVK_OK
    assert plan(d) == "gemm16_mfma_256x256"
    assert list(fresh_table.iterdir()) == []
