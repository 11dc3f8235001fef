"""Every kernel the GEMM kernel-choice table can hold computes the product.

Each candidate tvk_gemm_candidates offers for a case is recorded with
tvk_gemm_choose and run through tvk_gemm, then held to the parity bar of the
other GEMM tests: float32 and TVK_GEMM_EXACT bit-equal to the oracle's
sequential order, float16/bfloat16 within the north_star tolerance of the
oracle. Cases cover a ragged product with repacked operands, split-K, the
M <= 16 streaming kernel and the tiled kernels beside it, transposed and
batched operands, and a bias with gelu. Then tvk_gemm_tune: it records one
candidate per shape class, persists it once, and its timed launches never
change an operand (c is the bias of an in-place baddbmm)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gemm_cases import assert_bit_exact, assert_close, decode, oracle_mm, randn, to_np
from torchvulkan_amd import _abi

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def fresh_table(tmp_path, monkeypatch):
    monkeypatch.setenv("TORCHVULKAN_CACHE_DIR", str(tmp_path))
    _abi.tune_reset()
    yield tmp_path
    _abi.tune_reset()


def operands(M, N, K, batch, ta, tb, dtype, seed):
    sa = (batch, K, M) if ta else (batch, M, K)
    sb = (batch, N, K) if tb else (batch, K, N)
    a = randn(sa, dtype, seed)
    b = randn(sb, dtype, seed + 1)
    a = a.transpose(1, 2) if ta else a
    b = b.transpose(1, 2) if tb else b
    if batch == 1:
        a, b = a[0], b[0]
    return a, b


def device_view(t):
    base = t.as_strided((t.untyped_storage().nbytes() // t.element_size(),), (1,), 0).to(DEV)
    return base.as_strided(t.shape, t.stride(), t.storage_offset())


CASES = [
    # M, N, K, batch, A transposed, B transposed, dtype, bias + gelu, exact
    (1000, 3000, 777, 1, False, False, torch.float16, False, False),    # rows not 16-byte aligned: repacks
    (256, 1024, 4096, 1, False, True, torch.bfloat16, False, False),    # few tiles, long K: split-K plans
    (16, 2048, 1024, 1, False, False, torch.float16, False, False),     # streaming kernel and tiled ones
    (300, 520, 256, 1, False, True, torch.bfloat16, True, False),       # bias + gelu epilogue
    (128, 256, 512, 4, True, False, torch.float16, False, False),       # batched, A m-contiguous
    (1024, 1024, 1024, 1, False, False, torch.float32, False, False),   # C1: sequential order, bit-exact
    (130, 257, 320, 1, True, True, torch.float16, False, True),         # exact mode, bit-exact
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}b{c[3]}{str(c[6])[6:]}")
def test_every_candidate_computes_the_product(gpu, case):
    M, N, K, batch, ta, tb, dtype, epi, exact = case
    a, b = operands(M, N, K, batch, ta, tb, dtype, 70)
    bias = randn((N,), dtype, 72) if epi else None
    act = _abi.TVK_ACT_GELU if epi else _abi.TVK_ACT_NONE
    kw = dict(bias=None if bias is None else bias.to(DEV), alpha=1.0, beta=1.0 if epi else 0.0, activation=act,
              exact=exact)
    ref = oracle_mm(a, b, dtype, bias=bias, beta=1.0 if epi else 0.0,
                    act=orc.ACT_GELU if epi else orc.ACT_NONE)
    da, db = device_view(a), device_view(b)
    c = torch.empty(((batch,) if batch > 1 else ()) + (M, N), dtype=dtype, device=DEV)
    names = _abi.gemm_candidates(da, db, c, **kw)
    assert len(names) >= 2, names
    for name in names:
        print(f"case {case} kernel {name}", flush=True)
        _abi.tune_reset()
        _abi.gemm_choose(da, db, c, name, **kw)
        assert _abi.gemm_plan(da, db, c, **kw) == name.split(":")[0]
        c.fill_(float("nan"))
        _abi.gemm(da, db, c, **kw)
        torch.cuda.synchronize()
        got = decode(to_np(c), dtype)
        if dtype == torch.float32 or exact:
            assert_bit_exact(got, ref, name)
        else:
            assert_close(got, ref, dtype, name)


def test_tune_records_once_and_keeps_operands(gpu, fresh_table):
    # in-place baddbmm: c is the bias, so the timed launches must not accumulate into it
    dtype = torch.float16
    a, b = operands(512, 512, 512, 1, False, False, dtype, 80)
    inp = randn((512, 512), dtype, 82)
    ref = oracle_mm(a, b, dtype, bias=inp, alpha=0.5, beta=1.0)
    da, db, dc = a.to(DEV), b.to(DEV), inp.to(DEV)
    name = _abi.gemm_tune(da, db, dc, bias=dc, alpha=0.5, beta=1.0)
    torch.cuda.synchronize()
    assert name in _abi.gemm_candidates(da, db, dc, bias=dc, alpha=0.5, beta=1.0)
    assert_close(decode(to_np(dc), dtype), ref, dtype, f"tuned {name}")
    lines = open(_abi.tune_path()).read().splitlines()
    assert len(lines) == 1 and lines[0].split()[3] == name
    # recorded: the next call of the class runs it without timing again
    assert _abi.gemm_plan(da, db, dc, bias=dc, alpha=0.5, beta=1.0) == name.split(":")[0]
    dc2 = inp.to(DEV)
    assert _abi.gemm_tune(da, db, dc2, bias=dc2, alpha=0.5, beta=1.0) == name
    torch.cuda.synchronize()
    assert np.array_equal(to_np(dc2), to_np(dc))
    assert len(open(_abi.tune_path()).read().splitlines()) == 1


def test_tune_fp32_stays_bit_exact(gpu):
    a, b = operands(1024, 1024, 1024, 1, False, False, torch.float32, 90)
    da, db = a.to(DEV), b.to(DEV)
    c = torch.empty((1024, 1024), device=DEV)
    name = _abi.gemm_tune(da, db, c)
    torch.cuda.synchronize()
    assert name.startswith("gemm_seq_mfma")
    assert_bit_exact(decode(to_np(c), torch.float32), oracle_mm(a, b, torch.float32), name)


def test_backend_autotune_on_first_sight(gpu, tmp_path):
    # TORCHVULKAN_AUTOTUNE=1 is read once per process: a child process runs the matmuls
    import os
    import subprocess
    import sys

    script = (
        "import torch, torchvulkan_amd\n"
        "g = torch.Generator().manual_seed(5)\n"
        "a = torch.randn(384, 640, generator=g).half(); b = torch.randn(640, 512, generator=g).half()\n"
        "for _ in range(2):\n"
        "    got = torch.mm(a.to('vulkan'), b.to('vulkan')).cpu().double()\n"
        "    ref = a.double() @ b.double()\n"
        "    assert ((got - ref).abs() <= 5e-3 * (ref.abs() + 1)).all()\n"
        "print('ok', flush=True)\n"
    )
    env = dict(os.environ, TORCHVULKAN_AUTOTUNE="1", TORCHVULKAN_CACHE_DIR=str(tmp_path))
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", script], env=env, cwd=root, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr
    files = list(tmp_path.glob("tuning-*.txt"))
    assert len(files) == 1
    lines = files[0].read_text().splitlines()
    assert len(lines) == 1 and lines[0].split()[:2] == ["tvk1", "gemm"]   # tuned once, then read from the table


def test_ahead_of_time_tuner_records_fastest(gpu, fresh_table, capsys):
    from torchvulkan_amd import tune

    assert tune.main(["--shape", "512x768x1024:f16:nt", "--shape", "96x96x96:bf16:tn:3:c", "--record"]) == 0
    out = capsys.readouterr().out
    assert out.count("| 512x768x1024") == 1 and "recorded in" in out
    lines = open(_abi.tune_path()).read().splitlines()
    assert len(lines) == 2 and all(l.startswith("tvk1 gemm ") for l in lines)
