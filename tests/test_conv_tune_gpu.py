"""Kernel choice for convolutions through the C ABI (tvk_conv_candidates,
tvk_conv_choose, tvk_conv_tune), after the reference's per-problem conv
tuning (src/api/ops/conv.cpp:499-659).

- Every candidate family of every C4 layer direction (fp16 and bf16, batch 8),
  recorded in turn in the kernel-choice table and run through the ordinary
  entry point, against the oracle; grouped and 1-D problems likewise.
- float32, TVK_GEMM_EXACT and three spatial dimensions offer one family, the
  implicit GEMM, so a recorded choice never changes an exact result; a family
  that does not apply is rejected.
- tvk_conv_tune times the candidates once per shape class, records and
  persists the fastest (a `tvk1 conv` line in the tuning file), and runs it.

Tolerances: tests/gemm_cases.py.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gemm_cases import ORC_DT, assert_bit_exact, assert_close, decode, gen, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"
FAMILIES = {"conv_stem", "conv_halo", "conv_ring", "conv_implicit_gemm"}

C4 = [
    # name, cin, cout, k, stride, pad, spatial
    ("stem_3_64", 3, 64, 3, 1, 1, 32),
    ("3x3_64_64", 64, 64, 3, 1, 1, 32),
    ("3x3_64_128_s2", 64, 128, 3, 2, 1, 32),
    ("3x3_128_256_s2", 128, 256, 3, 2, 1, 16),
    ("1x1_64_128_s2", 64, 128, 1, 2, 0, 32),
    ("1x1_128_256_s2", 128, 256, 1, 2, 0, 16),
]


@pytest.fixture
def fresh_table(gpu, tmp_path, monkeypatch):
    monkeypatch.setenv("TORCHVULKAN_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("TORCHVULKAN_PIPELINE_CACHE", raising=False)
    gpu.tune_reset()
    yield tmp_path
    gpu.tune_reset()


def _problem(shape_x, shape_w, dtype, seed, groups=1):
    x = torch.randn(shape_x, generator=gen(seed)).to(dtype)
    fan_in = int(np.prod(shape_w[1:]))
    w = (torch.randn(shape_w, generator=gen(seed + 1)) * np.sqrt(2.0 / fan_in)).to(dtype)
    b = torch.randn((shape_w[0],), generator=gen(seed + 2)).to(dtype)
    return x, w, b


def _refs(x, w, b, dy, s, p, groups, dtype, nd=2):
    od = ORC_DT[dtype]
    if nd == 3:
        y = orc.conv3d(to_np(x), to_np(w), od, bias=to_np(b), stride=(s,) * 3, padding=(p,) * 3, groups=groups)
        gx = orc.conv3d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, (s,) * 3, (p,) * 3, (1,) * 3, groups)
        gw = orc.conv3d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, (s,) * 3, (p,) * 3, (1,) * 3, groups)
    else:
        y = orc.conv2d(to_np(x), to_np(w), od, bias=to_np(b), stride=(s, s), padding=(p, p), groups=groups)
        gx = orc.conv2d_dgrad(to_np(dy), to_np(w), tuple(x.shape), od, (s, s), (p, p), (1, 1), groups)
        gw = orc.conv2d_wgrad(to_np(x), to_np(dy), tuple(w.shape), od, (s, s), (p, p), (1, 1), groups, acc64=True)
    return [decode(r, dtype) for r in (y, gx, gw)]


def _descs(gpu, x, w, b, dy, s, p, groups, exact=False, one_d=False):
    """Device tensors and one descriptor per mode over them: fwd writes y, dgrad dx, wgrad dw. one_d: the
    height-1 problem described with one spatial dimension ([N, C, W] tensors)."""
    if one_d:
        x, w, dy = x[:, :, 0], w[:, :, 0], dy[:, :, 0]
    xd, wd, bd, dyd = x.to(DEV), w.to(DEV), b.to(DEV), dy.to(DEV)
    y = torch.full(tuple(dy.shape), float("nan"), dtype=x.dtype, device=DEV)
    dx = torch.full(tuple(x.shape), float("nan"), dtype=x.dtype, device=DEV)
    dw = torch.full(tuple(w.shape), float("nan"), dtype=x.dtype, device=DEV)
    kw = dict(stride=s, padding=p, groups=groups, exact=exact)
    d_fwd = gpu.conv_problem(xd, wd, y, bias=bd, **kw)
    d_dgrad = gpu.conv_problem(dx, wd, dyd, **kw)
    d_wgrad = gpu.conv_problem(xd, dw, dyd, **kw)
    keep = (xd, wd, bd, dyd)
    return keep, [(gpu.TVK_CONV_FWD, d_fwd, y), (gpu.TVK_CONV_DGRAD, d_dgrad, dx), (gpu.TVK_CONV_WGRAD, d_wgrad, dw)]


def _every_candidate(gpu, x, w, b, s, p, groups, dtype, nd=2, seed=0, one_d=False):
    od_shape = (x.shape[0], w.shape[0]) + tuple((x.shape[2 + i] + 2 * p - w.shape[2 + i]) // s + 1 for i in range(nd))
    dy = torch.randn(od_shape, generator=gen(seed + 7)).to(dtype)
    refs = _refs(x, w, b, dy, s, p, groups, dtype, nd)
    keep, modes = _descs(gpu, x, w, b, dy, s, p, groups, one_d=one_d)
    seen = {}
    for (mode, d, out), ref in zip(modes, refs):
        names = gpu.conv_candidates(d, mode)
        assert set(names) <= FAMILIES and names[-1] == "conv_implicit_gemm", names
        seen[mode] = names
        for name in names:
            gpu.tune_reset()
            gpu.conv_choose(d, mode, name)
            out.fill_(float("nan"))
            print(f"{dtype} mode {mode}: {name}", flush=True)
            gpu.conv_run(d, mode)
            torch.cuda.synchronize()
            assert_close(decode(to_np(out.cpu()), dtype).reshape(ref.shape), ref, dtype, f"mode {mode}, {name}")
    del keep
    return seen


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layer", C4, ids=[c[0] for c in C4])
def test_every_candidate_of_the_c4_layers(gpu, fresh_table, dtype, layer):
    _, cin, cout, k, s, p, hw = layer
    x, w, b = _problem((8, cin, hw, hw), (cout, cin, k, k), dtype, seed=cin + k)
    seen = _every_candidate(gpu, x, w, b, s, p, 1, dtype)
    # the specialised families are the rule's first choice on these layers, with the implicit GEMM behind
    assert all(len(v) >= 2 for v in seen.values()), seen


@pytest.mark.parametrize("case", ["grouped", "one_d"])
def test_every_candidate_other_geometries(gpu, fresh_table, case):
    f16 = torch.float16
    if case == "grouped":
        x, w, b = _problem((4, 64, 16, 16), (64, 16, 3, 3), f16, seed=3, groups=4)
        _every_candidate(gpu, x, w, b, 1, 1, 4, f16)
    else:
        # one spatial dimension: the 2-D families on a height of 1, against the oracle's height-1 problem
        x, w, b = _problem((4, 64, 1, 96), (32, 64, 1, 5), f16, seed=5)
        seen = _every_candidate(gpu, x, w, b, 1, 0, 1, f16, one_d=True)
        assert all(v for v in seen.values())


def test_one_family_where_bits_are_fixed(gpu, fresh_table):
    # float32 and exact mode: the implicit GEMM only (sequential order); 3-D: the 3-D implicit GEMM only
    x, w, b = _problem((2, 64, 16, 16), (64, 64, 3, 3), torch.float32, seed=9)
    dy = torch.randn((2, 64, 16, 16), generator=gen(10))
    keep, modes = _descs(gpu, x, w, b, dy, 1, 1, 1)
    for mode, d, _ in modes:
        assert gpu.conv_candidates(d, mode) == ["conv_implicit_gemm"]
        with pytest.raises(gpu.TvkError):
            gpu.conv_choose(d, mode, "conv_halo")
    h = torch.float16
    keep2, modes2 = _descs(gpu, x.to(h), w.to(h), b.to(h), dy.to(h), 1, 1, 1, exact=True)
    for mode, d, _ in modes2:
        assert gpu.conv_candidates(d, mode) == ["conv_implicit_gemm"]
    x3, w3, b3 = _problem((2, 8, 6, 8, 8), (16, 8, 3, 3, 3), h, seed=11)
    dy3 = torch.randn((2, 16, 6, 8, 8), generator=gen(12)).to(h)
    keep3, modes3 = _descs(gpu, x3, w3, b3, dy3, 1, 1, 1)
    for mode, d, out in modes3:
        assert gpu.conv_candidates(d, mode) == ["conv_implicit_gemm"]
        gpu.conv_choose(d, mode, "conv_implicit_gemm")
        assert gpu.conv_tune(d, mode) == "conv_implicit_gemm"
    torch.cuda.synchronize()
    refs = _refs(x3, w3, b3, dy3, 1, 1, 1, h, nd=3)
    for (mode, d, out), ref in zip(modes3, refs):
        assert_close(decode(to_np(out.cpu()), h), ref, h, f"3-D mode {mode} through tvk_conv_tune")
    # a mode outside 0..2 and a name that is no family
    assert gpu.load().tvk_conv_choose(gpu.C.byref(modes3[0][1]), 3, b"conv_halo", 0) == gpu.TVK_ERR_INVALID
    with pytest.raises(gpu.TvkError):
        gpu.conv_choose(modes3[0][1], gpu.TVK_CONV_FWD, "no_such_kernel")


def test_tune_records_and_persists(gpu, fresh_table):
    h = torch.float16
    x, w, b = _problem((16, 64, 32, 32), (64, 64, 3, 3), h, seed=13)
    dy = torch.randn((16, 64, 32, 32), generator=gen(14)).to(h)
    refs = _refs(x[:4], w, b, dy[:4], 1, 1, 1, h)
    keep, modes = _descs(gpu, x, w, b, dy, 1, 1, 1)
    for mode, d, out in modes[:2]:      # forward and grad input (per-image results: a sample suffices)
        cands = gpu.conv_candidates(d, mode)
        first = gpu.conv_tune(d, mode)
        assert first in cands
        assert gpu.conv_tune(d, mode) == first      # recorded: no second timing, same family
        torch.cuda.synchronize()
        assert_close(decode(to_np(out[:4].cpu()), h), refs[mode], h, f"mode {mode} after tuning")
    path = fresh_table / next(p.name for p in fresh_table.iterdir())
    lines = [l.split() for l in path.read_text().splitlines()]
    assert sum(1 for l in lines if l[:2] == ["tvk1", "conv"]) == 2, lines
    # a fresh table reads the records back from the file
    gpu.tune_reset()
    for mode, d, _ in modes[:2]:
        rec = [l[3] for l in lines if l[:2] == ["tvk1", "conv"]]
        assert gpu.conv_tune(d, mode) in rec
