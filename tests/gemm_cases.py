"""Shared helpers of the GEMM parity tests: seeded host inputs, conversion of
torch tensors to the oracle's bit patterns, and the north_star tolerances.

Tolerances (stated once, used by every parity test):
  float32:            |got - ref| <= 1e-5 * (|ref| + 1)
  float16 / bfloat16: |got - ref| <= 5e-3 * (|ref| + 1)   (float32 accumulate)
where ref is the oracle's restatement of the reference SIMD tile
(oracle/gemm_oracle.c). The float32 path and every dtype under TVK_GEMM_EXACT
are held to bit equality with the oracle's fused-multiply-add form.

bfloat16 on the fast MFMA path: one bfloat16 step is 2^-7 of the value at
the bottom of each binade, more than the 5e-3 bound, so a float32
accumulator that differs from the reference's in its last bits (a different
summation order) can round to the neighbouring bfloat16 and miss the bound
by construction. For that path an element passes if it is within the bound
OR within one bfloat16 spacing of ref; the fraction of elements that needed
the spacing is reported and capped (BF16_STEP_FRACTION).
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc

TOL = {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 5e-3}
ORC_DT = {torch.float32: orc.F32, torch.float16: orc.F16, torch.bfloat16: orc.BF16}


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, dtype, seed, std=1.0):
    return (torch.randn(shape, generator=gen(seed), dtype=torch.float32) * std).to(dtype)


def randint(shape, dtype, seed, lo=-4, hi=5):
    return torch.randint(lo, hi, shape, generator=gen(seed)).to(dtype)


def to_np(t: torch.Tensor) -> np.ndarray:
    """Host numpy view of a tensor with its strides kept; 16-bit types as uint16 bits."""
    t = t.detach().cpu() if t.device.type != "cpu" else t.detach()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def decode(x: np.ndarray, dtype) -> np.ndarray:
    return orc.to_f32(x, ORC_DT[dtype])


def oracle_mm(a, b, dtype, bias=None, alpha=1.0, beta=0.0, act=orc.ACT_NONE, fma=True) -> np.ndarray:
    """Oracle result (float32 values) of act(alpha*a@b + beta*bias) for host tensors."""
    bias_np = None if bias is None else np.ascontiguousarray(to_np(bias))
    out = orc.gemm(to_np(a), to_np(b), ORC_DT[dtype], bias=bias_np, alpha=alpha, beta=beta, act=act, fma=fma)
    return decode(out, dtype)


BF16_STEP_FRACTION = 0.01


def _bf16_spacing(ref: np.ndarray) -> np.ndarray:
    a = np.abs(ref.astype(np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, np.exp2(e - 7), 2.0 ** -133)


def max_violation(got: np.ndarray, ref: np.ndarray, dtype, bf16_step: bool = False) -> tuple[float, float]:
    """(max over elements of |got-ref| / allowed, fraction that needed the bf16 step); <= 1 passes."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    both_nan = np.isnan(got) & np.isnan(ref)
    err = np.where(both_nan, 0.0, np.abs(got - ref))
    bound = TOL[dtype] * (np.abs(ref) + 1.0)
    allowed = bound
    frac = 0.0
    if bf16_step and dtype == torch.bfloat16:
        allowed = np.maximum(bound, _bf16_spacing(ref) * (1 + 1e-9))
        frac = float((err > bound).mean()) if err.size else 0.0
    v = err / allowed
    v = np.where(np.isnan(v), np.inf, v)
    return (float(v.max()) if v.size else 0.0), frac


def assert_close(got: np.ndarray, ref: np.ndarray, dtype, what="", bf16_step: bool = True):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    v, frac = max_violation(got, ref, dtype, bf16_step)
    assert v <= 1.0, f"{what}: max error is {v:.3f}x the {dtype} tolerance"
    assert frac <= BF16_STEP_FRACTION, f"{what}: {frac:.4f} of the elements needed the one-bf16-step allowance"


def assert_bit_exact(got: np.ndarray, ref: np.ndarray, what=""):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    g = got.view(np.uint32)
    r = ref.view(np.uint32)
    bad = int((g != r).sum())
    assert bad == 0, f"{what}: {bad} of {g.size} elements differ from the oracle's bits"
