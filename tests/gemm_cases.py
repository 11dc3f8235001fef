"""Shared helpers of the GEMM parity tests: seeded host inputs, conversion of
torch tensors to the oracle's bit patterns, and the north_star tolerances.

Tolerances (stated once, used by every parity test):
  float32:            |got - ref| <= 1e-5 * (|ref| + 1)
  float16 / bfloat16: |got - ref| <= 5e-3 * (|ref| + 1)   (float32 accumulate)
where ref is the oracle's restatement of the reference SIMD tile
(oracle/gemm_oracle.c). The float32 path is additionally held to bit
equality with the oracle's fused-multiply-add form where that is claimed.
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


def max_violation(got: np.ndarray, ref: np.ndarray, dtype) -> float:
    """max over elements of |got-ref| / (tol*(|ref|+1)); <= 1 passes."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    both_nan = np.isnan(got) & np.isnan(ref)
    err = np.where(both_nan, 0.0, np.abs(got - ref))
    v = err / (TOL[dtype] * (np.abs(ref) + 1.0))
    v = np.where(np.isnan(v), np.inf, v)
    return float(v.max()) if v.size else 0.0


def assert_close(got: np.ndarray, ref: np.ndarray, dtype, what=""):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    v = max_violation(got, ref, dtype)
    assert v <= 1.0, f"{what}: max error is {v:.3f}x the {dtype} tolerance"
