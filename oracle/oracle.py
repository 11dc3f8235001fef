"""Python driver of the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker: the product path never calls it.

Arrays are numpy arrays; float16 and bfloat16 operands travel as their raw
16-bit patterns (dtype uint16) together with a dtype code, so the oracle sees
exactly the bits the device sees. See gemm_oracle.c for the reference lines
each function restates.
"""
from __future__ import annotations

import concurrent.futures as cf
import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "build" / "liboracle.so"

F32, F16, BF16, F64, I64, I32, I16, I8, U8, BOOL, F8E4M3FN, F8E5M2 = range(12)
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2

_lib = None
_P64 = C.POINTER(C.c_int64)


def build() -> Path:
    """Compiles the oracle with its Makefile (gcc), output under oracle/build/."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = C.CDLL(str(LIB))
        lib.oracle_f32_to_f16.argtypes = [C.c_float]
        lib.oracle_f32_to_f16.restype = C.c_uint16
        lib.oracle_f16_to_f32.argtypes = [C.c_uint16]
        lib.oracle_f16_to_f32.restype = C.c_float
        lib.oracle_f32_to_bf16.argtypes = [C.c_float]
        lib.oracle_f32_to_bf16.restype = C.c_uint16
        lib.oracle_bf16_to_f32.argtypes = [C.c_uint16]
        lib.oracle_bf16_to_f32.restype = C.c_float
        lib.oracle_gelu.argtypes = [C.c_float]
        lib.oracle_gelu.restype = C.c_float
        lib.oracle_gemm_rows.argtypes = [
            C.c_int, C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
            C.c_void_p, _P64, C.c_void_p, _P64, C.c_void_p, _P64, C.c_void_p, _P64,
            C.c_double, C.c_double, C.POINTER(C.c_float),
        ]
        lib.oracle_gemm_rows.restype = C.c_int
        lib.oracle_gemm_wide_rows.argtypes = [
            C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
            C.c_void_p, C.POINTER(C.c_int64), C.c_void_p, C.POINTER(C.c_int64), C.c_void_p, C.POINTER(C.c_int64),
            C.c_void_p, C.POINTER(C.c_int64), C.c_double, C.c_double]
        lib.oracle_gemm_wide_rows.restype = C.c_int
        lib.oracle_cast.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int64]
        lib.oracle_cast.restype = C.c_int
        lib.oracle_f64_to_f16.argtypes = [C.c_double]
        lib.oracle_f64_to_f16.restype = C.c_uint16
        _lib = lib
    return _lib


# ---------------------------------------------------------------------------
# element conversions (vectorised through the C functions)
# ---------------------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    f = np.vectorize(load().oracle_f32_to_f16, otypes=[np.uint16])
    return f(np.asarray(x, dtype=np.float32))


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    f = np.vectorize(load().oracle_f16_to_f32, otypes=[np.float32])
    return f(np.asarray(h, dtype=np.uint16))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    f = np.vectorize(load().oracle_f32_to_bf16, otypes=[np.uint16])
    return f(np.asarray(x, dtype=np.float32))


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f32(bits_or_f32: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F32:
        return np.asarray(bits_or_f32, dtype=np.float32)
    if dtype == F16:
        return np.asarray(bits_or_f32, dtype=np.uint16).view(np.float16).astype(np.float32)
    return bf16_bits_to_f32(bits_or_f32)


# ---------------------------------------------------------------------------
# element conversion of tvk_copy (copy_oracle.c)
# ---------------------------------------------------------------------------

# numpy storage of each code; float16/bfloat16 travel as raw uint16 patterns
STORAGE = {F32: np.float32, F16: np.uint16, BF16: np.uint16, F64: np.float64, I64: np.int64, I32: np.int32,
           I16: np.int16, I8: np.int8, U8: np.uint8, BOOL: np.uint8, F8E4M3FN: np.uint8, F8E5M2: np.uint8}


def cast(src: np.ndarray, sdt: int, ddt: int) -> np.ndarray:
    """castValue<sdt, ddt> of every element (the reference's cast rules); any shape, returns a dense array."""
    s = np.ascontiguousarray(src, dtype=STORAGE[sdt])
    d = np.zeros(s.shape, dtype=STORAGE[ddt])
    if s.size and load().oracle_cast(sdt, s.ctypes.data, ddt, d.ctypes.data, s.size) != 0:
        raise ValueError("oracle_cast rejected its dtypes")
    return d


# ---------------------------------------------------------------------------
# element-wise add / sub / mul of tvk_binary
# ---------------------------------------------------------------------------

BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV = 0, 1, 2, 3
_NP_INT = {I64: np.int64, I32: np.int32, I16: np.int16, I8: np.int8, U8: np.uint8}


def _round_to(x32: np.ndarray, dt: int) -> np.ndarray:
    """float32 values rounded to dt, returned as float32 values."""
    if dt == F32:
        return x32.astype(np.float32)
    if dt == F16:
        return x32.astype(np.float32).astype(np.float16).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(x32))


def binary(a: np.ndarray, b: np.ndarray, dt: int, op: int, alpha: float = 1.0) -> np.ndarray:
    """AddOp / SubOp / MulOp / DivOp of the reference's binary shader in dtype dt
    (src/shaders/ops/binary.slang:39-60): alpha converted to dt; with
    alpha != 1, T(a op T(alpha*b)); float16/bfloat16 compute each operation
    in float32 and round back (src/shaders/core/dtype.slang:911-913); float32
    and float64 round every operation (no fused multiply-add); integers wrap.
    a, b: storage arrays (uint16 patterns for float16/bfloat16), broadcast."""
    a, b = np.broadcast_arrays(np.asarray(a, dtype=STORAGE[dt]), np.asarray(b, dtype=STORAGE[dt]))
    has_alpha = op in (BIN_ADD, BIN_SUB) and alpha != 1.0
    if op == BIN_DIV and dt in _NP_INT:
        raise ValueError("division is defined for the float dtypes only")
    if dt in _NP_INT:
        t = _NP_INT[dt]
        with np.errstate(over="ignore"):
            a64, b64 = a.astype(np.int64).astype(np.uint64), b.astype(np.int64).astype(np.uint64)
            al = np.uint64(np.int64(int(alpha)).astype(np.uint64))
            if op == BIN_MUL:
                r = a64 * b64
            else:
                tb = al * b64 if has_alpha else b64
                r = a64 + tb if op == BIN_ADD else a64 - tb
        return r.astype(np.int64).astype(t)
    if dt == F64:
        a64, b64, al = a.astype(np.float64), b.astype(np.float64), np.float64(alpha)
        if op == BIN_MUL:
            return a64 * b64
        if op == BIN_DIV:
            with np.errstate(divide="ignore", invalid="ignore"):
                return a64 / b64
        t = al * b64 if has_alpha else b64
        return a64 + t if op == BIN_ADD else a64 - t
    fa, fb = to_f32(a, dt), to_f32(b, dt)
    al = _round_to(np.array([alpha], dtype=np.float32), dt)[0]
    if op == BIN_MUL:
        r = _round_to(fa * fb, dt)
    elif op == BIN_DIV:
        with np.errstate(divide="ignore", invalid="ignore"):
            r = _round_to(fa / fb, dt)
    else:
        t = _round_to(al * fb, dt) if has_alpha else fb
        r = _round_to(fa + t if op == BIN_ADD else fa - t, dt)
    if dt == F32:
        return r
    if dt == F16:
        return r.astype(np.float16).view(np.uint16)
    return f32_to_bf16_bits(r)


# ---------------------------------------------------------------------------
# scaled dot-product attention (float64 restatement)
# ---------------------------------------------------------------------------

def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, bias: np.ndarray | None = None, causal: bool = False,
              scale: float | None = None) -> tuple[np.ndarray, np.ndarray]:
    """(out, lse) of the reference's attention rows in float64
    (chunked_forward, src/api/ops/attention.cpp:115-139; scores per
    chunk_scores, :101-113): s = scale*q.k (+ bias), -inf where causal and
    key j > query i; a row with every key masked gives out 0 and lse +inf.
    q [B,Hq,L,D], k [B,Hk,S,D], v [B,Hk,S,Dv] as float64 values; query head
    h reads key/value head h // (Hq/Hk)."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    B, Hq, L, D = q.shape
    Hk, S = k.shape[1], k.shape[2]
    g = Hq // Hk
    scale = D ** -0.5 if scale is None else scale
    kk = np.repeat(k, g, axis=1)
    vv = np.repeat(v, g, axis=1)
    s = np.einsum("bhld,bhsd->bhls", q, kk) * scale
    if bias is not None:
        s = s + np.broadcast_to(np.asarray(bias, dtype=np.float64), s.shape)
    if causal:
        s = np.where(np.arange(S)[None, :] > np.arange(L)[:, None], -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    safe = np.where(np.isneginf(mx), 0.0, mx)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - safe)
    tot = p.sum(axis=-1, keepdims=True)
    empty = tot == 0.0
    out = np.einsum("bhls,bhsd->bhld", p, vv) / np.where(empty, 1.0, tot)
    with np.errstate(divide="ignore"):
        lse = np.where(empty, np.inf, safe + np.log(np.where(empty, 1.0, tot)))[..., 0]
    return out, lse


def attention_bwd(q, k, v, dout, bias=None, causal=False, scale=None, out=None, round_to=None, return_ds=False):
    """(dq, dk, dv) of attention() in float64, as the reference's
    chunked_backward (src/api/ops/attention.cpp:141-199): P = exp(s - lse),
    delta = rowsum(dout*out), dS = P*(dout.v^T - delta), dq = scale*dS.k,
    dk = scale*dS^T.q and dv = P^T.dout summed over each kv head's query
    heads. `out` is the forward output as stored (rounded to its dtype); the
    reference forms delta from that tensor (:156). Without it, the exact
    float64 output is used. round_to (F16/BF16): P and dS are formed in
    float32 and rounded to that dtype before their products, as the
    reference's cooperative-matrix backward stages them
    (src/shaders/ops/attention_coop.slang:283-305). return_ds: also the
    score gradient dS [B,Hq,L,S] before any rounding, the gradient of an
    additive bias before its broadcast dimensions are summed (the
    reference's grad_bias is sum_to(ds, bias shape), :187-196)."""
    q, k, v, dout = (np.asarray(t, dtype=np.float64) for t in (q, k, v, dout))
    B, Hq, L, D = q.shape
    Hk, S = k.shape[1], k.shape[2]
    g = Hq // Hk
    scale = D ** -0.5 if scale is None else scale
    exact_out, lse = attention(q, k, v, bias, causal, scale)
    out = exact_out if out is None else np.asarray(out, dtype=np.float64)
    kk, vv = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    s = np.einsum("bhld,bhsd->bhls", q, kk) * scale
    if bias is not None:
        s = s + np.broadcast_to(np.asarray(bias, dtype=np.float64), s.shape)
    if causal:
        s = np.where(np.arange(S)[None, :] > np.arange(L)[:, None], -np.inf, s)
    with np.errstate(invalid="ignore"):
        p = np.where(np.isinf(lse)[..., None], 0.0, np.exp(s - lse[..., None]))
    delta = (dout * out).sum(-1, keepdims=True)
    dp = np.einsum("bhld,bhsd->bhls", dout, vv)
    ds = p * (dp - delta)
    ds_exact = ds
    if round_to is not None:
        rt = lambda x: to_f32(cast(x.astype(np.float32), F32, round_to), round_to).astype(np.float64)
        p, ds = rt(p), rt(ds)
    dq = np.einsum("bhls,bhsd->bhld", ds, kk) * scale
    dk = np.einsum("bhls,bhld->bhsd", ds, q).reshape(B, Hk, g, S, D).sum(2) * scale
    dv = np.einsum("bhls,bhld->bhsd", p, dout).reshape(B, Hk, g, S, v.shape[3]).sum(2)
    if return_ds:
        return dq, dk, dv, ds_exact
    return dq, dk, dv


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

def _estrides3(x: np.ndarray) -> tuple[int, int, int]:
    es = x.itemsize
    st = [s // es for s in x.strides]
    if x.ndim == 2:
        return (0, st[0], st[1])
    if x.ndim == 3:
        return (st[0], st[1], st[2])
    raise ValueError("expected 2-D or 3-D")


# element storage of the float64 and integer products (oracle_gemm_wide_rows)
WIDE_STORE = {F64: np.float64, I64: np.int64, I32: np.int32, I16: np.int16, I8: np.int8, U8: np.uint8}


def gemm(a: np.ndarray, b: np.ndarray, dtype: int, bias: np.ndarray | None = None, alpha: float = 1.0,
         beta: float = 0.0, act: int = ACT_NONE, fma: bool = True, threads: int | None = None) -> np.ndarray:
    """C = act(alpha*A@B + beta*bias) in the reference SIMD tile's order.

    a: [M,K] or [B,M,K]; b: [K,N] or [B,K,N] (any strides, including
    broadcast); bias broadcasts to C. Returns a contiguous array of the same
    element storage (float32, uint16 bit patterns for float16/bfloat16, the
    numpy type itself for float64 and the integer types).
    """
    lib = load()
    batched = a.ndim == 3 or b.ndim == 3
    if batched:
        nb = max(a.shape[0] if a.ndim == 3 else 1, b.shape[0] if b.ndim == 3 else 1)
        if a.ndim == 2:
            a = np.broadcast_to(a, (nb,) + a.shape)
        if b.ndim == 2:
            b = np.broadcast_to(b, (nb,) + b.shape)
    else:
        nb = 1
    M, K = a.shape[-2], a.shape[-1]
    K2, N = b.shape[-2], b.shape[-1]
    if K != K2:
        raise ValueError(f"shapes cannot be multiplied ({M}x{K} and {K2}x{N})")
    store = WIDE_STORE.get(dtype, np.float32 if dtype == F32 else np.uint16)
    out_shape = (nb, M, N) if batched else (M, N)
    c = np.zeros(out_shape, dtype=store)
    if c.size == 0:
        return c
    sa = (C.c_int64 * 3)(*_estrides3(a))
    sb = (C.c_int64 * 3)(*_estrides3(b))
    sc = (C.c_int64 * 3)(*_estrides3(c))
    bias_e = None
    sbias = (C.c_int64 * 3)(0, 0, 0)
    if bias is not None:
        bias_e = np.broadcast_to(np.asarray(bias, dtype=store), out_shape)
        sbias = (C.c_int64 * 3)(*_estrides3(bias_e))
    a_p = a.ctypes.data if a.size else None
    b_p = b.ctypes.data if b.size else None
    bias_p = bias_e.ctypes.data if bias_e is not None else None

    threads = threads or max(1, min(16, os.cpu_count() or 1))
    jobs = []
    rows_per = max(1, -(-M // max(1, threads)))
    for bi in range(nb):
        for m0 in range(0, M, rows_per):
            jobs.append((bi, m0, min(M, m0 + rows_per)))

    def run(job):
        bi, m0, m1 = job
        if dtype in WIDE_STORE:
            rc = lib.oracle_gemm_wide_rows(dtype, act, bi, m0, m1, N, K, a_p, sa, b_p, sb, bias_p, sbias, c.ctypes.data,
                                           sc, float(alpha), float(beta))
            if rc != 0:
                raise ValueError("oracle_gemm_wide_rows rejected its arguments")
            return
        scratch = (C.c_float * max(1, N))()
        rc = lib.oracle_gemm_rows(dtype, act, 1 if fma else 0, bi, m0, m1, N, K, a_p, sa, b_p, sb, bias_p, sbias,
                                  c.ctypes.data, sc, float(alpha), float(beta), scratch)
        if rc != 0:
            raise ValueError("oracle_gemm_rows rejected its arguments")

    if len(jobs) == 1:
        run(jobs[0])
    else:
        with cf.ThreadPoolExecutor(max_workers=threads) as ex:
            list(ex.map(run, jobs))
    return c


def complex_gemm(a: np.ndarray, b: np.ndarray, bias: np.ndarray | None = None, alpha: complex = 1.0,
                 beta: complex = 0.0) -> np.ndarray:
    """complex_matmul (src/api/ops/matmul.cpp:355-371) of complex64 or
    complex128 operands ([M,K]/[B,M,K] and [K,N]/[B,K,N], bias broadcasting
    to the result): the real and imaginary parts multiplied by the real
    product (gemm above, in the real type), re = T(re.re) - T(im.im) and
    im = T(re.im) + T(im.re) each rounded in the real type; then, when
    alpha != 1, r = r * alpha and, when a bias is given with beta != 0,
    r = r + bias * beta, as complex_mul (src/api/ops/complex.cpp:43-46):
    (x.re*s.re - x.im*s.im, x.re*s.im + x.im*s.re), every operation rounded
    in the real type. complex32 operands compute as complex64 (the caller
    widens them and rounds the result)."""
    real = np.float64 if a.dtype == np.complex128 else np.float32
    dt = F64 if real == np.float64 else F32

    def parts(z):
        z = np.asarray(z)
        return np.ascontiguousarray(z.real, dtype=real), np.ascontiguousarray(z.imag, dtype=real)

    def cmul(xr, xi, s):
        sr, si = real(complex(s).real), real(complex(s).imag)
        return (xr * sr - xi * si).astype(real), (xr * si + xi * sr).astype(real)

    ar, ai = parts(a)
    br, bi = parts(b)
    re = (gemm(ar, br, dt) - gemm(ai, bi, dt)).astype(real)
    im = (gemm(ar, bi, dt) + gemm(ai, br, dt)).astype(real)
    if complex(alpha) != 1:
        re, im = cmul(re, im, alpha)
    if bias is not None and complex(beta) != 0:
        cr, ci = parts(np.broadcast_to(bias, re.shape))
        cr, ci = cmul(cr, ci, beta)
        re, im = (re + cr).astype(real), (im + ci).astype(real)
    out = np.empty(re.shape, dtype=np.complex128 if real == np.float64 else np.complex64)
    out.real, out.imag = re, im
    return out


def scaled_mm(a_codes: np.ndarray, a_dt: int, b_codes: np.ndarray, b_dt: int, scale_a, scale_b, out_dt: int,
              bias: np.ndarray | None = None, bias_dt: int = F32, scale_result: float | None = None) -> np.ndarray:
    """torch's emulated _scaled_mm as the reference computes it
    (scaled_mm_out_vulkan, src/api/ops/matmul.cpp:706-747): float8 codes
    decoded to float32 and multiplied by their scale (one each, or a [M,1]
    column for A and a [1,N] row for B) in float32; the float32 product
    (gemm above); the bias (storage of bias_dt, [N]) added in float32; times
    the float32 1 / scale_result when out_dt is a float8 type; rounded to
    out_dt (cast above). Returns out_dt storage."""
    fa = cast(a_codes, a_dt, F32) * np.asarray(scale_a, dtype=np.float32)
    fb = cast(b_codes, b_dt, F32) * np.asarray(scale_b, dtype=np.float32)
    p = gemm(fa.astype(np.float32), fb.astype(np.float32), F32)
    if bias is not None:
        p = (p + cast(np.asarray(bias), bias_dt, F32)).astype(np.float32)
    if scale_result is not None and out_dt in (F8E4M3FN, F8E5M2):
        p = (p * (np.float32(1.0) / np.float32(scale_result))).astype(np.float32)
    return cast(p, F32, out_dt)


# ---------------------------------------------------------------------------
# 2-D convolution (conv_oracle.c)
# ---------------------------------------------------------------------------

class ConvGeom(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "n", "cin", "h", "w", "cout", "kh", "kw", "sh", "sw", "ph", "pw", "dh", "dw", "groups", "ho", "wo")]


def conv_out_size(size: int, k: int, s: int, p: int, d: int) -> int:
    return (size + 2 * p - d * (k - 1) - 1) // s + 1


def make_geom(x_shape, w_shape, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1, out_hw=None) -> ConvGeom:
    n, cin, h, w = x_shape
    cout, _, kh, kw = w_shape
    if out_hw is None:
        out_hw = (conv_out_size(h, kh, stride[0], padding[0], dilation[0]),
                  conv_out_size(w, kw, stride[1], padding[1], dilation[1]))
    return ConvGeom(n, cin, h, w, cout, kh, kw, stride[0], stride[1], padding[0], padding[1],
                    dilation[0], dilation[1], groups, out_hw[0], out_hw[1])


def _conv_lib():
    lib = load()
    if not getattr(lib, "_conv_ready", False):
        P = C.POINTER(ConvGeom)
        lib.oracle_conv_fwd.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.oracle_conv_dgrad.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.oracle_conv_wgrad.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        lib.oracle_winograd_fwd.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        for f in ("oracle_conv_fwd", "oracle_conv_dgrad", "oracle_conv_wgrad", "oracle_winograd_fwd"):
            getattr(lib, f).restype = C.c_int
        lib._conv_ready = True
    return lib


def _parallel(total: int, fn, threads: int | None):
    threads = threads or max(1, min(16, os.cpu_count() or 1))
    per = max(1, -(-total // threads))
    ranges = [(b, min(total, b + per)) for b in range(0, total, per)]

    def run(r):
        if fn(*r) != 0:
            raise ValueError("conv oracle rejected its arguments")

    if len(ranges) <= 1:
        for r in ranges:
            run(r)
    else:
        with cf.ThreadPoolExecutor(max_workers=threads) as ex:
            list(ex.map(run, ranges))


def _c(x):
    return np.ascontiguousarray(x)


def conv2d(x, w, dtype: int, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
           threads=None) -> np.ndarray:
    """Forward implicit-GEMM convolution in the reference's k order (c, kh, kw)."""
    lib = _conv_lib()
    x, w = _c(x), _c(w)
    g = make_geom(x.shape, w.shape, stride, padding, dilation, groups)
    y = np.zeros((g.n, g.cout, g.ho, g.wo), dtype=x.dtype)
    b = None if bias is None else _c(bias)
    _parallel(g.n, lambda s, e: lib.oracle_conv_fwd(dtype, C.byref(g), s, e, x.ctypes.data, w.ctypes.data,
                                                    None if b is None else b.ctypes.data, y.ctypes.data), threads)
    return y


def conv2d_dgrad(dy, w, x_shape, dtype: int, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
                 threads=None) -> np.ndarray:
    lib = _conv_lib()
    dy, w = _c(dy), _c(w)
    g = make_geom(x_shape, w.shape, stride, padding, dilation, groups, out_hw=dy.shape[2:])
    dx = np.zeros(tuple(x_shape), dtype=dy.dtype)
    _parallel(g.n, lambda s, e: lib.oracle_conv_dgrad(dtype, C.byref(g), s, e, dy.ctypes.data, w.ctypes.data,
                                                      dx.ctypes.data), threads)
    return dx


def conv2d_wgrad(x, dy, w_shape, dtype: int, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1,
                 acc64=True, threads=None) -> np.ndarray:
    lib = _conv_lib()
    x, dy = _c(x), _c(dy)
    g = make_geom(x.shape, w_shape, stride, padding, dilation, groups, out_hw=dy.shape[2:])
    dw = np.zeros(tuple(w_shape), dtype=x.dtype)
    _parallel(g.cout, lambda s, e: lib.oracle_conv_wgrad(dtype, C.byref(g), s, e, x.ctypes.data, dy.ctypes.data,
                                                         dw.ctypes.data, 1 if acc64 else 0), threads)
    return dw


def winograd_conv2d(x, w, dtype: int, bias=None, padding=(1, 1), threads=None) -> np.ndarray:
    """The reference's Winograd F(2x2,3x3) forward, intermediates rounded to dtype."""
    lib = _conv_lib()
    x, w = _c(x), _c(w)
    g = make_geom(x.shape, w.shape, (1, 1), padding, (1, 1), 1)
    y = np.zeros((g.n, g.cout, g.ho, g.wo), dtype=x.dtype)
    b = None if bias is None else _c(bias)
    _parallel(g.n, lambda s, e: lib.oracle_winograd_fwd(dtype, C.byref(g), s, e, x.ctypes.data, w.ctypes.data,
                                                        None if b is None else b.ctypes.data, y.ctypes.data), threads)
    return y


# ---------------------------------------------------------------------------
# 3-D convolution (conv_oracle.c, oracle_conv3d_*)
# ---------------------------------------------------------------------------

class Conv3Geom(C.Structure):
    _fields_ = [("n", C.c_int64), ("cin", C.c_int64), ("cout", C.c_int64), ("groups", C.c_int64)] + \
               [(f, C.c_int64 * 3) for f in ("inn", "k", "s", "p", "d", "out")]


def _triple(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v, v)


def make_geom3(x_shape, w_shape, stride=1, padding=0, dilation=1, groups=1, out=None) -> Conv3Geom:
    n, cin = x_shape[:2]
    cout = w_shape[0]
    s, p, d = _triple(stride), _triple(padding), _triple(dilation)
    k = tuple(w_shape[2:])
    if out is None:
        out = tuple(conv_out_size(x_shape[2 + i], k[i], s[i], p[i], d[i]) for i in range(3))
    A = C.c_int64 * 3
    return Conv3Geom(n, cin, cout, groups, A(*x_shape[2:]), A(*k), A(*s), A(*p), A(*d), A(*out))


def _conv3_lib():
    lib = load()
    if not getattr(lib, "_conv3_ready", False):
        P = C.POINTER(Conv3Geom)
        lib.oracle_conv3d_fwd.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.oracle_conv3d_dgrad.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.oracle_conv3d_wgrad.argtypes = [C.c_int, P, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        for f in ("oracle_conv3d_fwd", "oracle_conv3d_dgrad", "oracle_conv3d_wgrad"):
            getattr(lib, f).restype = C.c_int
        lib._conv3_ready = True
    return lib


def conv3d(x, w, dtype: int, bias=None, stride=1, padding=0, dilation=1, groups=1, threads=None) -> np.ndarray:
    """Forward 3-D implicit-GEMM convolution in the reference's k order (c, kd, kh, kw)."""
    lib = _conv3_lib()
    x, w = _c(x), _c(w)
    g = make_geom3(x.shape, w.shape, stride, padding, dilation, groups)
    y = np.zeros((g.n, g.cout) + tuple(g.out), dtype=x.dtype)
    b = None if bias is None else _c(bias)
    _parallel(g.n, lambda s, e: lib.oracle_conv3d_fwd(dtype, C.byref(g), s, e, x.ctypes.data, w.ctypes.data,
                                                      None if b is None else b.ctypes.data, y.ctypes.data), threads)
    return y


def conv3d_dgrad(dy, w, x_shape, dtype: int, stride=1, padding=0, dilation=1, groups=1, threads=None) -> np.ndarray:
    lib = _conv3_lib()
    dy, w = _c(dy), _c(w)
    g = make_geom3(x_shape, w.shape, stride, padding, dilation, groups, out=dy.shape[2:])
    dx = np.zeros(tuple(x_shape), dtype=dy.dtype)
    _parallel(g.n, lambda s, e: lib.oracle_conv3d_dgrad(dtype, C.byref(g), s, e, dy.ctypes.data, w.ctypes.data,
                                                        dx.ctypes.data), threads)
    return dx


def conv3d_wgrad(x, dy, w_shape, dtype: int, stride=1, padding=0, dilation=1, groups=1, acc64=True,
                 threads=None) -> np.ndarray:
    lib = _conv3_lib()
    x, dy = _c(x), _c(dy)
    g = make_geom3(x.shape, w_shape, stride, padding, dilation, groups, out=dy.shape[2:])
    dw = np.zeros(tuple(w_shape), dtype=x.dtype)
    _parallel(g.cout, lambda s, e: lib.oracle_conv3d_wgrad(dtype, C.byref(g), s, e, x.ctypes.data, dy.ctypes.data,
                                                           dw.ctypes.data, 1 if acc64 else 0), threads)
    return dw
