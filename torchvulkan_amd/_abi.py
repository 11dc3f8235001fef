"""ctypes binding of the C ABI declared in include/tvk_hip.h.

This is the binding a Python caller of the boundary uses (tests, the
benchmark and the smoke check call the library through it). It never falls
back to anything: if ``libtvk_hip.so`` is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "libtvk_hip.so"

TVK_OK, TVK_ERR_UNSUPPORTED, TVK_ERR_OOM, TVK_ERR_INVALID, TVK_ERR_DEVICE = range(5)
(TVK_F32, TVK_F16, TVK_BF16, TVK_F64, TVK_I64, TVK_I32, TVK_I16, TVK_I8, TVK_U8,
 TVK_BOOL, TVK_F8E4M3FN, TVK_F8E5M2) = range(12)
TVK_COPY_MAX_DIMS = 16
TVK_ACT_NONE, TVK_ACT_RELU, TVK_ACT_GELU = range(3)
TVK_GEMM_EXACT = 1

STATUS_NAMES = {0: "OK", 1: "UNSUPPORTED", 2: "OOM", 3: "INVALID", 4: "DEVICE"}


class TvkError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"tvk status {STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class TvkUnsupported(TvkError):
    """The call cannot run on the device (the caller takes its CPU fallback)."""


class TvkOutOfMemory(TvkError):
    pass


I64x3 = C.c_int64 * 3


class GemmDesc(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("activation", C.c_int32),
        ("flags", C.c_uint32),
        ("reserved", C.c_int32),
        ("batch", C.c_int64),
        ("M", C.c_int64),
        ("N", C.c_int64),
        ("K", C.c_int64),
        ("a", C.c_void_p), ("a_stride", I64x3),
        ("b", C.c_void_p), ("b_stride", I64x3),
        ("bias", C.c_void_p), ("bias_stride", I64x3),
        ("c", C.c_void_p), ("c_stride", I64x3),
        ("alpha", C.c_double),
        ("beta", C.c_double),
        ("stream", C.c_void_p),
        ("batch_inner", C.c_int64),
        ("a_stride_inner", C.c_int64), ("b_stride_inner", C.c_int64),
        ("bias_stride_inner", C.c_int64), ("c_stride_inner", C.c_int64),
    ]


class ConvDesc(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("flags", C.c_uint32),
        ("n", C.c_int64), ("c_in", C.c_int64), ("h", C.c_int64), ("w", C.c_int64),
        ("c_out", C.c_int64), ("kh", C.c_int64), ("kw", C.c_int64),
        ("stride", C.c_int64 * 2), ("padding", C.c_int64 * 2), ("dilation", C.c_int64 * 2),
        ("groups", C.c_int64),
        ("h_out", C.c_int64), ("w_out", C.c_int64),
        ("x", C.c_void_p),
        ("weight", C.c_void_p),
        ("bias", C.c_void_p),
        ("y", C.c_void_p),
        ("stream", C.c_void_p),
    ]


I64x3s = C.c_int64 * 3


class ConvNdDesc(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("flags", C.c_uint32),
        ("spatial_dims", C.c_int32),
        ("reserved", C.c_int32),
        ("n", C.c_int64), ("c_in", C.c_int64), ("c_out", C.c_int64), ("groups", C.c_int64),
        ("in_size", I64x3s), ("kernel", I64x3s), ("stride", I64x3s), ("padding", I64x3s), ("dilation", I64x3s),
        ("out_size", I64x3s),
        ("x", C.c_void_p),
        ("weight", C.c_void_p),
        ("bias", C.c_void_p),
        ("y", C.c_void_p),
        ("stream", C.c_void_p),
    ]


I64xD = C.c_int64 * TVK_COPY_MAX_DIMS


class CopyDesc(C.Structure):
    _fields_ = [
        ("src_dtype", C.c_int32),
        ("dst_dtype", C.c_int32),
        ("ndim", C.c_int32),
        ("reserved", C.c_int32),
        ("sizes", I64xD),
        ("src", C.c_void_p), ("src_strides", I64xD),
        ("dst", C.c_void_p), ("dst_strides", I64xD),
        ("stream", C.c_void_p),
    ]


class FillDesc(C.Structure):
    _fields_ = [
        ("elem_size", C.c_int32),
        ("ndim", C.c_int32),
        ("sizes", I64xD),
        ("dst", C.c_void_p), ("dst_strides", I64xD),
        ("pattern", C.c_uint64),
        ("stream", C.c_void_p),
    ]


class ReduceDesc(C.Structure):
    _fields_ = [
        ("src_dtype", C.c_int32),
        ("dst_dtype", C.c_int32),
        ("ndim", C.c_int32),
        ("reduce_mask", C.c_uint32),
        ("sizes", I64xD),
        ("src", C.c_void_p), ("src_strides", I64xD),
        ("dst", C.c_void_p), ("dst_strides", I64xD),
        ("stream", C.c_void_p),
    ]


TVK_BIN_ADD, TVK_BIN_SUB, TVK_BIN_MUL, TVK_BIN_DIV = range(4)


class BinaryDesc(C.Structure):
    _fields_ = [
        ("op", C.c_int32),
        ("dtype", C.c_int32),
        ("ndim", C.c_int32),
        ("reserved", C.c_int32),
        ("sizes", I64xD),
        ("a", C.c_void_p), ("a_strides", I64xD),
        ("b", C.c_void_p), ("b_strides", I64xD),
        ("out", C.c_void_p), ("out_strides", I64xD),
        ("alpha", C.c_double),
        ("stream", C.c_void_p),
    ]


I64x4 = C.c_int64 * 4


class AttentionDesc(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("causal", C.c_int32),
        ("batch", C.c_int64), ("heads_q", C.c_int64), ("heads_kv", C.c_int64), ("len_q", C.c_int64),
        ("len_kv", C.c_int64), ("head_dim", C.c_int64), ("head_dim_v", C.c_int64),
        ("q", C.c_void_p), ("q_stride", I64x4),
        ("k", C.c_void_p), ("k_stride", I64x4),
        ("v", C.c_void_p), ("v_stride", I64x4),
        ("bias", C.c_void_p), ("bias_stride", I64x4),
        ("out", C.c_void_p), ("out_stride", I64x4),
        ("lse", C.c_void_p), ("lse_stride", I64x3),
        ("scale", C.c_double),
        ("stream", C.c_void_p),
    ]


class AttentionBwdDesc(C.Structure):
    _fields_ = [
        ("fwd", AttentionDesc),
        ("dout", C.c_void_p), ("dout_stride", I64x4),
        ("dq", C.c_void_p), ("dq_stride", I64x4),
        ("dk", C.c_void_p), ("dk_stride", I64x4),
        ("dv", C.c_void_p), ("dv_stride", I64x4),
        ("dscores", C.c_void_p), ("dscores_stride", I64x4),
    ]


class DeviceProps(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("arch", C.c_char * 64),
        ("total_memory", C.c_size_t),
        ("compute_units", C.c_int),
        ("clock_khz", C.c_int),
        ("wavefront_size", C.c_int),
        ("lds_per_block", C.c_size_t),
        ("pci_bus_id", C.c_int),
        ("has_fp64", C.c_int),
        ("has_fp16", C.c_int),
        ("has_bf16", C.c_int),
    ]


_lib = None


def lib_path() -> Path:
    return _LIB_PATH


def load() -> C.CDLL:
    """Loads libtvk_hip.so (raises OSError when it has not been built)."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise OSError(f"{_LIB_PATH} is not built; run python torchvulkan_amd/build.py")
        lib = C.CDLL(str(_LIB_PATH))
        lib.tvk_last_error.restype = C.c_char_p
        lib.tvk_gemm.argtypes = [C.POINTER(GemmDesc)]
        lib.tvk_gemm_plan.argtypes = [C.POINTER(GemmDesc), C.c_char_p, C.c_size_t]
        lib.tvk_gemm_candidates.argtypes = [C.POINTER(GemmDesc), C.c_char_p, C.c_size_t]
        lib.tvk_gemm_choose.argtypes = [C.POINTER(GemmDesc), C.c_char_p, C.c_int]
        lib.tvk_gemm_tune.argtypes = [C.POINTER(GemmDesc), C.c_char_p, C.c_size_t]
        lib.tvk_tune_reset.argtypes = []
        lib.tvk_tune_path.argtypes = [C.c_char_p, C.c_size_t]
        lib.tvk_malloc.argtypes = [C.c_int, C.c_size_t, C.POINTER(C.c_void_p)]
        lib.tvk_free.argtypes = [C.c_void_p]
        lib.tvk_pointer_device.argtypes = [C.c_void_p, C.POINTER(C.c_int)]
        lib.tvk_memcpy_h2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_int]
        lib.tvk_memcpy_d2h.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_int]
        lib.tvk_memcpy_d2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        lib.tvk_get_stream.argtypes = [C.c_int, C.POINTER(C.c_void_p)]
        for fn in ("tvk_memory_allocated", "tvk_max_memory_allocated", "tvk_memory_reserved"):
            getattr(lib, fn).argtypes = [C.c_int, C.POINTER(C.c_size_t)]
        lib.tvk_set_memory_limit.argtypes = [C.c_int, C.c_size_t]
        lib.tvk_set_strict_allocation.argtypes = [C.c_int]
        lib.tvk_get_strict_allocation.argtypes = [C.POINTER(C.c_int)]
        lib.tvk_last_malloc_spilled.argtypes = [C.POINTER(C.c_int)]
        lib.tvk_host_malloc.argtypes = [C.c_size_t, C.POINTER(C.c_void_p)]
        lib.tvk_host_free.argtypes = [C.c_void_p]
        lib.tvk_host_pointer_pinned.argtypes = [C.c_void_p, C.POINTER(C.c_int)]
        lib.tvk_mem_get_info.argtypes = [C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        lib.tvk_device_properties.argtypes = [C.c_int, C.POINTER(DeviceProps)]
        for fn in ("tvk_conv2d_fwd", "tvk_conv2d_dgrad", "tvk_conv2d_wgrad"):
            getattr(lib, fn).argtypes = [C.POINTER(ConvDesc)]
        for fn in ("tvk_conv_fwd", "tvk_conv_dgrad", "tvk_conv_wgrad"):
            getattr(lib, fn).argtypes = [C.POINTER(ConvNdDesc)]
        lib.tvk_conv_candidates.argtypes = [C.POINTER(ConvNdDesc), C.c_int, C.c_char_p, C.c_size_t]
        lib.tvk_conv_choose.argtypes = [C.POINTER(ConvNdDesc), C.c_int, C.c_char_p, C.c_int]
        lib.tvk_conv_tune.argtypes = [C.POINTER(ConvNdDesc), C.c_int, C.c_char_p, C.c_size_t]
        lib.tvk_copy.argtypes = [C.POINTER(CopyDesc)]
        lib.tvk_copy_plan.argtypes = [C.POINTER(CopyDesc), C.c_char_p, C.c_size_t]
        lib.tvk_fill.argtypes = [C.POINTER(FillDesc)]
        lib.tvk_reduce_sum.argtypes = [C.POINTER(ReduceDesc)]
        lib.tvk_binary.argtypes = [C.POINTER(BinaryDesc)]
        lib.tvk_attention_fwd.argtypes = [C.POINTER(AttentionDesc)]
        lib.tvk_attention_bwd.argtypes = [C.POINTER(AttentionBwdDesc)]
        lib.tvk_calibrate_mfma.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        lib.tvk_calibrate_mfma_operands.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double),
                                                    C.POINTER(C.c_double)]
        lib.tvk_calibrate_hbm.argtypes = [C.c_int, C.c_size_t, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        for fn in _ALL_ENTRY_POINTS:
            getattr(lib, fn).restype = C.c_int if fn != "tvk_last_error" else C.c_char_p
        _lib = lib
    return _lib


_ALL_ENTRY_POINTS = (
    "tvk_last_error", "tvk_device_count", "tvk_set_device", "tvk_get_device", "tvk_get_stream",
    "tvk_synchronize", "tvk_device_properties", "tvk_malloc", "tvk_free", "tvk_empty_cache",
    "tvk_pointer_device", "tvk_set_memory_limit", "tvk_set_strict_allocation", "tvk_get_strict_allocation",
    "tvk_last_malloc_spilled", "tvk_host_malloc", "tvk_host_free", "tvk_host_pointer_pinned", "tvk_memory_allocated", "tvk_max_memory_allocated",
    "tvk_memory_reserved", "tvk_reset_peak_memory_stats", "tvk_mem_get_info", "tvk_memcpy_h2d",
    "tvk_memcpy_d2h", "tvk_memcpy_d2d", "tvk_gemm", "tvk_gemm_plan", "tvk_gemm_candidates",
    "tvk_gemm_choose", "tvk_gemm_tune", "tvk_tune_reset", "tvk_tune_path",
    "tvk_conv2d_fwd", "tvk_conv2d_dgrad", "tvk_conv2d_wgrad", "tvk_conv_fwd", "tvk_conv_dgrad", "tvk_conv_wgrad",
    "tvk_conv_candidates", "tvk_conv_choose", "tvk_conv_tune",
    "tvk_copy", "tvk_copy_plan",
    "tvk_fill", "tvk_reduce_sum", "tvk_binary", "tvk_attention_fwd",
    "tvk_attention_bwd", "tvk_gemm_noalloc", "tvk_event_create", "tvk_event_destroy", "tvk_event_record",
    "tvk_event_query", "tvk_event_synchronize", "tvk_event_elapsed", "tvk_stream_wait_event", "tvk_stream_query",
    "tvk_calibrate_mfma", "tvk_calibrate_mfma_operands",
    "tvk_calibrate_hbm",
)


def check(status: int) -> None:
    if status == TVK_OK:
        return
    msg = load().tvk_last_error().decode(errors="replace")
    if status == TVK_ERR_UNSUPPORTED:
        raise TvkUnsupported(status, msg)
    if status == TVK_ERR_OOM:
        raise TvkOutOfMemory(status, msg)
    raise TvkError(status, msg)


def device_count() -> int:
    n = C.c_int(0)
    check(load().tvk_device_count(C.byref(n)))
    return n.value


# ---------------------------------------------------------------------------
# torch-tensor helpers (torch supplies device memory and the stream)
# ---------------------------------------------------------------------------

def _torch():
    import torch

    return torch


def calibrate_hbm(device: int = 0, window_bytes: int = 4096 * 14336 * 2, iterations: int = 60) -> tuple[float, float]:
    """(GB/s, ms per launch) of tvk_calibrate_hbm: a plain streaming read over three rotating windows."""
    gb, ms = C.c_double(), C.c_double()
    check(load().tvk_calibrate_hbm(device, window_bytes, iterations, C.byref(gb), C.byref(ms)))
    return gb.value, ms.value


def calibrate_mfma(device: int = 0, waves_per_simd: int = 2, iterations: int = 20000,
                   zeros: bool = False, mfma32: bool = False) -> tuple[float, float]:
    """(TFLOP/s, ms) of tvk_calibrate_mfma_operands: the float16 MFMA rate with random (or all-zero) operands,
    on v_mfma_f32_16x16x32_f16 (or v_mfma_f32_32x32x16_f16 with mfma32)."""
    tf, ms = C.c_double(), C.c_double()
    operands = (1 if zeros else 0) + (2 if mfma32 else 0)
    check(load().tvk_calibrate_mfma_operands(device, waves_per_simd, iterations, operands, C.byref(tf), C.byref(ms)))
    return tf.value, ms.value


def _dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: TVK_F32, torch.float16: TVK_F16, torch.bfloat16: TVK_BF16}
    if dtype not in codes:
        raise TvkUnsupported(TVK_ERR_UNSUPPORTED, f"dtype {dtype} is not on the dense-contraction path")
    return codes[dtype]


def copy_dtype_code(dtype) -> int:
    """tvk_dtype of a torch dtype tvk_copy handles (TvkUnsupported for the others)."""
    import torch

    codes = {torch.float32: TVK_F32, torch.float16: TVK_F16, torch.bfloat16: TVK_BF16, torch.float64: TVK_F64,
             torch.int64: TVK_I64, torch.int32: TVK_I32, torch.int16: TVK_I16, torch.int8: TVK_I8,
             torch.uint8: TVK_U8, torch.bool: TVK_BOOL, torch.float8_e4m3fn: TVK_F8E4M3FN,
             torch.float8_e5m2: TVK_F8E5M2}
    if dtype not in codes:
        raise TvkUnsupported(TVK_ERR_UNSUPPORTED, f"dtype {dtype} has no device copy")
    return codes[dtype]


def make_copy_desc(src, dst, stream=None) -> CopyDesc:
    """Describes dst.copy_(src) for device tensors; src is broadcast to dst's shape."""
    src = src.expand(dst.shape)
    if dst.dim() > TVK_COPY_MAX_DIMS:
        raise TvkUnsupported(TVK_ERR_UNSUPPORTED, f"{dst.dim()} dimensions")
    d = CopyDesc()
    d.src_dtype = copy_dtype_code(src.dtype)
    d.dst_dtype = copy_dtype_code(dst.dtype)
    d.ndim = dst.dim()
    d.reserved = 0
    d.sizes = I64xD(*dst.shape)
    d.src = src.data_ptr() if src.numel() else None
    d.src_strides = I64xD(*src.stride())
    d.dst = dst.data_ptr() if dst.numel() else None
    d.dst_strides = I64xD(*dst.stride())
    d.stream = stream
    return d


def copy(src, dst, stream=None) -> None:
    """dst.copy_(src) through tvk_copy (torch device tensors; torch's current stream by default)."""
    import torch

    if stream is None and dst.is_cuda:
        stream = torch.cuda.current_stream(dst.device).cuda_stream
    d = make_copy_desc(src, dst, stream)
    check(load().tvk_copy(C.byref(d)))


def copy_plan(src, dst) -> str:
    d = make_copy_desc(src, dst)
    buf = C.create_string_buffer(64)
    check(load().tvk_copy_plan(C.byref(d), buf, 64))
    return buf.value.decode()


def fill(dst, value, stream=None) -> None:
    """Fills a torch device tensor through tvk_fill; the element bytes come from a one-element CPU tensor."""
    import torch

    if stream is None and dst.is_cuda:
        stream = torch.cuda.current_stream(dst.device).cuda_stream
    one = torch.empty(1, dtype=dst.dtype).fill_(value)
    d = FillDesc()
    d.elem_size = dst.element_size()
    d.ndim = dst.dim()
    d.sizes = I64xD(*dst.shape)
    d.dst = dst.data_ptr() if dst.numel() else None
    d.dst_strides = I64xD(*dst.stride())
    d.pattern = int.from_bytes(one.view(torch.uint8).numpy().tobytes(), "little")
    d.stream = stream
    check(load().tvk_fill(C.byref(d)))


def _stream_of(t, stream):
    import torch

    if stream is None and t.is_cuda:
        stream = torch.cuda.current_stream(t.device).cuda_stream
    return stream


def reduce_sum(src, dims, keepdim=False, out_dtype=None, stream=None):
    """torch.sum(src, dims, keepdim, dtype=out_dtype) through tvk_reduce_sum (device tensors)."""
    import torch

    nd = src.dim()
    dims = [d % nd for d in dims] if dims else list(range(nd))
    out_dtype = out_dtype or src.dtype
    shape = [1 if d in dims else src.shape[d] for d in range(nd)] if keepdim else \
        [src.shape[d] for d in range(nd) if d not in dims]
    out = torch.empty(shape, dtype=out_dtype, device=src.device)
    d = ReduceDesc()
    d.src_dtype = copy_dtype_code(src.dtype)
    d.dst_dtype = copy_dtype_code(out_dtype)
    d.ndim = nd
    d.reduce_mask = sum(1 << k for k in dims)
    d.sizes = I64xD(*src.shape)
    d.src = src.data_ptr() if src.numel() else None
    d.src_strides = I64xD(*src.stride())
    view = out.view([1 if k in dims else src.shape[k] for k in range(nd)]) if out.numel() else out
    d.dst = out.data_ptr() if out.numel() else None
    d.dst_strides = I64xD(*[0 if k in dims else (view.stride(k) if out.numel() else 0) for k in range(nd)])
    d.stream = _stream_of(src, stream)
    check(load().tvk_reduce_sum(C.byref(d)))
    return out


def binary(a, b, out, op, alpha=1.0, stream=None) -> None:
    """out = op(a, b) through tvk_binary; a and b broadcast to out's shape (one dtype for all three)."""
    a, b = a.expand(out.shape), b.expand(out.shape)
    d = BinaryDesc()
    d.op = op
    d.dtype = copy_dtype_code(out.dtype)
    d.ndim = out.dim()
    d.reserved = 0
    d.sizes = I64xD(*out.shape)
    d.a, d.a_strides = a.data_ptr(), I64xD(*a.stride())
    d.b, d.b_strides = b.data_ptr(), I64xD(*b.stride())
    d.out, d.out_strides = out.data_ptr(), I64xD(*out.stride())
    d.alpha = float(alpha)
    d.stream = _stream_of(out, stream)
    check(load().tvk_binary(C.byref(d)))


def make_attention_desc(q, k, v, out, lse, bias=None, causal=False, scale=None, stream=None) -> AttentionDesc:
    """Describes tvk_attention_fwd over [B, H, L, D] device tensors (bias broadcast to [B, Hq, L, S])."""
    d = AttentionDesc()
    d.dtype = _dtype_code(q.dtype)
    d.causal = 1 if causal else 0
    d.batch, d.heads_q, d.len_q, d.head_dim = q.shape
    d.heads_kv, d.len_kv = k.shape[1], k.shape[2]
    d.head_dim_v = v.shape[3]
    d.q, d.q_stride = q.data_ptr(), I64x4(*q.stride())
    d.k, d.k_stride = k.data_ptr(), I64x4(*k.stride())
    d.v, d.v_stride = v.data_ptr(), I64x4(*v.stride())
    if bias is not None:
        be = bias.expand(q.shape[0], q.shape[1], q.shape[2], k.shape[2])
        d.bias, d.bias_stride = be.data_ptr(), I64x4(*be.stride())
    d.out, d.out_stride = out.data_ptr(), I64x4(*out.stride())
    d.lse, d.lse_stride = lse.data_ptr(), I64x3(*lse.stride())
    d.scale = float(scale if scale is not None else q.shape[3] ** -0.5)
    d.stream = stream
    return d


def attention_fwd(q, k, v, bias=None, causal=False, scale=None, stream=None):
    """(out, lse) of tvk_attention_fwd; out is a new [B, Hq, L, Dv] tensor, lse float32 [B, Hq, L]."""
    import torch

    out = torch.empty((q.shape[0], q.shape[1], q.shape[2], v.shape[3]), dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    d = make_attention_desc(q, k, v, out, lse, bias, causal, scale, _stream_of(q, stream))
    check(load().tvk_attention_fwd(C.byref(d)))
    return out, lse


def attention_bwd(q, k, v, out, lse, dout, bias=None, causal=False, scale=None, stream=None, dscores=False):
    """(dq, dk, dv) of tvk_attention_bwd (new dense tensors) from the forward's out and lse; with
    dscores=True also the float32 score gradient [B, Hq, L, S] as a fourth tensor."""
    import torch

    dq, dk, dv = torch.empty_like(q, memory_format=torch.contiguous_format), \
        torch.empty_like(k, memory_format=torch.contiguous_format), torch.empty_like(v, memory_format=torch.contiguous_format)
    d = AttentionBwdDesc()
    d.fwd = make_attention_desc(q, k, v, out, lse, bias, causal, scale, _stream_of(q, stream))
    d.dout, d.dout_stride = dout.data_ptr(), I64x4(*dout.stride())
    d.dq, d.dq_stride = dq.data_ptr(), I64x4(*dq.stride())
    d.dk, d.dk_stride = dk.data_ptr(), I64x4(*dk.stride())
    d.dv, d.dv_stride = dv.data_ptr(), I64x4(*dv.stride())
    ds = None
    if dscores:
        ds = torch.empty((q.shape[0], q.shape[1], q.shape[2], k.shape[2]), dtype=torch.float32, device=q.device)
        d.dscores, d.dscores_stride = ds.data_ptr(), I64x4(*ds.stride())
    check(load().tvk_attention_bwd(C.byref(d)))
    return (dq, dk, dv, ds) if dscores else (dq, dk, dv)


def _strides3(t) -> tuple[int, int, int]:
    if t.dim() == 2:
        return (0, t.stride(0), t.stride(1))
    if t.dim() in (3, 4):
        return (t.stride(0), t.stride(-2), t.stride(-1))
    raise ValueError("expected a 2-D, 3-D or 4-D tensor")


def make_gemm_desc(a, b, c, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, stream=None, exact=False) -> GemmDesc:
    """Describes C = act(alpha*A@B + beta*bias) over 2-D, batched 3-D or 4-D tensors.

    `bias` may be any tensor that broadcasts to C's shape (it is expanded with
    stride-0 views, as the reference's prepare_matmul_operands does). 4-D
    operands [B, H, rows, cols] use the descriptor's second batch dimension
    (batch_inner = H, the H strides), so head-strided views need no copy.
    """
    batch = c.shape[0] if c.dim() == 3 else (c.shape[0] * c.shape[1] if c.dim() == 4 else 1)
    M, N = c.shape[-2], c.shape[-1]
    K = a.shape[-1]
    d = GemmDesc()
    d.dtype = copy_dtype_code(c.dtype) if c.dtype not in (_torch().float32, _torch().float16, _torch().bfloat16) \
        else _dtype_code(c.dtype)
    d.activation = activation
    d.flags = TVK_GEMM_EXACT if exact else 0
    d.batch, d.M, d.N, d.K = batch, M, N, K
    d.a = a.data_ptr() if a.numel() else None
    d.a_stride = I64x3(*_strides3(a))
    d.b = b.data_ptr() if b.numel() else None
    d.b_stride = I64x3(*_strides3(b))
    if bias is not None:
        bias_e = bias.expand(c.shape)
        d.bias = bias_e.data_ptr()
        d.bias_stride = I64x3(*_strides3(bias_e))
    d.c = c.data_ptr() if c.numel() else None
    d.c_stride = I64x3(*_strides3(c))
    if c.dim() == 4:
        if a.dim() != 4 or b.dim() != 4:
            raise ValueError("a 4-D output needs 4-D operands")
        d.batch_inner = c.shape[1]
        d.a_stride_inner, d.b_stride_inner, d.c_stride_inner = a.stride(1), b.stride(1), c.stride(1)
        if bias is not None:
            d.bias_stride_inner = bias.expand(c.shape).stride(1)
    d.alpha = float(alpha)
    d.beta = float(beta)
    d.stream = stream
    return d


def gemm(a, b, c, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, stream=None, exact=False) -> None:
    """Runs tvk_gemm on torch device tensors; `stream` defaults to torch's current stream."""
    import torch

    if stream is None and c.is_cuda:
        stream = torch.cuda.current_stream(c.device).cuda_stream
    d = make_gemm_desc(a, b, c, bias, alpha, beta, activation, stream, exact)
    check(load().tvk_gemm(C.byref(d)))


def gemm_noalloc(a, b, c, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, stream=None, exact=False) -> None:
    """tvk_gemm_noalloc: tvk_gemm with its scratch in the library's fixed per-device array (no allocation)."""
    import torch

    if stream is None and c.is_cuda:
        stream = torch.cuda.current_stream(c.device).cuda_stream
    d = make_gemm_desc(a, b, c, bias, alpha, beta, activation, stream, exact)
    check(load().tvk_gemm_noalloc(C.byref(d)))


def gemm_plan(a, b, c, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, exact=False) -> str:
    d = make_gemm_desc(a, b, c, bias, alpha, beta, activation, None, exact)
    buf = C.create_string_buffer(128)
    check(load().tvk_gemm_plan(C.byref(d), buf, 128))
    return buf.value.decode()


def gemm_candidates(a, b, c, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, exact=False) -> list[str]:
    """Every kernel that computes this product (tvk_gemm_candidates), the shape-chosen one first."""
    d = make_gemm_desc(a, b, c, bias, alpha, beta, activation, None, exact)
    buf = C.create_string_buffer(4096)
    check(load().tvk_gemm_candidates(C.byref(d), buf, 4096))
    return buf.value.decode().split("\n")


def gemm_choose(a, b, c, kernel: str, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, exact=False,
                persist=False) -> None:
    """Records `kernel` for this product's shape class in the kernel-choice table (tvk_gemm_choose)."""
    d = make_gemm_desc(a, b, c, bias, alpha, beta, activation, None, exact)
    check(load().tvk_gemm_choose(C.byref(d), kernel.encode(), int(persist)))


def gemm_tune(a, b, c, bias=None, alpha=1.0, beta=0.0, activation=TVK_ACT_NONE, stream=None, exact=False) -> str:
    """tvk_gemm_tune: times the candidates when the shape class has no recorded choice, then runs the
    product; returns the kernel used."""
    import torch

    if stream is None and c.is_cuda:
        stream = torch.cuda.current_stream(c.device).cuda_stream
    d = make_gemm_desc(a, b, c, bias, alpha, beta, activation, stream, exact)
    buf = C.create_string_buffer(128)
    check(load().tvk_gemm_tune(C.byref(d), buf, 128))
    return buf.value.decode()


def tune_reset() -> None:
    check(load().tvk_tune_reset())


def tune_path() -> str:
    buf = C.create_string_buffer(4096)
    check(load().tvk_tune_path(buf, 4096))
    return buf.value.decode()


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def make_conv_desc(x_shape, w_shape, dtype, stride=1, padding=0, dilation=1, groups=1, x=None, weight=None, bias=None,
                   y=None, stream=None, exact=False) -> ConvDesc:
    """Describes a 2-D convolution over contiguous NCHW tensors (pointers from torch tensors or None)."""
    stride, padding, dilation = _pair(stride), _pair(padding), _pair(dilation)
    n, cin, h, w = x_shape
    cout, _, kh, kw = w_shape
    ho = (h + 2 * padding[0] - dilation[0] * (kh - 1) - 1) // stride[0] + 1
    wo = (w + 2 * padding[1] - dilation[1] * (kw - 1) - 1) // stride[1] + 1
    d = ConvDesc()
    d.dtype = _dtype_code(dtype)
    d.flags = TVK_GEMM_EXACT if exact else 0
    d.n, d.c_in, d.h, d.w, d.c_out, d.kh, d.kw = n, cin, h, w, cout, kh, kw
    d.stride = (C.c_int64 * 2)(*stride)
    d.padding = (C.c_int64 * 2)(*padding)
    d.dilation = (C.c_int64 * 2)(*dilation)
    d.groups = groups
    d.h_out, d.w_out = ho, wo
    ptr = lambda t: None if t is None or t.numel() == 0 else t.data_ptr()
    d.x, d.weight, d.bias, d.y = ptr(x), ptr(weight), ptr(bias), ptr(y)
    d.stream = stream
    return d


def _conv_call(fn, d):
    check(getattr(load(), fn)(C.byref(d)))


def conv2d_fwd(x, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, exact=False):
    """y = conv2d(x, weight) + bias through tvk_conv2d_fwd (torch device tensors, contiguous NCHW)."""
    import torch

    d = make_conv_desc(x.shape, weight.shape, x.dtype, stride, padding, dilation, groups, exact=exact)
    y = torch.empty((d.n, d.c_out, d.h_out, d.w_out), dtype=x.dtype, device=x.device)
    d.x, d.weight, d.y = x.data_ptr(), weight.data_ptr(), y.data_ptr()
    d.bias = None if bias is None else bias.data_ptr()
    d.stream = torch.cuda.current_stream(x.device).cuda_stream
    _conv_call("tvk_conv2d_fwd", d)
    return y


def conv2d_dgrad(dy, weight, x_shape, stride=1, padding=0, dilation=1, groups=1, exact=False):
    import torch

    d = make_conv_desc(x_shape, weight.shape, dy.dtype, stride, padding, dilation, groups, exact=exact)
    dx = torch.empty(tuple(x_shape), dtype=dy.dtype, device=dy.device)
    d.x, d.weight, d.y = dx.data_ptr(), weight.data_ptr(), dy.data_ptr()
    d.stream = torch.cuda.current_stream(dy.device).cuda_stream
    _conv_call("tvk_conv2d_dgrad", d)
    return dx


def conv2d_wgrad(x, dy, w_shape, stride=1, padding=0, dilation=1, groups=1, exact=False):
    import torch

    d = make_conv_desc(x.shape, w_shape, x.dtype, stride, padding, dilation, groups, exact=exact)
    dw = torch.empty(tuple(w_shape), dtype=x.dtype, device=x.device)
    d.x, d.weight, d.y = x.data_ptr(), dw.data_ptr(), dy.data_ptr()
    d.stream = torch.cuda.current_stream(x.device).cuda_stream
    _conv_call("tvk_conv2d_wgrad", d)
    return dw


def _nd(v, nd):
    return (v,) * nd if isinstance(v, int) else tuple(v)


def make_convnd_desc(x_shape, w_shape, dtype, stride=1, padding=0, dilation=1, groups=1, exact=False) -> ConvNdDesc:
    """Describes a convolution with 1-3 spatial dimensions over contiguous NC[D][H]W tensors."""
    nd = len(x_shape) - 2
    if nd < 1 or nd > 3 or len(w_shape) != nd + 2:
        raise ValueError(f"shapes {tuple(x_shape)} / {tuple(w_shape)} are not a 1-3 spatial-dimension convolution")
    s, p, dl = _nd(stride, nd), _nd(padding, nd), _nd(dilation, nd)
    k = tuple(w_shape[2:])
    o = tuple((x_shape[2 + i] + 2 * p[i] - dl[i] * (k[i] - 1) - 1) // s[i] + 1 for i in range(nd))
    pad3 = lambda v, fill: I64x3s(*(tuple(v) + (fill,) * (3 - nd)))
    d = ConvNdDesc()
    d.dtype = _dtype_code(dtype)
    d.flags = TVK_GEMM_EXACT if exact else 0
    d.spatial_dims = nd
    d.n, d.c_in, d.c_out, d.groups = x_shape[0], x_shape[1], w_shape[0], groups
    d.in_size, d.kernel, d.out_size = pad3(x_shape[2:], 1), pad3(k, 1), pad3(o, 1)
    d.stride, d.padding, d.dilation = pad3(s, 1), pad3(p, 0), pad3(dl, 1)
    return d


def conv_fwd(x, weight, bias=None, stride=1, padding=0, dilation=1, groups=1, exact=False):
    """y = conv(x, weight) + bias with 1-3 spatial dimensions through tvk_conv_fwd (contiguous device tensors)."""
    import torch

    d = make_convnd_desc(x.shape, weight.shape, x.dtype, stride, padding, dilation, groups, exact=exact)
    y = torch.empty((d.n, d.c_out) + tuple(d.out_size[:d.spatial_dims]), dtype=x.dtype, device=x.device)
    d.x, d.weight, d.y = x.data_ptr(), weight.data_ptr(), y.data_ptr()
    d.bias = None if bias is None else bias.data_ptr()
    d.stream = torch.cuda.current_stream(x.device).cuda_stream
    _conv_call("tvk_conv_fwd", d)
    return y


def conv_dgrad(dy, weight, x_shape, stride=1, padding=0, dilation=1, groups=1, exact=False):
    import torch

    d = make_convnd_desc(x_shape, weight.shape, dy.dtype, stride, padding, dilation, groups, exact=exact)
    dx = torch.empty(tuple(x_shape), dtype=dy.dtype, device=dy.device)
    d.x, d.weight, d.y = dx.data_ptr(), weight.data_ptr(), dy.data_ptr()
    d.stream = torch.cuda.current_stream(dy.device).cuda_stream
    _conv_call("tvk_conv_dgrad", d)
    return dx


def conv_wgrad(x, dy, w_shape, stride=1, padding=0, dilation=1, groups=1, exact=False):
    import torch

    d = make_convnd_desc(x.shape, w_shape, x.dtype, stride, padding, dilation, groups, exact=exact)
    dw = torch.empty(tuple(w_shape), dtype=x.dtype, device=x.device)
    d.x, d.weight, d.y = x.data_ptr(), dw.data_ptr(), dy.data_ptr()
    d.stream = torch.cuda.current_stream(x.device).cuda_stream
    _conv_call("tvk_conv_wgrad", d)
    return dw


TVK_CONV_FWD, TVK_CONV_DGRAD, TVK_CONV_WGRAD = 0, 1, 2
_CONV_ENTRY = {TVK_CONV_FWD: "tvk_conv_fwd", TVK_CONV_DGRAD: "tvk_conv_dgrad", TVK_CONV_WGRAD: "tvk_conv_wgrad"}


def conv_problem(x, weight, y, bias=None, stride=1, padding=0, dilation=1, groups=1, exact=False,
                 stream=None) -> ConvNdDesc:
    """The descriptor of one convolution over existing contiguous device tensors: x [N, C, ...], weight,
    y [N, C_out, ...] (which one a call writes depends on its mode)."""
    import torch

    d = make_convnd_desc(x.shape, weight.shape, x.dtype, stride, padding, dilation, groups, exact=exact)
    if tuple(y.shape) != (d.n, d.c_out) + tuple(d.out_size[:d.spatial_dims]):
        raise ValueError(f"y has shape {tuple(y.shape)}; the geometry gives {(d.n, d.c_out) + tuple(d.out_size[:d.spatial_dims])}")
    d.x, d.weight, d.y = x.data_ptr(), weight.data_ptr(), y.data_ptr()
    d.bias = None if bias is None else bias.data_ptr()
    d.stream = stream if stream is not None else torch.cuda.current_stream(x.device).cuda_stream
    return d


def conv_run(d: ConvNdDesc, mode: int) -> None:
    _conv_call(_CONV_ENTRY[mode], d)


def conv_candidates(d: ConvNdDesc, mode: int) -> list[str]:
    """Kernel families that compute the convolution (tvk_conv_candidates), the shape-chosen one first."""
    buf = C.create_string_buffer(256)
    check(load().tvk_conv_candidates(C.byref(d), mode, buf, len(buf)))
    return buf.value.decode().split("\n")


def conv_choose(d: ConvNdDesc, mode: int, kernel: str, persist: bool = False) -> None:
    """Records `kernel` for the convolution's shape class (tvk_conv_choose)."""
    check(load().tvk_conv_choose(C.byref(d), mode, kernel.encode(), 1 if persist else 0))


def conv_tune(d: ConvNdDesc, mode: int) -> str:
    """Runs the convolution through tvk_conv_tune; returns the family used."""
    buf = C.create_string_buffer(64)
    check(load().tvk_conv_tune(C.byref(d), mode, buf, len(buf)))
    return buf.value.decode()

