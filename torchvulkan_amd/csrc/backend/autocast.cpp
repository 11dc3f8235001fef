// Automatic mixed precision for the vulkan (PrivateUse1) device, as the
// reference registers it (src/api/registration.cpp:4-21).
//
// Under `torch.autocast("vulkan", dtype)` the AutocastPrivateUse1 key sits in
// front of PrivateUse1. Every op without an autocast kernel falls through to
// its ordinary kernel; the op lists below are torch's own policy tables
// (ATen/autocast_mode.h), so the casts are exactly the ones torch applies on
// its other devices:
//  - lower_precision_fp: mm, addmm, bmm, baddbmm, addbmm, linear, matmul,
//    conv{1,2,3}d, conv_transpose*, _convolution, SDPA, ... run in the autocast
//    dtype. Their floating-point tensor arguments are cast first (tvk_copy on
//    the device; the weight casts are cached for the autocast region), and the
//    op then reaches the fp16/bf16 MFMA kernels of this backend.
//  - fp32 / fp32_set_opt_dtype: reductions and losses that torch runs in
//    float32 under autocast.
//  - promote: ops that take the widest floating type of their arguments.
#include <ATen/autocast_mode.h>
#include <torch/library.h>

TORCH_LIBRARY_IMPL(_, AutocastPrivateUse1, m) {
    m.fallback(torch::CppFunction::makeFallthrough());
}

namespace at::autocast {

TORCH_LIBRARY_IMPL(aten, AutocastPrivateUse1, m) {
#define TVKB_AUTOCAST_LOWER(...) KERNEL_PRIVATEUSEONE(__VA_ARGS__, lower_precision_fp)
#define TVKB_AUTOCAST_FP32(...) KERNEL_PRIVATEUSEONE(__VA_ARGS__, fp32)
#define TVKB_AUTOCAST_FP32_OPT(...) KERNEL_PRIVATEUSEONE(__VA_ARGS__, fp32_set_opt_dtype)
#define TVKB_AUTOCAST_PROMOTE(...) KERNEL_PRIVATEUSEONE(__VA_ARGS__, promote)
    AT_FORALL_LOWER_PRECISION_FP(TVKB_AUTOCAST_LOWER)
    AT_FORALL_FP32(TVKB_AUTOCAST_FP32)
    AT_FORALL_FP32_SET_OPT_DTYPE(TVKB_AUTOCAST_FP32_OPT)
    AT_FORALL_DIFFERENT_REDISPATCH_SIGNATURE(KERNEL_DIFFERENT_REDISPATCH_SIGNATURE_PRIVATEUSEONE)
    AT_FORALL_PROMOTE(TVKB_AUTOCAST_PROMOTE)
#undef TVKB_AUTOCAST_LOWER
#undef TVKB_AUTOCAST_FP32
#undef TVKB_AUTOCAST_FP32_OPT
#undef TVKB_AUTOCAST_PROMOTE
}

}  // namespace at::autocast
