// sum and add/sub/mul on the vulkan device, the reductions and element-wise
// ops next to the contractions (bias gradients, gradient accumulation,
// residual adds). Registered as the reference registers them
// (src/api/ops/reduce.cpp:750-751, src/api/ops/binary.cpp:1090-1118); the
// arithmetic runs in tvk_reduce_sum / tvk_binary.
#include "common.h"

#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/WrapDimUtilsMulti.h>
#include <ATen/native/BinaryOps.h>
#include <ATen/native/Resize.h>

#include <bitset>
#include <functional>

#include <cstring>

namespace tvkb {
namespace {

// ---------------------------------------------------------------------------
// sum
// ---------------------------------------------------------------------------

// reduce_compute_dtype (src/api/ops/helpers.h:466-473): the requested dtype,
// else int64 for integral and bool inputs, else the input's
at::ScalarType sum_dtype(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
    if (dtype.has_value()) return *dtype;
    if (at::isIntegralType(self.scalar_type(), /*includeBool=*/true) && self.scalar_type() != at::kLong) return at::kLong;
    return self.scalar_type();
}

bool sum_on_device(const at::Tensor& self, at::ScalarType out) {
    bool ok = false;
    copy_dtype_of(self.scalar_type(), ok);
    const bool out_ok = out == at::kFloat || out == at::kHalf || out == at::kBFloat16 || out == at::kDouble || out == at::kLong;
    return ok && out_ok && !at::isFloat8Type(self.scalar_type()) && self.dim() <= TVK_COPY_MAX_DIMS && !self.is_conj() &&
           !self.is_neg();
}

at::Tensor sum_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim, std::optional<at::ScalarType> dtype) {
    const at::ScalarType out_dtype = sum_dtype(self, dtype);
    const int64_t nd = self.dim();
    std::bitset<64> mask;
    if (dim.has_value() && !dim->empty()) mask = at::dim_list_to_bitset(*dim, nd);   // CPU's checks and messages
    else for (int64_t d = 0; d < nd; ++d) mask.set(d);
    if (!sum_on_device(self, out_dtype)) {
        TVKB_FALLBACK("A sum of ", self.scalar_type(), " to ", out_dtype, " can't run on the device. Falling back to CPU.");
        return at::sum(self.cpu(), dim, keepdim, dtype).to(self.device());
    }
    std::vector<int64_t> out_shape;
    for (int64_t d = 0; d < nd; ++d) {
        if (!mask[d]) out_shape.push_back(self.size(d));
        else if (keepdim) out_shape.push_back(1);
    }
    at::Tensor out = at::empty(out_shape, self.options().dtype(out_dtype));
    if (out.numel() == 0) return out;
    tvk_reduce_desc d;
    std::memset(&d, 0, sizeof(d));
    bool ok = false;
    d.src_dtype = copy_dtype_of(self.scalar_type(), ok);
    d.dst_dtype = copy_dtype_of(out_dtype, ok);
    d.ndim = (int32_t)nd;
    int64_t od = 0;
    for (int64_t k = 0; k < nd; ++k) {
        d.sizes[k] = self.size(k);
        d.src_strides[k] = self.stride(k);
        if (mask[k]) {
            d.reduce_mask |= 1u << k;
            d.dst_strides[k] = 0;
            if (keepdim) ++od;
        } else {
            d.dst_strides[k] = out.stride(od++);
        }
    }
    d.src = self.numel() ? self.data_ptr() : nullptr;
    d.dst = out.data_ptr();
    d.stream = stream_of(self);
    check_status(tvk_reduce_sum(&d), "tvk_reduce_sum");
    return out;
}

at::Tensor sum_all(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
    return sum_dim(self, at::OptionalIntArrayRef(), false, dtype);
}

// ---------------------------------------------------------------------------
// add / sub / mul
// ---------------------------------------------------------------------------

bool is_cpu_scalar(const at::Tensor& t) {
    return t.unsafeGetTensorImpl()->is_wrapped_number() || (t.dim() == 0 && t.device().is_cpu());
}

bool binary_dtype_ok(at::ScalarType t) {
    return t == at::kFloat || t == at::kHalf || t == at::kBFloat16 || t == at::kDouble || t == at::kLong ||
           t == at::kInt || t == at::kShort || t == at::kChar || t == at::kByte;
}

// fits_dtype (src/api/ops/binary.cpp:133-140): a float scalar a float16 or
// bfloat16 cannot hold sends the op to float32
bool fits_low_prec(const at::Scalar& s, at::ScalarType dtype) {
    if (s.isComplex() || !s.isFloatingPoint()) return true;
    const double v = s.toDouble();
    if (!std::isfinite(v)) return true;
    return std::abs(v) <= (dtype == at::kHalf ? 65504.0 : 3.3895313892515355e38);
}

// The operand as a device tensor of dtype t (a CPU scalar becomes a 0-dim
// device tensor holding its value converted to t).
at::Tensor operand(const at::Tensor& x, at::ScalarType t, const at::Device& dev) {
    if (is_cpu_scalar(x)) {
        at::Tensor v = at::empty({}, x.options().dtype(t).device(dev));
        v.fill_(x.item());
        return v;
    }
    return x.scalar_type() == t ? x : x.to(t);
}

using CpuFn = std::function<at::Tensor(const at::Tensor&, const at::Tensor&)>;

// out (defined: written in place / as .out) = op(self, other)
at::Tensor binary(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha, int op, at::Tensor out,
                  const CpuFn& cpu_op, bool inplace = false) {
    const at::ScalarType common = at::result_type(self, other);
    if (op != TVK_BIN_MUL) at::native::alpha_check(common, alpha);
    const at::Tensor& dev_t = self.is_privateuseone() ? self : other;
    if (!is_cpu_scalar(self) && !is_cpu_scalar(other) && self.device() != other.device())
        TORCH_CHECK(false, "Expected all tensors to be on the same device, but found at least two devices, ", dev_t.device(),
                    " and ", (self.is_privateuseone() ? other : self).device(), "!");
    at::ScalarType compute = common;
    const bool scalar_other = is_cpu_scalar(other) && !is_cpu_scalar(self);
    if ((common == at::kHalf || common == at::kBFloat16) &&
        ((scalar_other && !fits_low_prec(other.item(), common)) || (op != TVK_BIN_MUL && !fits_low_prec(alpha, common))))
        compute = at::kFloat;
    const std::vector<int64_t> shape = at::infer_size(self.sizes(), other.sizes());
    if (inplace)
        TORCH_CHECK(self.sizes().equals(shape), "output with shape ", self.sizes(), " doesn't match the broadcast shape ",
                    c10::IntArrayRef(shape));
    if (out.defined()) {
        TORCH_CHECK(at::canCast(common, out.scalar_type()), "result type ", common, " can't be cast to the desired output type ",
                    out.scalar_type());
    }
    if (!binary_dtype_ok(compute) || shape.size() > TVK_COPY_MAX_DIMS || self.is_complex() || other.is_complex()) {
        TVKB_FALLBACK("A binary op on ", common, " can't run on the device. Falling back to CPU.");
        at::Tensor r = cpu_op(self.cpu(), other.cpu());
        if (!out.defined()) return r.to(dev_t.device());
        at::native::resize_output(out, r.sizes());
        out.copy_(r);
        return out;
    }
    const at::Tensor a = operand(self, compute, dev_t.device()).expand(shape);
    const at::Tensor b = operand(other, compute, dev_t.device()).expand(shape);
    at::Tensor dst;
    if (out.defined()) {
        at::native::resize_output(out, shape);
        at::assert_no_internal_overlap(out);
        at::assert_no_partial_overlap(out, a);
        at::assert_no_partial_overlap(out, b);
        dst = out.scalar_type() == compute ? out : at::empty(shape, out.options().dtype(compute));
    } else {
        dst = at::empty(shape, dev_t.options().dtype(compute));
    }
    if (dst.numel() > 0) {
        tvk_binary_desc d;
        std::memset(&d, 0, sizeof(d));
        bool ok = false;
        d.op = op;
        d.dtype = copy_dtype_of(compute, ok);
        d.ndim = (int32_t)shape.size();
        for (size_t k = 0; k < shape.size(); ++k) {
            d.sizes[k] = shape[k];
            d.a_strides[k] = a.stride(k);
            d.b_strides[k] = b.stride(k);
            d.out_strides[k] = dst.stride(k);
        }
        d.a = a.data_ptr();
        d.b = b.data_ptr();
        d.out = dst.data_ptr();
        d.alpha = op == TVK_BIN_MUL ? 1.0 : alpha.toDouble();
        d.stream = stream_of(dst);
        check_status(tvk_binary(&d), "tvk_binary");
    }
    if (out.defined()) {
        if (!dst.is_same(out)) out.copy_(dst);
        return out;
    }
    return compute == common ? dst : dst.to(common);
}

at::Tensor add_t(const at::Tensor& s, const at::Tensor& o, const at::Scalar& alpha) {
    if (s.scalar_type() == at::kBool && o.scalar_type() == at::kBool) {
        TVKB_FALLBACK("A bool add can't run on the device. Falling back to CPU.");
        return at::add(s.cpu(), o.cpu(), alpha).to(s.device());
    }
    return binary(s, o, alpha, TVK_BIN_ADD, at::Tensor(), [&](const at::Tensor& a, const at::Tensor& b) { return at::add(a, b, alpha); });
}
at::Tensor& add_i(at::Tensor& s, const at::Tensor& o, const at::Scalar& alpha) {
    binary(s, o, alpha, TVK_BIN_ADD, s, [&](const at::Tensor& a, const at::Tensor& b) { return at::add(a, b, alpha); }, true);
    return s;
}
at::Tensor& add_o(const at::Tensor& s, const at::Tensor& o, const at::Scalar& alpha, at::Tensor& out) {
    binary(s, o, alpha, TVK_BIN_ADD, out, [&](const at::Tensor& a, const at::Tensor& b) { return at::add(a, b, alpha); });
    return out;
}
at::Tensor sub_t(const at::Tensor& s, const at::Tensor& o, const at::Scalar& alpha) {
    at::native::sub_check(s, o);
    return binary(s, o, alpha, TVK_BIN_SUB, at::Tensor(), [&](const at::Tensor& a, const at::Tensor& b) { return at::sub(a, b, alpha); });
}
at::Tensor& sub_i(at::Tensor& s, const at::Tensor& o, const at::Scalar& alpha) {
    at::native::sub_check(s, o);
    binary(s, o, alpha, TVK_BIN_SUB, s, [&](const at::Tensor& a, const at::Tensor& b) { return at::sub(a, b, alpha); }, true);
    return s;
}
at::Tensor& sub_o(const at::Tensor& s, const at::Tensor& o, const at::Scalar& alpha, at::Tensor& out) {
    at::native::sub_check(s, o);
    binary(s, o, alpha, TVK_BIN_SUB, out, [&](const at::Tensor& a, const at::Tensor& b) { return at::sub(a, b, alpha); });
    return out;
}
at::Tensor mul_t(const at::Tensor& s, const at::Tensor& o) {
    if (s.scalar_type() == at::kBool && o.scalar_type() == at::kBool) {
        TVKB_FALLBACK("A bool mul can't run on the device. Falling back to CPU.");
        return at::mul(s.cpu(), o.cpu()).to(s.device());
    }
    return binary(s, o, 1, TVK_BIN_MUL, at::Tensor(), [](const at::Tensor& a, const at::Tensor& b) { return at::mul(a, b); });
}
at::Tensor& mul_i(at::Tensor& s, const at::Tensor& o) {
    binary(s, o, 1, TVK_BIN_MUL, s, [](const at::Tensor& a, const at::Tensor& b) { return at::mul(a, b); }, true);
    return s;
}
at::Tensor& mul_o(const at::Tensor& s, const at::Tensor& o, at::Tensor& out) {
    binary(s, o, 1, TVK_BIN_MUL, out, [](const at::Tensor& a, const at::Tensor& b) { return at::mul(a, b); });
    return out;
}

}  // namespace
}  // namespace tvkb

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
    m.impl("sum.dim_IntList", &tvkb::sum_dim);
    m.impl("sum", &tvkb::sum_all);
    m.impl("add.Tensor", &tvkb::add_t);
    m.impl("add_.Tensor", &tvkb::add_i);
    m.impl("add.out", &tvkb::add_o);
    m.impl("sub.Tensor", &tvkb::sub_t);
    m.impl("sub_.Tensor", &tvkb::sub_i);
    m.impl("sub.out", &tvkb::sub_o);
    m.impl("mul.Tensor", &tvkb::mul_t);
    m.impl("mul_.Tensor", &tvkb::mul_i);
    m.impl("mul.out", &tvkb::mul_o);
}
