// aten::convolution_overrideable / convolution_backward_overrideable for the
// vulkan (PrivateUse1) device, computed by tvk_conv2d_{fwd,dgrad,wgrad}.
//
// Follows convolution_vulkan and convolution_backward_vulkan
// (src/api/ops/conv.cpp:1088-1172): the input is cast to the weight's dtype,
// operands are made contiguous NCHW, transposed convolution runs the
// grad-input kernel forward (and the forward kernel for its input gradient),
// the bias gradient is a sum over (N, H, W), and the output takes the inputs'
// memory format (conv.cpp:1080-1086). Shapes the implicit-GEMM kernels do not
// take (other than 2-D spatial, non-float dtypes) run on the CPU through the
// fallback path with the reference's warning.
#include "common.h"

namespace tvkb {
namespace {

std::vector<int64_t> ints(c10::SymIntArrayRef a) {
    std::vector<int64_t> v;
    for (const auto& x : a) v.push_back(x.guard_int(__FILE__, __LINE__));
    return v;
}

std::vector<int64_t> expand2(std::vector<int64_t> v) {
    if (v.size() == 1) v.push_back(v[0]);
    return v;
}

at::MemoryFormat conv_memory_format(const at::Tensor& input, const at::Tensor& weight) {
    for (at::MemoryFormat f : {input.suggest_memory_format(), weight.suggest_memory_format()})
        if (f != at::MemoryFormat::Contiguous) return f;
    return at::MemoryFormat::Contiguous;
}

bool supported(const at::Tensor& x, const at::Tensor& w) {
    bool ok = false;
    (void)tvk_dtype_of(w.scalar_type(), ok);
    return ok && x.dim() == 4 && w.dim() == 4;
}

bool exact_env() {
    const char* e = std::getenv("TORCHVULKAN_EXACT");
    return e && e[0] && std::strcmp(e, "0") != 0;
}

// x: [n, c_in, h, w] (the forward input), w: [c_out, c_in/g, kh, kw], y spatial (ho, wo)
tvk_conv_desc make_desc(const at::Tensor& x_like, int64_t c_in, int64_t h, int64_t wd, const at::Tensor& w, int64_t groups,
                        const std::vector<int64_t>& stride, const std::vector<int64_t>& padding,
                        const std::vector<int64_t>& dilation, int64_t ho, int64_t wo) {
    tvk_conv_desc d;
    std::memset(&d, 0, sizeof(d));
    bool ok = false;
    d.dtype = tvk_dtype_of(w.scalar_type(), ok);
    d.flags = exact_env() ? TVK_GEMM_EXACT : 0;
    d.n = x_like.size(0);
    d.c_in = c_in;
    d.h = h;
    d.w = wd;
    d.c_out = w.size(0);
    d.kh = w.size(2);
    d.kw = w.size(3);
    for (int i = 0; i < 2; ++i) {
        d.stride[i] = stride[i];
        d.padding[i] = padding[i];
        d.dilation[i] = dilation[i];
    }
    d.groups = groups;
    d.h_out = ho;
    d.w_out = wo;
    d.stream = stream_of(w);
    return d;
}

int64_t out_size(int64_t in, int64_t k, int64_t s, int64_t p, int64_t d) { return (in + 2 * p - d * (k - 1) - 1) / s + 1; }

at::Tensor conv_forward_impl(const at::Tensor& x, const at::Tensor& w, const at::Tensor& b, const std::vector<int64_t>& s,
                             const std::vector<int64_t>& p, const std::vector<int64_t>& dl, int64_t groups) {
    const int64_t ho = out_size(x.size(2), w.size(2), s[0], p[0], dl[0]);
    const int64_t wo = out_size(x.size(3), w.size(3), s[1], p[1], dl[1]);
    at::Tensor y = at::empty({x.size(0), w.size(0), ho, wo}, x.options());
    tvk_conv_desc d = make_desc(x, x.size(1), x.size(2), x.size(3), w, groups, s, p, dl, ho, wo);
    d.x = x.data_ptr();
    d.weight = w.data_ptr();
    d.bias = b.defined() ? b.data_ptr() : nullptr;
    d.y = y.data_ptr();
    check_status(tvk_conv2d_fwd(&d), "tvk_conv2d_fwd");
    return y;
}

// input gradient of a forward conv: dy [n, c_out, ho, wo] -> dx [n, c_in, h, w]
at::Tensor conv_dgrad_impl(const at::Tensor& dy, const at::Tensor& w, int64_t c_in, int64_t h, int64_t wd,
                           const std::vector<int64_t>& s, const std::vector<int64_t>& p, const std::vector<int64_t>& dl,
                           int64_t groups) {
    at::Tensor dx = at::empty({dy.size(0), c_in, h, wd}, dy.options());
    tvk_conv_desc d = make_desc(dy, c_in, h, wd, w, groups, s, p, dl, dy.size(2), dy.size(3));
    d.x = dx.data_ptr();
    d.weight = w.data_ptr();
    d.y = dy.data_ptr();
    check_status(tvk_conv2d_dgrad(&d), "tvk_conv2d_dgrad");
    return dx;
}

at::Tensor conv_wgrad_impl(const at::Tensor& x, const at::Tensor& dy, c10::IntArrayRef w_sizes, const std::vector<int64_t>& s,
                           const std::vector<int64_t>& p, const std::vector<int64_t>& dl, int64_t groups) {
    at::Tensor dw = at::empty(w_sizes, x.options());
    tvk_conv_desc d = make_desc(x, x.size(1), x.size(2), x.size(3), dw, groups, s, p, dl, dy.size(2), dy.size(3));
    d.x = x.data_ptr();
    d.weight = dw.data_ptr();
    d.y = dy.data_ptr();
    check_status(tvk_conv2d_wgrad(&d), "tvk_conv2d_wgrad");
    return dw;
}

at::Tensor convolution(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                       c10::SymIntArrayRef stride_, c10::SymIntArrayRef padding_, c10::SymIntArrayRef dilation_,
                       bool transposed, c10::SymIntArrayRef output_padding_, c10::SymInt groups_) {
    const int64_t groups = groups_.guard_int(__FILE__, __LINE__);
    auto s = expand2(ints(stride_)), p = expand2(ints(padding_)), dl = expand2(ints(dilation_)), op = expand2(ints(output_padding_));
    const at::MemoryFormat format = conv_memory_format(input, weight);
    if (!supported(input, weight) || s.size() != 2) {
        TVKB_FALLBACK("A ", weight.scalar_type(), " ", weight.dim() - 2, "-d convolution can't run on the Vulkan device. Falling back to CPU.");
        std::optional<at::Tensor> bc = bias.has_value() && bias->defined() ? std::optional<at::Tensor>(bias->cpu()) : std::nullopt;
        return at::convolution(input.cpu(), weight.cpu(), bc, s, p, dl, transposed, op, groups).to(input.device()).contiguous(format);
    }
    at::Tensor x = input.to(weight.scalar_type()).contiguous();
    at::Tensor w = weight.contiguous();
    at::Tensor b = bias.has_value() && bias->defined() ? bias->to(x.scalar_type()).contiguous() : at::Tensor();
    at::Tensor y;
    if (!transposed) {
        y = conv_forward_impl(x, w, b, s, p, dl, groups);
    } else {
        // transposed: w is [c_in, c_out/g, kh, kw]; the output is the input
        // gradient of the forward conv whose output x is
        const int64_t h = (x.size(2) - 1) * s[0] - 2 * p[0] + dl[0] * (w.size(2) - 1) + op[0] + 1;
        const int64_t wd = (x.size(3) - 1) * s[1] - 2 * p[1] + dl[1] * (w.size(3) - 1) + op[1] + 1;
        y = conv_dgrad_impl(x, w, w.size(1) * groups, h, wd, s, p, dl, groups);
        if (b.defined()) y = y + b.view({1, -1, 1, 1});
    }
    return y.contiguous(format);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> convolution_backward(
    const at::Tensor& grad_output, const at::Tensor& input, const at::Tensor& weight, c10::SymIntArrayRef stride_,
    c10::SymIntArrayRef padding_, c10::SymIntArrayRef dilation_, bool transposed, c10::SymIntArrayRef output_padding_,
    c10::SymInt groups_, std::array<bool, 3> mask) {
    const int64_t groups = groups_.guard_int(__FILE__, __LINE__);
    auto s = expand2(ints(stride_)), p = expand2(ints(padding_)), dl = expand2(ints(dilation_)), op = expand2(ints(output_padding_));
    const at::MemoryFormat format = conv_memory_format(input, weight);
    at::Tensor gi, gw, gb;
    if (!supported(input, weight) || s.size() != 2 || grad_output.scalar_type() != weight.scalar_type() ||
        input.scalar_type() != weight.scalar_type()) {
        TVKB_FALLBACK("A ", weight.scalar_type(), " ", weight.dim() - 2, "-d convolution backward can't run on the Vulkan device. Falling back to CPU.");
        auto r = at::convolution_backward(grad_output.cpu(), input.cpu(), weight.cpu(), std::nullopt, s, p, dl, transposed, op,
                                          groups, mask);
        auto dev = [&](const at::Tensor& t) { return t.defined() ? t.to(input.device()).contiguous(format) : t; };
        return {dev(std::get<0>(r)), dev(std::get<1>(r)), dev(std::get<2>(r))};
    }
    at::Tensor go = grad_output.contiguous();
    at::Tensor in = input.contiguous();
    at::Tensor w = weight.contiguous();
    if (!transposed) {
        if (mask[0]) gi = conv_dgrad_impl(go, w, in.size(1), in.size(2), in.size(3), s, p, dl, groups);
        if (mask[1]) gw = conv_wgrad_impl(in, go, w.sizes(), s, p, dl, groups);
    } else {
        // forward conv with input go and output `in`
        if (mask[0]) gi = conv_forward_impl(go, w, at::Tensor(), s, p, dl, groups);
        if (mask[1]) gw = conv_wgrad_impl(go, in, w.sizes(), s, p, dl, groups);
    }
    if (mask[2]) gb = at::sum(grad_output, {0, 2, 3});
    if (gi.defined()) gi = gi.contiguous(format);
    if (gw.defined()) gw = gw.contiguous(format);
    return {gi, gw, gb};
}

}  // namespace
}  // namespace tvkb

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
    m.impl("convolution_overrideable", &tvkb::convolution);
    m.impl("convolution_backward_overrideable", &tvkb::convolution_backward);
}
