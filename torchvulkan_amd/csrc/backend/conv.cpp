// aten::convolution_overrideable / convolution_backward_overrideable for the
// vulkan (PrivateUse1) device, computed by tvk_conv_{fwd,dgrad,wgrad} for one
// to three spatial dimensions (the reference's bound, conv.cpp:295-311).
//
// Follows convolution_vulkan and convolution_backward_vulkan
// (src/api/ops/conv.cpp:1088-1172): the input is cast to the weight's dtype,
// operands are made contiguous NC(D)HW, transposed convolution runs the
// grad-input kernel forward (and the forward kernel for its input gradient),
// the bias gradient is a sum over (N, spatial), and the output takes the
// inputs' memory format (conv.cpp:1080-1086). float64 and integer
// convolutions run as a device im2col plus the wide GEMM (the reference's
// im2col_nd + matmul, conv.cpp:32-58,200-216). Other dtypes (complex, bool)
// run on the CPU through the fallback path with the reference's warning.
#include "common.h"

#include <ATen/native/Resize.h>

namespace tvkb {
namespace {

std::vector<int64_t> ints(c10::SymIntArrayRef a) {
    std::vector<int64_t> v;
    for (const auto& x : a) v.push_back(x.guard_int(__FILE__, __LINE__));
    return v;
}

// one value per spatial dimension (a single value applies to all of them)
std::vector<int64_t> expand_nd(std::vector<int64_t> v, size_t nd) {
    if (v.size() == 1 && nd > 1) v.resize(nd, v[0]);
    return v;
}

at::MemoryFormat conv_memory_format(const at::Tensor& input, const at::Tensor& weight) {
    for (at::MemoryFormat f : {input.suggest_memory_format(), weight.suggest_memory_format()})
        if (f != at::MemoryFormat::Contiguous) return f;
    return at::MemoryFormat::Contiguous;
}

// 1 to 3 spatial dimensions, every geometry vector of that length
bool geometry_ok(const at::Tensor& x, const at::Tensor& w, const std::vector<int64_t>& s) {
    const int64_t nd = w.dim() - 2;
    return nd >= 1 && nd <= 3 && x.dim() == w.dim() && (int64_t)s.size() == nd;
}

bool supported(const at::Tensor& x, const at::Tensor& w, const std::vector<int64_t>& s) {
    bool ok = false;
    (void)tvk_dtype_of(w.scalar_type(), ok);
    return ok && geometry_ok(x, w, s);
}

// TORCHVULKAN_EXACT is read once, at the first convolution
bool exact_env() {
    static const bool exact = [] {
        const char* e = std::getenv("TORCHVULKAN_EXACT");
        return e && e[0] && std::strcmp(e, "0") != 0;
    }();
    return exact;
}

// TORCHVULKAN_AUTOTUNE=1: a convolution whose shape class has no recorded
// kernel family times every candidate first and records the fastest (the
// reference tunes its conv tilings on first sight, src/api/ops/conv.cpp:643-651)
tvk_status run_conv_mode(tvk_convnd_desc& d, int mode) {
    static const bool autotune = [] {
        const char* e = std::getenv("TORCHVULKAN_AUTOTUNE");
        return e != nullptr && e[0] && std::strcmp(e, "0") != 0;
    }();
    if (autotune) return tvk_conv_tune(&d, mode, nullptr, 0);
    return mode == TVK_CONV_FWD ? tvk_conv_fwd(&d) : mode == TVK_CONV_DGRAD ? tvk_conv_dgrad(&d) : tvk_conv_wgrad(&d);
}

int64_t out_size(int64_t in, int64_t k, int64_t s, int64_t p, int64_t d) { return (in + 2 * p - d * (k - 1) - 1) / s + 1; }

std::vector<int64_t> out_sizes(c10::IntArrayRef in_sp, c10::IntArrayRef k, const std::vector<int64_t>& s,
                               const std::vector<int64_t>& p, const std::vector<int64_t>& dl) {
    std::vector<int64_t> o;
    for (size_t i = 0; i < in_sp.size(); ++i) o.push_back(out_size(in_sp[i], k[i], s[i], p[i], dl[i]));
    return o;
}

// spatial extent of a transposed convolution's output (the input gradient's)
std::vector<int64_t> transposed_sizes(c10::IntArrayRef in_sp, c10::IntArrayRef k, const std::vector<int64_t>& s,
                                      const std::vector<int64_t>& p, const std::vector<int64_t>& dl,
                                      const std::vector<int64_t>& op) {
    std::vector<int64_t> o;
    for (size_t i = 0; i < in_sp.size(); ++i) o.push_back((in_sp[i] - 1) * s[i] - 2 * p[i] + dl[i] * (k[i] - 1) + op[i] + 1);
    return o;
}

std::vector<int64_t> cat_shape(int64_t a, int64_t b, c10::IntArrayRef rest) {
    std::vector<int64_t> v{a, b};
    v.insert(v.end(), rest.begin(), rest.end());
    return v;
}

// x spatial in_sp (the forward input's), w: [c_out, c_in/g, kernel...], y spatial out_sp
tvk_convnd_desc make_desc(int64_t n, int64_t c_in, c10::IntArrayRef in_sp, const at::Tensor& w, int64_t groups,
                          const std::vector<int64_t>& stride, const std::vector<int64_t>& padding,
                          const std::vector<int64_t>& dilation, c10::IntArrayRef out_sp) {
    tvk_convnd_desc d;
    std::memset(&d, 0, sizeof(d));
    bool ok = false;
    d.dtype = tvk_dtype_of(w.scalar_type(), ok);
    d.flags = exact_env() ? TVK_GEMM_EXACT : 0;
    d.spatial_dims = (int32_t)in_sp.size();
    d.n = n;
    d.c_in = c_in;
    d.c_out = w.size(0);
    d.groups = groups;
    for (size_t i = 0; i < in_sp.size(); ++i) {
        d.in_size[i] = in_sp[i];
        d.kernel[i] = w.size(2 + i);
        d.stride[i] = stride[i];
        d.padding[i] = padding[i];
        d.dilation[i] = dilation[i];
        d.out_size[i] = out_sp[i];
    }
    d.stream = stream_of(w);
    return d;
}

at::Tensor conv_forward_impl(const at::Tensor& x, const at::Tensor& w, const at::Tensor& b, const std::vector<int64_t>& s,
                             const std::vector<int64_t>& p, const std::vector<int64_t>& dl, int64_t groups) {
    const auto in_sp = x.sizes().slice(2);
    const std::vector<int64_t> o = out_sizes(in_sp, w.sizes().slice(2), s, p, dl);
    at::Tensor y = at::empty(cat_shape(x.size(0), w.size(0), o), x.options());
    tvk_convnd_desc d = make_desc(x.size(0), x.size(1), in_sp, w, groups, s, p, dl, o);
    d.x = x.data_ptr();
    d.weight = w.data_ptr();
    d.bias = b.defined() ? b.data_ptr() : nullptr;
    d.y = y.data_ptr();
    check_status(run_conv_mode(d, TVK_CONV_FWD), "tvk_conv_fwd");
    return y;
}

// input gradient of a forward conv: dy [n, c_out, out...] -> dx [n, c_in, in_sp...]
at::Tensor conv_dgrad_impl(const at::Tensor& dy, const at::Tensor& w, int64_t c_in, c10::IntArrayRef in_sp,
                           const std::vector<int64_t>& s, const std::vector<int64_t>& p, const std::vector<int64_t>& dl,
                           int64_t groups) {
    at::Tensor dx = at::empty(cat_shape(dy.size(0), c_in, in_sp), dy.options());
    tvk_convnd_desc d = make_desc(dy.size(0), c_in, in_sp, w, groups, s, p, dl, dy.sizes().slice(2));
    d.x = dx.data_ptr();
    d.weight = w.data_ptr();
    d.y = dy.data_ptr();
    check_status(run_conv_mode(d, TVK_CONV_DGRAD), "tvk_conv_dgrad");
    return dx;
}

at::Tensor conv_wgrad_impl(const at::Tensor& x, const at::Tensor& dy, c10::IntArrayRef w_sizes, const std::vector<int64_t>& s,
                           const std::vector<int64_t>& p, const std::vector<int64_t>& dl, int64_t groups) {
    at::Tensor dw = at::empty(w_sizes, x.options());
    tvk_convnd_desc d = make_desc(x.size(0), x.size(1), x.sizes().slice(2), dw, groups, s, p, dl, dy.sizes().slice(2));
    d.x = x.data_ptr();
    d.weight = dw.data_ptr();
    d.y = dy.data_ptr();
    check_status(run_conv_mode(d, TVK_CONV_WGRAD), "tvk_conv_wgrad");
    return dw;
}

// ---------------------------------------------------------------------------
// float64 and integer convolutions: no implicit-GEMM kernel takes them. The
// reference runs them through im2col + matmul (conv.cpp:32-58,200-216); here
// the columns come from a strided window view of the zero-padded input copied
// by the device copy kernel, and the products from tvk_gemm's float64 /
// integer kernel, so the whole convolution stays on the device.
// ---------------------------------------------------------------------------

bool unfold_dtype(at::ScalarType t) {
    return t == at::kDouble || t == at::kLong || t == at::kInt || t == at::kShort || t == at::kChar || t == at::kByte;
}

// [n, c, spatial...] -> columns [n, c * prod(k), prod(out)], rows in (c, k...) order
at::Tensor im2col_nd(const at::Tensor& x, c10::IntArrayRef k, c10::IntArrayRef dl, c10::IntArrayRef p, c10::IntArrayRef s,
                     c10::IntArrayRef out) {
    const int64_t nd = (int64_t)k.size(), n = x.size(0), c = x.size(1);
    std::vector<int64_t> padded_sp;
    bool any_pad = false;
    for (int64_t i = 0; i < nd; ++i) {
        padded_sp.push_back(x.size(2 + i) + 2 * p[i]);
        any_pad |= p[i] != 0;
    }
    at::Tensor padded;
    if (!any_pad) {
        padded = x.contiguous();
    } else {
        padded = at::zeros(cat_shape(n, c, padded_sp), x.options());
        at::Tensor inner = padded;
        for (int64_t i = 0; i < nd; ++i) inner = inner.narrow(2 + i, p[i], x.size(2 + i));
        inner.copy_(x);
    }
    // element strides of the padded image's spatial dimensions
    std::vector<int64_t> sp_stride(nd, 1);
    for (int64_t i = nd - 2; i >= 0; --i) sp_stride[i] = sp_stride[i + 1] * padded_sp[i + 1];
    const int64_t plane = sp_stride[0] * padded_sp[0];
    std::vector<int64_t> shape{n, c}, stride{c * plane, plane};
    int64_t taps = 1, len = 1;
    for (int64_t i = 0; i < nd; ++i) { shape.push_back(k[i]); stride.push_back(dl[i] * sp_stride[i]); taps *= k[i]; }
    for (int64_t i = 0; i < nd; ++i) { shape.push_back(out[i]); stride.push_back(s[i] * sp_stride[i]); len *= out[i]; }
    at::Tensor cols = at::empty({n, c * taps, len}, x.options());
    if (cols.numel() != 0) cols.view(shape).copy_(padded.as_strided(shape, stride));
    return cols;
}

// columns [n, c * prod(k), prod(cols_out)] -> image [n, c, out_sp...]: each
// tap's column block is added into the matching strided view of a zeroed
// padded image (a tap's view holds every image element at most once, so each
// add is one pass without write collisions), taps in order; then the padding
// is cropped
at::Tensor col2im_nd(const at::Tensor& cols_in, c10::IntArrayRef out_sp, c10::IntArrayRef k, c10::IntArrayRef dl,
                     c10::IntArrayRef p, c10::IntArrayRef s, c10::IntArrayRef blocks) {
    const int64_t nd = (int64_t)k.size(), n = cols_in.size(0);
    int64_t taps = 1;
    for (int64_t i = 0; i < nd; ++i) taps *= k[i];
    const int64_t c = cols_in.size(1) / taps;
    std::vector<int64_t> padded_sp;
    bool any_pad = false;
    for (int64_t i = 0; i < nd; ++i) {
        padded_sp.push_back(out_sp[i] + 2 * p[i]);
        any_pad |= p[i] != 0;
    }
    std::vector<int64_t> sp_stride(nd, 1);
    for (int64_t i = nd - 2; i >= 0; --i) sp_stride[i] = sp_stride[i + 1] * padded_sp[i + 1];
    const int64_t plane = sp_stride[0] * padded_sp[0];
    at::Tensor image = at::zeros(cat_shape(n, c, padded_sp), cols_in.options());
    if (n != 0) {
        std::vector<int64_t> tshape{n, c, taps};
        tshape.insert(tshape.end(), blocks.begin(), blocks.end());
        const at::Tensor tapcols = cols_in.contiguous().view(tshape);
        std::vector<int64_t> vshape{n, c}, vstride{c * plane, plane};
        for (int64_t i = 0; i < nd; ++i) { vshape.push_back(blocks[i]); vstride.push_back(s[i] * sp_stride[i]); }
        for (int64_t t = 0; t < taps; ++t) {
            int64_t rem = t, off = 0;
            for (int64_t i = nd - 1; i >= 0; --i) {
                off += (rem % k[i]) * dl[i] * sp_stride[i];
                rem /= k[i];
            }
            at::Tensor dst = image.as_strided(vshape, vstride, off);
            dst.add_(tapcols.select(2, t));
        }
    }
    if (any_pad) {
        for (int64_t i = 0; i < nd; ++i) image = image.narrow(2 + i, p[i], out_sp[i]);
        image = image.contiguous();
    }
    return image;
}

// y[n, g*co + o, ...] = sum over (c, taps) of the group's weights x columns
at::Tensor unfold_forward(const at::Tensor& x, const at::Tensor& w, const at::Tensor& b, const std::vector<int64_t>& s,
                          const std::vector<int64_t>& p, const std::vector<int64_t>& dl, int64_t groups) {
    const int64_t n = x.size(0), cout = w.size(0), kk = w.numel() / std::max<int64_t>(1, cout);
    const std::vector<int64_t> o = out_sizes(x.sizes().slice(2), w.sizes().slice(2), s, p, dl);
    int64_t len = 1;
    for (int64_t v : o) len *= v;
    const at::Tensor cols = im2col_nd(x, w.sizes().slice(2), dl, p, s, o);                  // [n, c*taps, len]
    at::Tensor y = at::matmul(w.reshape({groups, cout / groups, kk}), cols.view({n, groups, kk, len}));
    y = y.reshape(cat_shape(n, cout, o));
    if (b.defined()) {
        std::vector<int64_t> bshape(y.dim(), 1);
        bshape[1] = cout;
        y = y + b.view(bshape);
    }
    return y;
}

// the transposed convolution of x (the input gradient of a forward one):
// columns = w^T x per group, folded back by col2im
at::Tensor unfold_transposed(const at::Tensor& x, const at::Tensor& w, c10::IntArrayRef out_sp, const std::vector<int64_t>& s,
                             const std::vector<int64_t>& p, const std::vector<int64_t>& dl, int64_t groups) {
    const int64_t n = x.size(0), cin_g = x.size(1) / groups, cout = w.size(1) * groups;
    int64_t kk = 1, l = 1;
    for (int64_t i = 2; i < w.dim(); ++i) kk *= w.size(i);
    for (int64_t i = 2; i < x.dim(); ++i) l *= x.size(i);
    const at::Tensor wg = w.reshape({groups, cin_g, (cout / groups) * kk}).transpose(1, 2);      // [g, co*kk, ci]
    const at::Tensor cols = at::matmul(wg, x.reshape({n, groups, cin_g, l})).reshape({n, cout * kk, l});
    return col2im_nd(cols, out_sp, w.sizes().slice(2), dl, p, s, x.sizes().slice(2));
}

std::vector<int64_t> bias_grad_dims(int64_t dim) {
    std::vector<int64_t> d{0};
    for (int64_t i = 2; i < dim; ++i) d.push_back(i);
    return d;
}

at::Tensor convolution(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                       c10::SymIntArrayRef stride_, c10::SymIntArrayRef padding_, c10::SymIntArrayRef dilation_,
                       bool transposed, c10::SymIntArrayRef output_padding_, c10::SymInt groups_) {
    const int64_t groups = groups_.guard_int(__FILE__, __LINE__);
    const size_t nd = (size_t)std::max<int64_t>(1, weight.dim() - 2);
    auto s = expand_nd(ints(stride_), nd), p = expand_nd(ints(padding_), nd), dl = expand_nd(ints(dilation_), nd),
         op = expand_nd(ints(output_padding_), nd);
    const at::MemoryFormat format = conv_memory_format(input, weight);
    if (unfold_dtype(weight.scalar_type()) && input.scalar_type() == weight.scalar_type() && geometry_ok(input, weight, s)) {
        const at::Tensor x = input.contiguous(), w = weight.contiguous();
        const at::Tensor b = bias.has_value() && bias->defined() ? bias->to(w.scalar_type()) : at::Tensor();
        at::Tensor y;
        if (!transposed) {
            y = unfold_forward(x, w, b, s, p, dl, groups);
        } else {
            const std::vector<int64_t> o = transposed_sizes(x.sizes().slice(2), w.sizes().slice(2), s, p, dl, op);
            y = unfold_transposed(x, w, o, s, p, dl, groups);
            if (b.defined()) {
                std::vector<int64_t> bshape(y.dim(), 1);
                bshape[1] = -1;
                y = y + b.view(bshape);
            }
        }
        return y.contiguous(format);
    }
    if (!supported(input, weight, s)) {
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
        // transposed: w is [c_in, c_out/g, kernel...]; the output is the input
        // gradient of the forward conv whose output x is
        const std::vector<int64_t> o = transposed_sizes(x.sizes().slice(2), w.sizes().slice(2), s, p, dl, op);
        y = conv_dgrad_impl(x, w, w.size(1) * groups, o, s, p, dl, groups);
        if (b.defined()) {
            std::vector<int64_t> bshape(y.dim(), 1);
            bshape[1] = -1;
            y = y + b.view(bshape);
        }
    }
    return y.contiguous(format);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> convolution_backward(
    const at::Tensor& grad_output, const at::Tensor& input, const at::Tensor& weight, c10::SymIntArrayRef stride_,
    c10::SymIntArrayRef padding_, c10::SymIntArrayRef dilation_, bool transposed, c10::SymIntArrayRef output_padding_,
    c10::SymInt groups_, std::array<bool, 3> mask) {
    const int64_t groups = groups_.guard_int(__FILE__, __LINE__);
    const size_t nd = (size_t)std::max<int64_t>(1, weight.dim() - 2);
    auto s = expand_nd(ints(stride_), nd), p = expand_nd(ints(padding_), nd), dl = expand_nd(ints(dilation_), nd),
         op = expand_nd(ints(output_padding_), nd);
    const at::MemoryFormat format = conv_memory_format(input, weight);
    at::Tensor gi, gw, gb;
    if (weight.scalar_type() == at::kDouble && input.scalar_type() == at::kDouble && grad_output.scalar_type() == at::kDouble &&
        geometry_ok(input, weight, s) && !transposed) {
        // float64 (the only unfold dtype with gradients): the input gradient is
        // the transposed convolution of dy, the weight gradient dy times the
        // columns summed over the batch
        const at::Tensor go = grad_output.contiguous(), in = input.contiguous(), w = weight.contiguous();
        if (mask[0]) gi = unfold_transposed(go, w, in.sizes().slice(2), s, p, dl, groups).contiguous(format);
        if (mask[1]) {
            const int64_t n = in.size(0), cout = w.size(0), kk = w.numel() / std::max<int64_t>(1, cout);
            int64_t l = 1;
            for (int64_t i = 2; i < go.dim(); ++i) l *= go.size(i);
            const at::Tensor cols = im2col_nd(in, w.sizes().slice(2), dl, p, s, go.sizes().slice(2));
            gw = at::matmul(go.reshape({n, groups, cout / groups, l}), cols.view({n, groups, kk, l}).transpose(-1, -2))
                     .sum(0)
                     .reshape(w.sizes())
                     .contiguous(format);
        }
        if (mask[2]) gb = at::sum(grad_output, bias_grad_dims(grad_output.dim()));
        return {gi, gw, gb};
    }
    if (!supported(input, weight, s) || grad_output.scalar_type() != weight.scalar_type() ||
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
        if (mask[0]) gi = conv_dgrad_impl(go, w, in.size(1), in.sizes().slice(2), s, p, dl, groups);
        if (mask[1]) gw = conv_wgrad_impl(in, go, w.sizes(), s, p, dl, groups);
    } else {
        // forward conv with input go and output `in`
        if (mask[0]) gi = conv_forward_impl(go, w, at::Tensor(), s, p, dl, groups);
        if (mask[1]) gw = conv_wgrad_impl(go, in, w.sizes(), s, p, dl, groups);
    }
    if (mask[2]) gb = at::sum(grad_output, bias_grad_dims(grad_output.dim()));
    if (gi.defined()) gi = gi.contiguous(format);
    if (gw.defined()) gw = gw.contiguous(format);
    return {gi, gw, gb};
}

// The legacy convolution entry points (slow_conv_transpose2d/3d,
// slow_conv_dilated2d/3d, _slow_conv2d_forward, slow_conv3d_forward,
// _conv_depthwise2d, conv_depthwise3d, and their .out forms) carry an explicit
// kernel_size and some omit dilation, output padding or groups. Each is one
// convolution() call with the omitted parameters at their neutral values;
// depthwise means one group per input channel. The reference registers the
// same set onto its convolution (src/api/ops/conv.cpp:1305-1320).
struct LegacyConv {
    bool transposed = false;
    bool depthwise = false;
};

at::Tensor legacy_conv(const LegacyConv& kind, const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                       const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                       c10::SymIntArrayRef dilation, c10::SymIntArrayRef output_padding) {
    const std::vector<int64_t> ks = ints(kernel_size);
    const std::vector<int64_t> wk(weight.sizes().begin() + std::min<int64_t>(2, weight.dim()), weight.sizes().end());
    TORCH_CHECK(ks == wk, "kernel_size ", c10::IntArrayRef(ks), " must match weight spatial dimensions ", c10::IntArrayRef(wk));
    const size_t nd = ks.size();
    std::vector<c10::SymInt> ones(nd, c10::SymInt(1)), zeros(nd, c10::SymInt(0));
    const int64_t groups = kind.depthwise ? self.size(1) : 1;
    return convolution(self, weight, bias, stride, padding, dilation.empty() ? c10::SymIntArrayRef(ones) : dilation,
                       kind.transposed, output_padding.empty() ? c10::SymIntArrayRef(zeros) : output_padding, c10::SymInt(groups));
}

at::Tensor& legacy_out(at::Tensor& out, const at::Tensor& res) {
    at::native::resize_output(out, res.sizes());
    out.copy_(res);
    return out;
}

// im2col / col2im (the unfold and fold ops; the reference's versions are
// src/api/ops/conv.cpp:115-185), with torch's CPU checks and messages. Both
// run on the device with the copy, fill and add kernels: im2col zero-pads the
// image once and copies the strided window view [n, c, kh, kw, oh, ow] of the
// padded image into the dense column tensor; col2im adds each tap's column
// block into the matching strided view of a zeroed padded image (a tap's view
// holds every output pixel at most once, so each add is one pass with no
// write collisions) in tap order, then crops the padding.
void unfold_param_checks(at::IntArrayRef k, at::IntArrayRef d, at::IntArrayRef p, at::IntArrayRef s) {
    TORCH_CHECK(k.size() == 2, "It is expected kernel_size equals to 2, but got size ", k.size());
    TORCH_CHECK(d.size() == 2, "It is expected dilation equals to 2, but got size ", d.size());
    TORCH_CHECK(p.size() == 2, "It is expected padding equals to 2, but got size ", p.size());
    TORCH_CHECK(s.size() == 2, "It is expected stride equals to 2, but got size ", s.size());
    TORCH_CHECK(k[0] > 0 && k[1] > 0, "kernel size should be greater than zero, but got kernel_height: ", k[0],
                " kernel_width: ", k[1]);
    TORCH_CHECK(s[0] > 0 && s[1] > 0, "stride should be greater than zero, but got stride_height: ", s[0],
                " stride_width: ", s[1]);
    TORCH_CHECK(d[0] > 0 && d[1] > 0, "dilation should be greater than zero, but got dilation_height: ", d[0],
                " dilation_width: ", d[1]);
    TORCH_CHECK(p[0] >= 0 && p[1] >= 0, "padding should be non-negative, but got pad_height: ", p[0], " pad_width: ", p[1]);
}

int64_t sliding_blocks(int64_t size, int64_t k, int64_t d, int64_t p, int64_t s) {
    const int64_t span = size + 2 * p - d * (k - 1) - 1;
    return (span < 0 ? -((-span + s - 1) / s) : span / s) + 1;   // floor division, as torch's div_rtn
}

at::Tensor im2col_vk(const at::Tensor& self, at::IntArrayRef k, at::IntArrayRef d, at::IntArrayRef p, at::IntArrayRef s) {
    unfold_param_checks(k, d, p, s);
    const int64_t nd = self.dim();
    const bool valid = (nd == 3 && self.numel() != 0) || (nd == 4 && self.size(1) != 0 && self.size(2) != 0 && self.size(3) != 0);
    TORCH_CHECK(valid, "Expected 3D or 4D (batch mode) tensor with possibly 0 batch size and other non-zero dimensions for input, but got: ",
                self.sizes());
    const at::Tensor x = nd == 4 ? self : self.unsqueeze(0);
    const int64_t h = x.size(2), w = x.size(3);
    const int64_t oh = sliding_blocks(h, k[0], d[0], p[0], s[0]), ow = sliding_blocks(w, k[1], d[1], p[1], s[1]);
    // (the CPU's message repeats the input height)
    TORCH_CHECK(oh >= 1 && ow >= 1, "Given input with spatial size (", h, ", ", h, "), kernel_size=(", k[0], ", ", k[1],
                "), dilation=(", d[0], ", ", d[1], "), padding=(", p[0], ", ", p[1],
                "), calculated shape of the array of sliding blocks as (", oh, ", ", ow,
                "), but its components must be at least one.");
    const at::Tensor cols = im2col_nd(x, k, d, p, s, {oh, ow});
    return nd == 4 ? cols : cols.squeeze(0);
}

at::Tensor col2im_vk(const at::Tensor& self, c10::SymIntArrayRef output_size, at::IntArrayRef k, at::IntArrayRef d,
                     at::IntArrayRef p, at::IntArrayRef s) {
    const std::vector<int64_t> os = ints(output_size);
    TORCH_CHECK(os.size() == 2, "It is expected output_size equals to 2, but got size ", os.size());
    unfold_param_checks(k, d, p, s);
    const int64_t nd = self.dim();
    TORCH_CHECK((nd == 2 && self.size(0) != 0 && self.size(1) != 0) || (nd == 3 && self.size(1) != 0 && self.size(2) != 0),
                "Expected 2D or 3D (batch mode) tensor for input with possibly 0 batch size and non-zero dimensions for input, but got: ",
                self.sizes());
    const at::Tensor cols = nd == 3 ? self : self.unsqueeze(0);
    const int64_t planes = cols.size(1), length = cols.size(2);
    TORCH_CHECK(planes % (k[0] * k[1]) == 0,
                "Expected size of input's dimension 1 to be divisible by the product of kernel_size, but got input.size(1)=",
                planes, " and kernel_size=(", k[0], ", ", k[1], ").");
    const int64_t oh = sliding_blocks(os[0], k[0], d[0], p[0], s[0]), ow = sliding_blocks(os[1], k[1], d[1], p[1], s[1]);
    TORCH_CHECK(length == oh * ow, "Given output_size=(", os[0], ", ", os[1], "), kernel_size=(", k[0], ", ", k[1],
                "), dilation=(", d[0], ", ", d[1], "), padding=(", p[0], ", ", p[1], "), stride=(", s[0], ", ", s[1],
                "), expected size of input's dimension 2 to match the calculated number of sliding blocks ", oh, " * ", ow,
                " = ", oh * ow, ", but got input.size(2)=", length, ".");
    TORCH_CHECK(oh >= 1 && ow >= 1, "Given output_size=(", os[0], ", ", os[1], "), kernel_size=(", k[0], ", ", k[1],
                "), dilation=(", d[0], ", ", d[1], "), padding=(", p[0], ", ", p[1], "), stride=(", s[0], ", ", s[1],
                "), calculated shape of the array of sliding blocks as (", oh, ", ", ow, "), which is too small (non-positive)");
    TORCH_CHECK(os[0] >= 1 && os[1] >= 1, "Expected output spatial size to be positive, but got: output_size=(", os[0], ", ",
                os[1], ").");
    const at::Tensor image = col2im_nd(cols, os, k, d, p, s, {oh, ow});
    return nd == 3 ? image : image.squeeze(0);
}

at::Tensor& im2col_out_vk(const at::Tensor& self, at::IntArrayRef k, at::IntArrayRef d, at::IntArrayRef p, at::IntArrayRef s,
                          at::Tensor& out) {
    return legacy_out(out, im2col_vk(self, k, d, p, s));
}

at::Tensor& col2im_out_vk(const at::Tensor& self, c10::SymIntArrayRef output_size, at::IntArrayRef k, at::IntArrayRef d,
                          at::IntArrayRef p, at::IntArrayRef s, at::Tensor& out) {
    return legacy_out(out, col2im_vk(self, output_size, k, d, p, s));
}

at::Tensor slow_conv_transpose(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                               const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                               c10::SymIntArrayRef output_padding, c10::SymIntArrayRef dilation) {
    return legacy_conv({true, false}, self, weight, kernel_size, bias, stride, padding, dilation, output_padding);
}
at::Tensor& slow_conv_transpose_out(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                                    const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                                    c10::SymIntArrayRef output_padding, c10::SymIntArrayRef dilation, at::Tensor& out) {
    return legacy_out(out, slow_conv_transpose(self, weight, kernel_size, bias, stride, padding, output_padding, dilation));
}
at::Tensor slow_conv_dilated(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                             const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                             c10::SymIntArrayRef dilation) {
    return legacy_conv({false, false}, self, weight, kernel_size, bias, stride, padding, dilation, {});
}
at::Tensor& slow_conv_dilated_out(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                                  const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                                  c10::SymIntArrayRef dilation, at::Tensor& out) {
    return legacy_out(out, slow_conv_dilated(self, weight, kernel_size, bias, stride, padding, dilation));
}
at::Tensor slow_conv_forward(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                             const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding) {
    return legacy_conv({false, false}, self, weight, kernel_size, bias, stride, padding, {}, {});
}
at::Tensor& slow_conv_forward_out(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                                  const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                                  at::Tensor& out) {
    return legacy_out(out, slow_conv_forward(self, weight, kernel_size, bias, stride, padding));
}
at::Tensor conv_depthwise(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                          const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                          c10::SymIntArrayRef dilation) {
    return legacy_conv({false, true}, self, weight, kernel_size, bias, stride, padding, dilation, {});
}
at::Tensor& conv_depthwise_out(const at::Tensor& self, const at::Tensor& weight, c10::SymIntArrayRef kernel_size,
                               const std::optional<at::Tensor>& bias, c10::SymIntArrayRef stride, c10::SymIntArrayRef padding,
                               c10::SymIntArrayRef dilation, at::Tensor& out) {
    return legacy_out(out, conv_depthwise(self, weight, kernel_size, bias, stride, padding, dilation));
}

}  // namespace
}  // namespace tvkb

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
    m.impl("convolution_overrideable", &tvkb::convolution);
    m.impl("convolution_backward_overrideable", &tvkb::convolution_backward);
    m.impl("im2col", &tvkb::im2col_vk);
    m.impl("im2col.out", &tvkb::im2col_out_vk);
    m.impl("col2im", &tvkb::col2im_vk);
    m.impl("col2im.out", &tvkb::col2im_out_vk);
    for (const char* name : {"slow_conv_transpose2d", "slow_conv_transpose3d"}) m.impl(name, &tvkb::slow_conv_transpose);
    for (const char* name : {"slow_conv_transpose2d.out", "slow_conv_transpose3d.out"}) m.impl(name, &tvkb::slow_conv_transpose_out);
    for (const char* name : {"slow_conv_dilated2d", "slow_conv_dilated3d"}) m.impl(name, &tvkb::slow_conv_dilated);
    for (const char* name : {"slow_conv_dilated2d.out", "slow_conv_dilated3d.out"}) m.impl(name, &tvkb::slow_conv_dilated_out);
    for (const char* name : {"_slow_conv2d_forward", "slow_conv3d_forward"}) m.impl(name, &tvkb::slow_conv_forward);
    for (const char* name : {"_slow_conv2d_forward.output", "slow_conv3d_forward.output"}) m.impl(name, &tvkb::slow_conv_forward_out);
    for (const char* name : {"_conv_depthwise2d", "conv_depthwise3d"}) m.impl(name, &tvkb::conv_depthwise);
    for (const char* name : {"_conv_depthwise2d.out", "conv_depthwise3d.out"}) m.impl(name, &tvkb::conv_depthwise_out);
}
