// Scaled dot-product attention on the vulkan device: the overrideable SDPA
// backend the reference registers (src/api/ops/attention.cpp:667-761).
// Every case runs on the device through tvk_attention_fwd / tvk_attention_bwd:
// the MFMA kernels for float16/bfloat16 with head dims 64/128, the library's
// general kernels for float32, other head dims, any strides, and the score
// gradient that gives the bias gradient (summed here over the bias's
// broadcast dimensions with the device sum).
#include "common.h"

#include <ATen/Context.h>
#include <ATen/SDPBackend.h>
#include <ATen/native/DispatchStub.h>
#include <ATen/native/transformers/attention.h>

#include <cmath>
#include <cstring>

namespace tvkb {
namespace {

// Sizes of one attention call and its operands in [batch, heads, rows, dim]
// form (key/value heads may be fewer: grouped-query attention).
struct Sdpa {
    at::Tensor q, k, v, bias;
    int64_t batch = 0, heads = 0, kv_heads = 0, len_q = 0, len_kv = 0, dim = 0, dim_v = 0;
    bool causal = false;
    double scale = 1.0;
};

// The operands' shape rules and messages are the reference's prepare_attention
// (src/api/ops/attention.cpp:44-82); the scale defaults to 1/sqrt(head dim).
Sdpa describe(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& bias, bool causal,
              std::optional<double> scale) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4,
                "torchvulkan [ERROR]: fused attention takes 4D query, key and value, got ", q.sizes(), ", ", k.sizes(),
                " and ", v.sizes(), ".");
    Sdpa s;
    s.batch = q.size(0);
    s.heads = q.size(1);
    s.len_q = q.size(2);
    s.dim = q.size(3);
    s.kv_heads = k.size(1);
    s.len_kv = k.size(2);
    s.dim_v = v.size(3);
    const bool match = k.size(0) == s.batch && v.size(0) == s.batch && v.size(1) == s.kv_heads && v.size(2) == s.len_kv &&
                       k.size(3) == s.dim;
    TORCH_CHECK(match, "torchvulkan [ERROR]: attention shapes don't match: query ", q.sizes(), ", key ", k.sizes(),
                ", value ", v.sizes(), ".");
    TORCH_CHECK(s.kv_heads > 0 && s.heads % s.kv_heads == 0, "torchvulkan [ERROR]: the number of query heads (", s.heads,
                ") must be a multiple of the key/value heads (", s.kv_heads, ").");
    s.q = q;
    s.k = k;
    s.v = v;
    if (bias.defined()) s.bias = bias.scalar_type() == q.scalar_type() ? bias : bias.to(q.scalar_type());
    s.causal = causal;
    s.scale = scale.has_value() ? *scale : 1.0 / std::sqrt((double)s.dim);
    return s;
}

bool device_dtype(at::ScalarType dt) { return dt == at::kFloat || dt == at::kHalf || dt == at::kBFloat16; }

// Shapes the library's kernels take (its general kernels: head dims up to 512,
// batch and heads up to 65535).
bool library_takes(at::ScalarType dt, int64_t dim, int64_t dim_v, int64_t batch, int64_t heads) {
    return device_dtype(dt) && dim >= 1 && dim <= 512 && dim_v >= 1 && dim_v <= 512 && batch <= 65535 && heads <= 65535;
}

// The MFMA kernels want unit stride along the head dim and 16-byte rows: for
// their shapes an operand without that layout is worth one dense copy.
at::Tensor mfma_layout(const at::Tensor& t, const Sdpa& s) {
    const bool mfma = (t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16) && s.dim == s.dim_v &&
                      (s.dim == 64 || s.dim == 128);
    if (!mfma) return t;
    bool ok = t.stride(3) == 1 && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
    for (int i = 0; i < 3; ++i) ok = ok && (t.size(i) <= 1 || t.stride(i) % 8 == 0);
    return ok ? t : t.contiguous();
}

// The output is laid out [batch, len_q, heads, dim_v] underneath when the
// query is (the projection's layout), so merging heads afterwards is a view;
// the reference picks its output the same way (attention.cpp:413-418).
at::Tensor new_output(const Sdpa& s) {
    if (s.q.stride(1) < s.q.stride(2))
        return at::empty({s.batch, s.len_q, s.heads, s.dim_v}, s.q.options()).transpose(1, 2);
    return at::empty({s.batch, s.heads, s.len_q, s.dim_v}, s.q.options());
}

void strides4(const at::Tensor& t, int64_t* out) {
    for (int i = 0; i < 4; ++i) out[i] = t.stride(i);
}

tvk_attention_desc forward_desc(const Sdpa& s, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                const at::Tensor& out, const at::Tensor& lse) {
    tvk_attention_desc d;
    std::memset(&d, 0, sizeof(d));
    bool ok = false;
    d.dtype = tvk_dtype_of(q.scalar_type(), ok);
    d.causal = s.causal ? 1 : 0;
    d.batch = s.batch;
    d.heads_q = s.heads;
    d.heads_kv = s.kv_heads;
    d.len_q = s.len_q;
    d.len_kv = s.len_kv;
    d.head_dim = s.dim;
    d.head_dim_v = s.dim_v;
    d.q = q.data_ptr();
    d.k = k.data_ptr();
    d.v = v.data_ptr();
    strides4(q, d.q_stride);
    strides4(k, d.k_stride);
    strides4(v, d.v_stride);
    if (s.bias.defined()) {
        const at::Tensor b = s.bias.expand({s.batch, s.heads, s.len_q, s.len_kv});
        d.bias = b.data_ptr();
        strides4(b, d.bias_stride);
    }
    d.out = out.data_ptr();
    strides4(out, d.out_stride);
    d.lse = lse.data_ptr<float>();
    for (int i = 0; i < 3; ++i) d.lse_stride[i] = lse.stride(i);
    d.scale = s.scale;
    d.stream = stream_of(q);
    return d;
}

int64_t sdp_choice(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                   const std::optional<at::Tensor>& attn_mask, double dropout_p, bool /*is_causal*/,
                   std::optional<double> /*scale*/, bool enable_gqa) {
    const int64_t math = static_cast<int64_t>(at::SDPBackend::math);
    if (!at::globalContext().userEnabledOverrideableSDP() || dropout_p > 0.0) return math;
    if (query.is_nested() || key.is_nested() || value.is_nested()) return math;
    if (query.dim() != 4 || key.dim() != 4 || value.dim() != 4) return math;
    const at::ScalarType dt = query.scalar_type();
    if (key.scalar_type() != dt || value.scalar_type() != dt) return math;
    if (attn_mask.has_value() && attn_mask->defined() && attn_mask->scalar_type() != at::kBool &&
        attn_mask->scalar_type() != dt)
        return math;
    const int64_t heads = query.size(1), kv_heads = key.size(1);
    if (key.size(0) != query.size(0) || value.size(0) != query.size(0) || value.size(1) != kv_heads) return math;
    if (key.size(2) != value.size(2) || key.size(3) != query.size(3)) return math;
    if (heads != kv_heads && !(enable_gqa && kv_heads > 0 && heads % kv_heads == 0)) return math;
    if (!library_takes(dt, query.size(3), value.size(3), query.size(0), heads)) return math;
    return static_cast<int64_t>(at::SDPBackend::overrideable);
}

void require_library(const Sdpa& s) {
    TORCH_CHECK(library_takes(s.q.scalar_type(), s.dim, s.dim_v, s.batch, s.heads),
                "torchvulkan [ERROR]: fused attention runs float32, float16 and bfloat16 with head dims from 1 to 512 and "
                "batch and heads up to 65535; got ",
                s.q.scalar_type(), " with head dims ", s.dim, "/", s.dim_v, ". scaled_dot_product_attention routes "
                "other cases to its math backend.");
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor, at::Tensor, at::Tensor>
sdpa_forward(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
             const std::optional<at::Tensor>& attn_bias, double dropout_p, bool is_causal, bool /*return_debug_mask*/,
             std::optional<double> scale) {
    TORCH_CHECK(dropout_p == 0.0, "torchvulkan [ERROR]: fused attention doesn't support dropout; it runs on the math backend.");
    Sdpa s = describe(query, key, value, attn_bias.has_value() ? *attn_bias : at::Tensor(), is_causal, scale);
    at::Tensor out = new_output(s);
    at::Tensor lse = at::empty({s.batch, s.heads, s.len_q}, s.q.options().dtype(at::kFloat));
    if (s.batch * s.heads * s.len_q > 0) {
        require_library(s);
        const at::Tensor q = mfma_layout(s.q, s), k = mfma_layout(s.k, s), v = mfma_layout(s.v, s);
        tvk_attention_desc d = forward_desc(s, q, k, v, out, lse);
        check_status(tvk_attention_fwd(&d), "tvk_attention_fwd");
    }
    at::Tensor philox = at::empty({}, at::TensorOptions().dtype(at::kLong));
    return {out, lse, at::Tensor(), at::Tensor(), c10::SymInt(s.len_q), c10::SymInt(s.len_kv), philox, philox.clone(),
            at::empty({0}, query.options())};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> sdpa_backward(
    const at::Tensor& grad_out, const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
    const at::Tensor& attn_bias, std::array<bool, 4> grad_input_mask, const at::Tensor& out, const at::Tensor& logsumexp,
    const at::Tensor& /*cum_seq_q*/, const at::Tensor& /*cum_seq_k*/, int64_t /*max_q*/, int64_t /*max_k*/,
    double dropout_p, bool is_causal, const at::Tensor& /*philox_seed*/, const at::Tensor& /*philox_offset*/,
    std::optional<double> scale) {
    TORCH_CHECK(dropout_p == 0.0, "torchvulkan [ERROR]: fused attention doesn't support dropout; it runs on the math backend.");
    Sdpa s = describe(query, key, value, attn_bias, is_causal, scale);
    if (!grad_input_mask[0] && !grad_input_mask[1] && !grad_input_mask[2] && !grad_input_mask[3]) return {};
    const at::ScalarType dt = s.q.scalar_type();
    at::Tensor gq = at::empty({s.batch, s.heads, s.len_q, s.dim}, s.q.options());
    at::Tensor gk = at::empty({s.batch, s.kv_heads, s.len_kv, s.dim}, s.q.options());
    at::Tensor gv = at::empty({s.batch, s.kv_heads, s.len_kv, s.dim_v}, s.q.options());
    const bool want_bias = grad_input_mask[3] && attn_bias.defined();
    at::Tensor dscores;
    if (want_bias) dscores = at::empty({s.batch, s.heads, s.len_q, s.len_kv}, s.q.options().dtype(at::kFloat));
    if (s.batch * s.heads * (s.len_q + s.len_kv) > 0) {
        require_library(s);
        const at::Tensor q = mfma_layout(s.q, s), k = mfma_layout(s.k, s), v = mfma_layout(s.v, s);
        const at::Tensor dout = mfma_layout(grad_out.scalar_type() == dt ? grad_out : grad_out.to(dt), s);
        const at::Tensor o = out.scalar_type() == dt ? out : out.to(dt);
        const at::Tensor lse = logsumexp.scalar_type() == at::kFloat ? logsumexp : logsumexp.to(at::kFloat);
        tvk_attention_bwd_desc bd;
        std::memset(&bd, 0, sizeof(bd));
        bd.fwd = forward_desc(s, q, k, v, o, lse);
        bd.dout = dout.data_ptr();
        strides4(dout, bd.dout_stride);
        bd.dq = gq.data_ptr();
        strides4(gq, bd.dq_stride);
        bd.dk = gk.data_ptr();
        strides4(gk, bd.dk_stride);
        bd.dv = gv.data_ptr();
        strides4(gv, bd.dv_stride);
        if (want_bias) {
            bd.dscores = dscores.data_ptr<float>();
            strides4(dscores, bd.dscores_stride);
        }
        check_status(tvk_attention_bwd(&bd), "tvk_attention_bwd");
    } else if (want_bias) {
        dscores.zero_();
    }
    at::Tensor gbias;
    if (want_bias) gbias = at::sum_to(dscores, s.bias.sizes()).to(attn_bias.scalar_type());
    return {gq, gk, gv, gbias};
}

}  // namespace
}  // namespace tvkb

// scaled_dot_product_attention asks this stub which backend to run
namespace at::native {
REGISTER_PRIVATEUSE1_DISPATCH(_fused_sdp_choice_stub, &tvkb::sdp_choice);
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
    m.impl("_fused_sdp_choice", &tvkb::sdp_choice);
    m.impl("_scaled_dot_product_fused_attention_overrideable", &tvkb::sdpa_forward);
    m.impl("_scaled_dot_product_fused_attention_overrideable_backward", &tvkb::sdpa_backward);
}
