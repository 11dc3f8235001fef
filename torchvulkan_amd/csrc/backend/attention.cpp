// Fused scaled dot-product attention on the vulkan device: the overrideable
// SDPA backend the reference registers (src/api/ops/attention.cpp:667-761).
// The forward runs tvk_attention_fwd and the backward tvk_attention_bwd. A
// requested bias gradient, or a shape the kernels decline, takes the
// reference's chunked path (attention.cpp:115-199) in float32 on the host,
// with the fallback warning (an error under TORCHVULKAN_STRICT=1).
#include "common.h"

#include <ATen/Context.h>
#include <ATen/SDPBackend.h>
#include <ATen/native/DispatchStub.h>
#include <ATen/native/transformers/attention.h>

#include <cmath>
#include <cstring>
#include <limits>

namespace tvkb {
namespace {

struct Attn {
    at::Tensor q, k, v, bias;
    int64_t B = 0, Hq = 0, Hk = 0, L = 0, S = 0, D = 0, Dv = 0, group = 1;
    bool causal = false;
    double scale = 1.0;
};

// prepare_attention (src/api/ops/attention.cpp:44-82), with its messages
Attn prepare(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& bias, bool causal,
             std::optional<double> scale) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4,
                "torchvulkan [ERROR]: fused attention takes 4D query, key and value, got ", q.sizes(), ", ", k.sizes(),
                " and ", v.sizes(), ".");
    Attn a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.B = q.size(0);
    a.Hq = q.size(1);
    a.Hk = k.size(1);
    a.L = q.size(2);
    a.S = k.size(2);
    a.D = q.size(3);
    a.Dv = v.size(3);
    TORCH_CHECK(k.size(0) == a.B && v.size(0) == a.B && v.size(1) == a.Hk && v.size(2) == a.S && k.size(3) == a.D,
                "torchvulkan [ERROR]: attention shapes don't match: query ", q.sizes(), ", key ", k.sizes(), ", value ",
                v.sizes(), ".");
    TORCH_CHECK(a.Hk > 0 && a.Hq % a.Hk == 0, "torchvulkan [ERROR]: the number of query heads (", a.Hq,
                ") must be a multiple of the key/value heads (", a.Hk, ").");
    a.group = a.Hq / a.Hk;
    a.causal = causal;
    a.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(a.D));
    if (bias.defined()) a.bias = bias.scalar_type() == q.scalar_type() ? bias : bias.to(q.scalar_type());
    return a;
}

bool kernel_takes(at::ScalarType dt, int64_t D, int64_t Dv, int64_t B, int64_t Hq) {
    return (dt == at::kHalf || dt == at::kBFloat16) && D == Dv && (D == 64 || D == 128) && B <= 65535 && Hq <= 65535;
}

// unit stride along the head dimension and 16-byte rows, else a dense copy
at::Tensor kernel_layout(const at::Tensor& t) {
    auto ok = [&]() {
        if (t.stride(3) != 1 || reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 != 0) return false;
        for (int i = 0; i < 3; ++i)
            if (t.size(i) > 1 && t.stride(i) % 8 != 0) return false;
        return true;
    };
    return ok() ? t : t.contiguous();
}

// attention_output (src/api/ops/attention.cpp:413-418): [B, L, Hq, Dv]
// underneath when the query is laid out that way, so merging heads is a view
at::Tensor attention_output(const Attn& a) {
    if (a.q.stride(1) < a.q.stride(2)) return at::empty({a.B, a.L, a.Hq, a.Dv}, a.q.options()).transpose(1, 2);
    return at::empty({a.B, a.Hq, a.L, a.Dv}, a.q.options());
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
    // the fused kernel's shapes; everything else runs the math decomposition
    if (!kernel_takes(dt, query.size(3), value.size(3), query.size(0), heads)) return math;
    return static_cast<int64_t>(at::SDPBackend::overrideable);
}

at::Tensor by_kv_head(const at::Tensor& t, const Attn& a) {
    return t.reshape({a.B, a.Hk, a.group * t.size(2), t.size(3)});
}

// chunked_scores (src/api/ops/attention.cpp:101-113) over all rows, float32 on the host
at::Tensor host_scores(const Attn& a, const at::Tensor& q, const at::Tensor& k, const at::Tensor& bias) {
    at::Tensor s = at::matmul(by_kv_head(q, a), k.transpose(-2, -1)).reshape({a.B, a.Hq, a.L, a.S}).mul(a.scale);
    if (bias.defined()) s = s.add(bias);
    if (a.causal) {
        at::Tensor row = at::arange(a.L, at::kLong).unsqueeze(1);
        at::Tensor col = at::arange(a.S, at::kLong).unsqueeze(0);
        s = at::where(col.gt(row), at::scalar_tensor(-std::numeric_limits<double>::infinity(), s.options()), s);
    }
    return s;
}

// The forward descriptor over kernel-layout q, k, v (bias broadcast to [B, Hq, L, S]).
tvk_attention_desc forward_desc(const Attn& a, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                const at::Tensor& bias, const at::Tensor& out, const at::Tensor& lse) {
    tvk_attention_desc d;
    std::memset(&d, 0, sizeof(d));
    bool ok = false;
    d.dtype = tvk_dtype_of(a.q.scalar_type(), ok);
    d.causal = a.causal ? 1 : 0;
    d.batch = a.B;
    d.heads_q = a.Hq;
    d.heads_kv = a.Hk;
    d.len_q = a.L;
    d.len_kv = a.S;
    d.head_dim = a.D;
    d.head_dim_v = a.Dv;
    for (int i = 0; i < 4; ++i) {
        d.q_stride[i] = q.stride(i);
        d.k_stride[i] = k.stride(i);
        d.v_stride[i] = v.stride(i);
        d.bias_stride[i] = bias.defined() ? bias.stride(i) : 0;
        d.out_stride[i] = out.stride(i);
    }
    for (int i = 0; i < 3; ++i) d.lse_stride[i] = lse.stride(i);
    d.q = q.data_ptr();
    d.k = k.data_ptr();
    d.v = v.data_ptr();
    d.bias = bias.defined() ? bias.data_ptr() : nullptr;
    d.out = out.data_ptr();
    d.lse = lse.data_ptr<float>();
    d.scale = a.scale;
    d.stream = stream_of(q);
    return d;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor, at::Tensor, at::Tensor>
sdpa_forward(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
             const std::optional<at::Tensor>& attn_bias, double dropout_p, bool is_causal, bool /*return_debug_mask*/,
             std::optional<double> scale) {
    TORCH_CHECK(dropout_p == 0.0, "torchvulkan [ERROR]: fused attention doesn't support dropout; it runs on the math backend.");
    Attn a = prepare(query, key, value, attn_bias.has_value() ? *attn_bias : at::Tensor(), is_causal, scale);
    at::Tensor out = attention_output(a);
    at::Tensor lse = at::empty({a.B, a.Hq, a.L}, a.q.options().dtype(at::kFloat));
    tvk_status st = TVK_ERR_UNSUPPORTED;
    if (kernel_takes(a.q.scalar_type(), a.D, a.Dv, a.B, a.Hq) && a.B * a.Hq * a.L > 0) {
        const at::Tensor q = kernel_layout(a.q), k = kernel_layout(a.k), v = kernel_layout(a.v);
        at::Tensor bias = a.bias.defined() ? a.bias.expand({a.B, a.Hq, a.L, a.S}) : at::Tensor();
        tvk_attention_desc d = forward_desc(a, q, k, v, bias, out, lse);
        st = tvk_attention_fwd(&d);
        if (st != TVK_ERR_UNSUPPORTED) check_status(st, "tvk_attention_fwd");
    } else if (a.B * a.Hq * a.L == 0) {
        st = TVK_OK;
    }
    if (st == TVK_ERR_UNSUPPORTED) {
        // chunked_forward (src/api/ops/attention.cpp:115-139) in float32 on the host
        TVKB_FALLBACK("This attention shape can't run on the device kernel. Falling back to CPU.");
        const double inf = std::numeric_limits<double>::infinity();
        at::Tensor q = a.q.cpu().to(at::kFloat), k = a.k.cpu().to(at::kFloat), v = a.v.cpu().to(at::kFloat);
        at::Tensor bias = a.bias.defined() ? a.bias.cpu().to(at::kFloat).expand({a.B, a.Hq, a.L, a.S}) : at::Tensor();
        at::Tensor s = host_scores(a, q, k, bias);
        at::Tensor mx = at::amax(s, {-1}, true);
        at::Tensor safe = at::where(mx.eq(-inf), at::scalar_tensor(0.0, mx.options()), mx);
        at::Tensor p = at::exp(s.sub(safe));
        at::Tensor sum = p.sum({-1}, true);
        at::Tensor empty = sum.eq(0.0);
        at::Tensor o = at::matmul(by_kv_head(p, a), v).reshape({a.B, a.Hq, a.L, a.Dv});
        o = o.div(at::where(empty, at::scalar_tensor(1.0, o.options()), sum));
        out.copy_(o);
        lse.copy_(at::where(empty, at::scalar_tensor(inf, sum.options()), safe.add(sum.log())).squeeze(-1));
    }
    at::Tensor philox = at::empty({}, at::TensorOptions().dtype(at::kLong));
    return {out, lse, at::Tensor(), at::Tensor(), c10::SymInt(a.L), c10::SymInt(a.S), philox, philox.clone(),
            at::empty({0}, query.options())};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> sdpa_backward(
    const at::Tensor& grad_out, const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
    const at::Tensor& attn_bias, std::array<bool, 4> grad_input_mask, const at::Tensor& out, const at::Tensor& logsumexp,
    const at::Tensor& /*cum_seq_q*/, const at::Tensor& /*cum_seq_k*/, int64_t /*max_q*/, int64_t /*max_k*/,
    double dropout_p, bool is_causal, const at::Tensor& /*philox_seed*/, const at::Tensor& /*philox_offset*/,
    std::optional<double> scale) {
    TORCH_CHECK(dropout_p == 0.0, "torchvulkan [ERROR]: fused attention doesn't support dropout; it runs on the math backend.");
    Attn a = prepare(query, key, value, attn_bias, is_causal, scale);
    if (!grad_input_mask[0] && !grad_input_mask[1] && !grad_input_mask[2] && !grad_input_mask[3]) return {};
    const bool want_bias = grad_input_mask[3] && attn_bias.defined();
    if (!want_bias && kernel_takes(a.q.scalar_type(), a.D, a.Dv, a.B, a.Hq) && out.scalar_type() == a.q.scalar_type()) {
        const at::Tensor q = kernel_layout(a.q), k = kernel_layout(a.k), v = kernel_layout(a.v);
        const at::Tensor dout = kernel_layout(grad_out.scalar_type() == a.q.scalar_type() ? grad_out : grad_out.to(a.q.scalar_type()));
        at::Tensor bias = a.bias.defined() ? a.bias.expand({a.B, a.Hq, a.L, a.S}) : at::Tensor();
        const at::Tensor lse = logsumexp.scalar_type() == at::kFloat ? logsumexp : logsumexp.to(at::kFloat);
        at::Tensor gq = at::empty({a.B, a.Hq, a.L, a.D}, a.q.options());
        at::Tensor gk = at::empty({a.B, a.Hk, a.S, a.D}, a.q.options());
        at::Tensor gv = at::empty({a.B, a.Hk, a.S, a.Dv}, a.q.options());
        tvk_attention_bwd_desc bd;
        std::memset(&bd, 0, sizeof(bd));
        bd.fwd = forward_desc(a, q, k, v, bias, out, lse);
        bd.dout = dout.data_ptr();
        bd.dq = gq.data_ptr();
        bd.dk = gk.data_ptr();
        bd.dv = gv.data_ptr();
        for (int i = 0; i < 4; ++i) {
            bd.dout_stride[i] = dout.stride(i);
            bd.dq_stride[i] = gq.stride(i);
            bd.dk_stride[i] = gk.stride(i);
            bd.dv_stride[i] = gv.stride(i);
        }
        const tvk_status st = tvk_attention_bwd(&bd);
        if (st != TVK_ERR_UNSUPPORTED) {
            check_status(st, "tvk_attention_bwd");
            return {gq, gk, gv, at::Tensor()};
        }
    }
    TVKB_FALLBACK("This attention backward runs on the CPU.");
    // chunked_backward (src/api/ops/attention.cpp:141-199) over all rows
    at::Tensor q = a.q.cpu().to(at::kFloat), k = a.k.cpu().to(at::kFloat), v = a.v.cpu().to(at::kFloat);
    at::Tensor dout = grad_out.cpu().to(at::kFloat);
    at::Tensor bias = a.bias.defined() ? a.bias.cpu().to(at::kFloat).expand({a.B, a.Hq, a.L, a.S}) : at::Tensor();
    at::Tensor delta = at::sum(dout.mul(out.cpu().to(at::kFloat)), {-1}, true);
    at::Tensor log_sum = logsumexp.cpu().to(at::kFloat).unsqueeze(-1);
    at::Tensor s = host_scores(a, q, k, bias);
    at::Tensor p = at::exp(s.sub(log_sum));
    at::Tensor dout_g = by_kv_head(dout, a);
    at::Tensor grad_v = at::matmul(by_kv_head(p, a).transpose(-2, -1), dout_g);
    at::Tensor dp = at::matmul(dout_g, v.transpose(-2, -1)).reshape({a.B, a.Hq, a.L, a.S});
    at::Tensor ds = p.mul(dp.sub(delta));
    at::Tensor dsg = by_kv_head(ds, a);
    at::Tensor grad_q = at::matmul(dsg, k).reshape({a.B, a.Hq, a.L, a.D}).mul(a.scale);
    at::Tensor grad_k = at::matmul(dsg.transpose(-2, -1), by_kv_head(q, a)).mul(a.scale);
    at::Tensor grad_bias;
    if (want_bias) grad_bias = at::sum_to(ds, a.bias.sizes()).to(a.bias.scalar_type()).to(query.device());
    const at::ScalarType dt = a.q.scalar_type();
    return {grad_q.to(dt).to(query.device()), grad_k.to(dt).to(query.device()), grad_v.to(dt).to(query.device()),
            grad_bias};
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
