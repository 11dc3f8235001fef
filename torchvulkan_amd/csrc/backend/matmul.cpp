// aten::mm / bmm / addmm / baddbmm / _addmm_activation (+ .out), addbmm,
// addmv, mm.dtype and _scaled_mm for the vulkan (PrivateUse1) device,
// computed by tvk_gemm (complex operands as products of their real parts).
//
// Follows src/api/ops/matmul.cpp: operand preparation and broadcasting
// (prepare_matmul_operands :27-78, get_matmul_shape :108-140,
// finish_matmul_output :142-149), the has_bias rule (:259), the empty / K == 0
// cases (:284-288), the CPU-identical error checks (check_matrix_product
// :600-606, bmm's meta checks :624-630, baddbmm's dtype check :662-663) and
// the registrations (:751-763). Operands are handed to the kernel as strided
// views: transposed and sliced operands are not copied.
#include "common.h"

#include <ATen/native/Resize.h>
#include <ATen/ops/matmul_native.h>

namespace tvkb {
namespace {

enum Activation { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2 };

// dtypes tvk_gemm computes: float32/16, bfloat16 on the MFMA kernels, float64
// and the integer types (accumulating in their own type, as the reference's
// device does, src/api/ops/helpers.h:59-82) on the wide kernel. bool stays on
// the CPU, which rejects it too.
int32_t gemm_dtype_of(c10::ScalarType t, bool& ok) {
    ok = true;
    switch (t) {
    case at::kDouble: return TVK_F64;
    case at::kLong: return TVK_I64;
    case at::kInt: return TVK_I32;
    case at::kShort: return TVK_I16;
    case at::kChar: return TVK_I8;
    case at::kByte: return TVK_U8;
    default: return tvk_dtype_of(t, ok);
    }
}

struct Shape {
    at::Tensor self, other;
    bool self_unsqueezed = false, other_unsqueezed = false;
    int64_t M = 0, K = 0, N = 0, B = 1;
    std::vector<int64_t> batch_shape, out_shape;
};

Shape matmul_shape(const at::Tensor& self_, const at::Tensor& other_) {
    Shape s;
    s.self = self_;
    s.other = other_;
    if (s.self.dim() < 2) { s.self = s.self.unsqueeze(0); s.self_unsqueezed = true; }
    if (s.other.dim() < 2) { s.other = s.other.unsqueeze(1); s.other_unsqueezed = true; }
    TORCH_CHECK(s.self.scalar_type() == s.other.scalar_type(), "expected m1 and m2 to have the same dtype, but got: ",
                s.self.dtype().name(), " != ", s.other.dtype().name());
    TORCH_CHECK(s.self.size(-1) == s.other.size(-2), "mat1 and mat2 shapes cannot be multiplied (", s.self.size(-2), "x",
                s.self.size(-1), " and ", s.other.size(-2), "x", s.other.size(-1), ")");
    s.M = s.self.size(-2);
    s.K = s.self.size(-1);
    s.N = s.other.size(-1);
    s.batch_shape = at::infer_size(s.self.sizes().slice(0, s.self.dim() - 2), s.other.sizes().slice(0, s.other.dim() - 2));
    for (int64_t v : s.batch_shape) s.B *= v;
    s.out_shape = s.batch_shape;
    s.out_shape.push_back(s.M);
    s.out_shape.push_back(s.N);
    return s;
}

at::Tensor finish(const at::Tensor& out, const Shape& s) {
    at::Tensor r = out.reshape(s.out_shape);
    if (s.self_unsqueezed && s.other_unsqueezed) return r.squeeze(-1).squeeze(-1);
    if (s.self_unsqueezed) return r.squeeze(-2);
    if (s.other_unsqueezed) return r.squeeze(-1);
    return r;
}

at::Tensor apply_activation(const at::Tensor& t, Activation act) {
    if (act == ACT_RELU) return at::relu(t);
    if (act == ACT_GELU) return at::gelu(t);
    return t;
}

// 3-D view [B, rows, cols] of an operand expanded to the batch shape, without
// a copy when the expanded batch dims collapse into one stride.
at::Tensor batched_view(const at::Tensor& t, const std::vector<int64_t>& batch_shape, int64_t rows, int64_t cols, int64_t B) {
    std::vector<int64_t> shape(batch_shape);
    shape.push_back(rows);
    shape.push_back(cols);
    at::Tensor e = t.expand(shape);
    if (e.dim() == 2) return e.unsqueeze(0);
    // the flattened batch index b has offset b * s when every non-1 batch dim
    // has stride s * (product of the batch dims after it); broadcast dims
    // (stride 0 throughout) collapse too
    int64_t s = -1, prod = 1;
    bool ok = true;
    for (int64_t d = (int64_t)batch_shape.size() - 1; d >= 0; --d) {
        if (batch_shape[d] == 1) continue;
        const int64_t st = e.stride(d);
        if (s < 0) {
            s = st;
        } else if (st != s * prod) {
            ok = false;
        }
        prod *= batch_shape[d];
    }
    if (s < 0) s = 0;
    if (ok) return e.as_strided({B, rows, cols}, {s, e.stride(-2), e.stride(-1)});
    return e.reshape({B, rows, cols});  // materialises a contiguous copy
}

// Whether batch dims [lo, hi) of an expanded operand collapse into one
// stride (returned in `stride`; 0 when every dim there is 1 or broadcast).
bool batch_range_collapses(const at::Tensor& e, const std::vector<int64_t>& batch_shape, int64_t lo, int64_t hi, int64_t& stride) {
    int64_t s = -1, prod = 1;
    for (int64_t d = hi - 1; d >= lo; --d) {
        if (batch_shape[d] == 1) continue;
        const int64_t st = e.stride(d);
        if (s < 0) s = st;
        else if (st != s * prod) return false;
        prod *= batch_shape[d];
    }
    stride = s < 0 ? 0 : s;
    return true;
}

// Two batch dimensions for operands whose batch dims do not collapse into
// one (head-strided [B, H, L, D] views): the first batch dims [0, split)
// and the rest [split, n) each collapse into one stride, for every operand.
// Returns the split (0: none found) and the 4-D views [B1, B2, rows, cols].
int64_t batched_views2(const std::vector<const at::Tensor*>& ops, const std::vector<std::pair<int64_t, int64_t>>& mats,
                       const std::vector<int64_t>& batch_shape, std::vector<at::Tensor>& views) {
    const int64_t n = (int64_t)batch_shape.size();
    for (int64_t split = n - 1; split >= 1; --split) {
        int64_t b1 = 1, b2 = 1;
        for (int64_t d = 0; d < split; ++d) b1 *= batch_shape[d];
        for (int64_t d = split; d < n; ++d) b2 *= batch_shape[d];
        if (b1 == 1 || b2 == 1) continue;
        std::vector<at::Tensor> vs;
        bool ok = true;
        for (size_t i = 0; i < ops.size() && ok; ++i) {
            if (!ops[i]->defined()) {
                vs.emplace_back();
                continue;
            }
            std::vector<int64_t> shape(batch_shape);
            shape.push_back(mats[i].first);
            shape.push_back(mats[i].second);
            const at::Tensor e = ops[i]->expand(shape);
            int64_t s0 = 0, s1 = 0;
            ok = batch_range_collapses(e, batch_shape, 0, split, s0) && batch_range_collapses(e, batch_shape, split, n, s1);
            if (ok) vs.push_back(e.as_strided({b1, b2, mats[i].first, mats[i].second}, {s0, s1, e.stride(-2), e.stride(-1)}));
        }
        if (ok) {
            views = vs;
            return split;
        }
    }
    return 0;
}

// One tvk_gemm: out[B, M, N] = act(alpha * a[B, M, K] . b[B, K, N] + beta * bias)
// on 3-D views, or on 4-D views [B1, B2, ., .] with two batch dimensions
// (bias undefined: none). False when the library declines the shape (the
// caller falls back); other failures throw.
tvk_gemm_desc base_desc(int32_t tdt, Activation act) {
    tvk_gemm_desc d;
    std::memset(&d, 0, sizeof(d));
    d.dtype = tdt;
    d.activation = act;
    // TORCHVULKAN_EXACT is read once, at the first product
    static const bool exact = [] {
        const char* e = std::getenv("TORCHVULKAN_EXACT");
        return e && e[0] && std::strcmp(e, "0") != 0;
    }();
    d.flags = exact ? TVK_GEMM_EXACT : 0;
    return d;
}

// Runs a filled descriptor; false when the library declines it (the caller
// falls back), other failures throw.
bool launch_desc(tvk_gemm_desc& d, const at::Tensor& out) {
    d.stream = stream_of(out);
    // TORCHVULKAN_AUTOTUNE=1: a shape class without a recorded kernel is timed
    // over every candidate first and the fastest recorded (the reference tunes
    // every matmul on first sight, src/api/ops/matmul.cpp:538-544); otherwise
    // the recorded or shape-chosen kernel runs
    static const bool autotune = [] {
        const char* e = std::getenv("TORCHVULKAN_AUTOTUNE");
        return e != nullptr && e[0] && std::strcmp(e, "0") != 0;
    }();
    const tvk_status st = autotune ? tvk_gemm_tune(&d, nullptr, 0) : tvk_gemm(&d);
    if (st == TVK_ERR_UNSUPPORTED) {
        TVKB_FALLBACK(tvk_last_error(), ". Falling back to CPU.");
        return false;
    }
    check_status(st, "tvk_gemm");
    return true;
}

bool run_gemm(const at::Tensor& a, const at::Tensor& b, const at::Tensor& bias, double alpha, double beta, Activation act,
              int32_t tdt, const at::Tensor& out) {
    tvk_gemm_desc d = base_desc(tdt, act);
    const bool two = out.dim() == 4;
    d.batch = two ? out.size(0) * out.size(1) : out.size(0);
    d.M = out.size(-2); d.N = out.size(-1); d.K = a.size(-1);
    d.a = a.data_ptr();
    d.b = b.data_ptr();
    d.c = out.data_ptr();
    // (batch, row, col) element strides; with two batch dims the inner one's separately
    auto st3 = [&](const at::Tensor& t, int64_t* dst) {
        dst[0] = t.stride(0);
        dst[1] = t.stride(-2);
        dst[2] = t.stride(-1);
    };
    st3(a, d.a_stride);
    st3(b, d.b_stride);
    st3(out, d.c_stride);
    if (bias.defined()) {
        d.bias = bias.data_ptr();
        st3(bias, d.bias_stride);
    }
    if (two) {
        d.batch_inner = out.size(1);
        d.a_stride_inner = a.stride(1);
        d.b_stride_inner = b.stride(1);
        d.c_stride_inner = out.stride(1);
        d.bias_stride_inner = bias.defined() ? bias.stride(1) : 0;
    }
    d.alpha = alpha;
    d.beta = bias.defined() ? beta : 0.0;
    return launch_desc(d, out);
}

// The 2-D products (mm, addmm, _addmm_activation: every nn.Linear layer and its
// gradients) with operands of one real dtype, a unit stride in each operand's
// matrix dims and a bias that broadcasts to [M, N] in at most two dims: the
// sizes and strides go straight into the descriptor, without the expand /
// as_strided / reshape views of the general path (each a dispatcher call).
// Returns an undefined tensor when the product is not of this kind.
at::Tensor gemm2d_direct(const at::Tensor& a, const at::Tensor& b, const at::Tensor& bias_, const at::Scalar& alpha,
                         const at::Scalar& beta, Activation act, bool& declined) {
    declined = false;
    if (a.dim() != 2 || b.dim() != 2 || a.scalar_type() != b.scalar_type() || a.is_conj() || b.is_conj() || a.is_neg() ||
        b.is_neg())
        return {};
    bool ok = false;
    const int32_t tdt = gemm_dtype_of(a.scalar_type(), ok);
    if (!ok) return {};
    const int64_t M = a.size(0), K = a.size(1), N = b.size(1);
    if (M == 0 || N == 0 || K == 0 || b.size(0) != K) return {};
    auto unit = [](const at::Tensor& t) {
        return (t.size(1) <= 1 || t.stride(1) == 1) || (t.size(0) <= 1 || t.stride(0) == 1);
    };
    if (!unit(a) || !unit(b) || a.stride(0) < 0 || a.stride(1) < 0 || b.stride(0) < 0 || b.stride(1) < 0) return {};
    const double be = beta.toDouble();
    const bool has_bias = bias_.defined() && be != 0.0;
    int64_t bs_row = 0, bs_col = 0;
    if (has_bias) {
        if (bias_.scalar_type() != a.scalar_type() || bias_.dim() > 2 || bias_.is_conj() || bias_.is_neg()) return {};
        // right-aligned broadcast of the bias to [M, N]
        const int64_t bn = bias_.dim() >= 1 ? bias_.size(-1) : 1, bm = bias_.dim() == 2 ? bias_.size(0) : 1;
        if ((bn != N && bn != 1) || (bm != M && bm != 1)) return {};
        bs_col = (bias_.dim() >= 1 && bn != 1) ? bias_.stride(-1) : 0;
        bs_row = (bias_.dim() == 2 && bm != 1) ? bias_.stride(0) : 0;
        if (bs_col < 0 || bs_row < 0) return {};
    }
    at::Tensor out = at::empty({M, N}, a.options());
    tvk_gemm_desc d = base_desc(tdt, act);
    d.batch = 1; d.M = M; d.N = N; d.K = K;
    d.a = a.data_ptr(); d.a_stride[1] = a.stride(0); d.a_stride[2] = a.stride(1);
    d.b = b.data_ptr(); d.b_stride[1] = b.stride(0); d.b_stride[2] = b.stride(1);
    d.c = out.data_ptr(); d.c_stride[1] = N; d.c_stride[2] = 1;
    if (has_bias) {
        d.bias = bias_.data_ptr();
        d.bias_stride[1] = bs_row;
        d.bias_stride[2] = bs_col;
    }
    d.alpha = alpha.toDouble();
    d.beta = has_bias ? be : 0.0;
    if (!launch_desc(d, out)) {
        declined = true;
        return {};
    }
    return out;
}

bool negative_strides(std::initializer_list<const at::Tensor*> ts) {
    for (const at::Tensor* t : ts) {
        if (!t->defined()) continue;
        for (int64_t d = 0; d < t->dim(); ++d)
            if (t->stride(d) < 0) return true;
    }
    return false;
}

// ---- complex operands ------------------------------------------------------
// complex_matmul (src/api/ops/matmul.cpp:355-371): four real products of the
// (real, imaginary) parts, in the real type (float32 for complex32),
//   re = A.re B.re - A.im B.im,  im = A.re B.im + A.im B.re,
// each product rounded to the real type and the pair then combined in one
// more rounding. Here the second product of each pair takes the first as its
// bias with beta = 1 and alpha = -1 or 1, which is that same rounding
// (acc * -1 is exact and the epilogue's one sum is the subtraction). Then
// r *= alpha and r += beta * bias as complex multiplications of the parts
// (complex_mul, src/api/ops/complex.cpp:43-46), when alpha != 1 and when a
// bias is given with beta != 0. Conjugate and negative views are not
// materialised: their signs fold into the products' alphas and the scalars.

// The parts of a complex tensor as dense real tensors, and the sign each one
// carries (conjugate view: imaginary negated; negative view: both).
struct Parts {
    at::Tensor re, im;
    double sre = 1.0, sim = 1.0;
};

Parts parts_of(const at::Tensor& z, c10::ScalarType real) {
    Parts p;
    at::Tensor w = z;
    if (w.is_neg()) {
        w = w._neg_view();
        p.sre = -p.sre;
        p.sim = -p.sim;
    }
    if (w.is_conj()) {
        w = w.conj();
        p.sim = -p.sim;
    }
    at::Tensor pairs = at::view_as_real(w);
    if (pairs.scalar_type() != real) pairs = pairs.to(real);
    p.re = pairs.select(-1, 0).contiguous();
    p.im = pairs.select(-1, 1).contiguous();
    return p;
}

// (re, im) * (s.re, s.im) with the parts' signs folded into the scalar:
// the reference's complex_mul of resolved parts, whose products differ from
// these only by exact sign flips.
void complex_scale(at::Tensor& re, at::Tensor& im, double sre, double sim, c10::complex<double> s) {
    auto sc = [&](double v) { return at::scalar_tensor(v, re.options()); };
    at::Tensor r = at::sub(at::mul(re, sc(sre * s.real())), at::mul(im, sc(sim * s.imag())));
    at::Tensor i = at::add(at::mul(re, sc(sre * s.imag())), at::mul(im, sc(sim * s.real())));
    re = r;
    im = i;
}

at::Tensor complex_product(const Shape& s, const at::Tensor& bias_, const at::Scalar& alpha, const at::Scalar& beta,
                           c10::ScalarType dtype, const std::function<at::Tensor()>& fallback) {
    const c10::ScalarType real = c10::toRealValueType(dtype == at::kComplexHalf ? at::kComplexFloat : dtype);
    bool ok = false;
    const int32_t tdt = gemm_dtype_of(real, ok);
    at::Tensor a3 = batched_view(s.self, s.batch_shape, s.M, s.K, s.B);
    at::Tensor b3 = batched_view(s.other, s.batch_shape, s.K, s.N, s.B);
    at::Tensor out = at::empty({s.B, s.M, s.N}, a3.options().dtype(dtype));
    if (s.M == 0 || s.N == 0 || s.B == 0) return out;
    const at::TensorOptions ro = a3.options().dtype(real);
    at::Tensor re, im;
    if (s.K == 0) {
        re = at::zeros({s.B, s.M, s.N}, ro);
        im = at::zeros({s.B, s.M, s.N}, ro);
    } else {
        const Parts A = parts_of(a3, real), B = parts_of(b3, real);
        at::Tensor t1 = at::empty({s.B, s.M, s.N}, ro), t3 = at::empty({s.B, s.M, s.N}, ro);
        re = at::empty({s.B, s.M, s.N}, ro);
        im = at::empty({s.B, s.M, s.N}, ro);
        if (!run_gemm(A.re, B.re, {}, A.sre * B.sre, 0.0, ACT_NONE, tdt, t1) ||
            !run_gemm(A.im, B.im, t1, -A.sim * B.sim, 1.0, ACT_NONE, tdt, re) ||
            !run_gemm(A.re, B.im, {}, A.sre * B.sim, 0.0, ACT_NONE, tdt, t3) ||
            !run_gemm(A.im, B.re, t3, A.sim * B.sre, 1.0, ACT_NONE, tdt, im))
            return fallback();
    }
    const c10::complex<double> al = alpha.toComplexDouble(), be = beta.toComplexDouble();
    if (al != c10::complex<double>(1.0)) complex_scale(re, im, 1.0, 1.0, al);
    if (bias_.defined() && be != c10::complex<double>(0.0)) {
        at::Tensor c3 = batched_view(bias_, s.batch_shape, s.M, s.N, s.B);
        Parts C = parts_of(c3.scalar_type() == dtype ? c3 : c3.to(dtype), real);
        complex_scale(C.re, C.im, C.sre, C.sim, be);
        re = at::add(re, C.re);
        im = at::add(im, C.im);
    }
    at::Tensor pairs = at::view_as_real(out);
    pairs.select(-1, 0).copy_(re);
    pairs.select(-1, 1).copy_(im);
    return out;
}

at::Tensor dispatch_matmul(const at::Tensor& self_, const at::Tensor& other_, const at::Tensor& bias_, const at::Scalar& alpha,
                           const at::Scalar& beta, Activation act, const std::function<at::Tensor()>& fallback) {
    Shape s = matmul_shape(self_, other_);
    // matmul_shape checked that both have one dtype (at::result_type would
    // first resolve a conjugate view through the math-bit fallback)
    const c10::ScalarType dtype = s.self.scalar_type();
    if (at::isComplexType(dtype)) {
        if (act != ACT_NONE || negative_strides({&s.self, &s.other, &bias_})) {
            TVKB_FALLBACK("A ", dtype, " matmul with an activation or negative strides. Falling back to CPU.");
            return fallback();
        }
        return finish(complex_product(s, bias_, alpha, beta, dtype, fallback), s);
    }
    const bool has_bias = bias_.defined() && beta.toDouble() != 0.0;
    bool ok = false;
    const int32_t tdt = gemm_dtype_of(dtype, ok);
    if (!ok) {
        TVKB_FALLBACK("A ", dtype, " matmul can't run on the Vulkan device. Falling back to CPU.");
        return fallback();
    }
    TORCH_CHECK(act != ACT_GELU || at::isFloatingType(dtype), "torchvulkan [ERROR]: gelu is only defined for floating point matmuls, not ", dtype);
    {
        bool declined = false;
        at::Tensor r = gemm2d_direct(self_, other_, bias_, alpha, beta, act, declined);
        if (declined) return fallback();
        if (r.defined()) return r;
    }

    // an operand with no unit stride in its matrix dims (a broadcast gradient, such
    // as sum()'s, arrives with stride 0 in both) would take the one-thread-per-
    // output kernel: one dense copy of it is far cheaper
    auto dense_rows = [](const at::Tensor& t) {
        const bool unit = (t.size(-1) <= 1 || t.stride(-1) == 1) || (t.size(-2) <= 1 || t.stride(-2) == 1);
        return unit ? t : t.contiguous();
    };
    const at::Tensor self_t = dense_rows(s.self.to(dtype)), other_t = dense_rows(s.other.to(dtype));
    const at::Tensor bias_t = has_bias ? bias_.to(self_t.options()) : at::Tensor();
    if (s.M != 0 && s.N != 0 && s.B != 0 && s.K != 0 && s.batch_shape.size() >= 2) {
        // operands whose batch dims do not collapse into one stride (head-strided
        // [B, H, L, D] views): two batch dimensions instead of a reshape copy
        auto collapses = [&](const at::Tensor& t, int64_t r, int64_t c) {
            if (!t.defined()) return true;
            std::vector<int64_t> shape(s.batch_shape);
            shape.push_back(r);
            shape.push_back(c);
            int64_t st = 0;
            return batch_range_collapses(t.expand(shape), s.batch_shape, 0, (int64_t)s.batch_shape.size(), st);
        };
        if (!collapses(self_t, s.M, s.K) || !collapses(other_t, s.K, s.N) || !collapses(bias_t, s.M, s.N)) {
            std::vector<at::Tensor> v;
            if (batched_views2({&self_t, &other_t, &bias_t}, {{s.M, s.K}, {s.K, s.N}, {s.M, s.N}}, s.batch_shape, v) &&
                !negative_strides({&v[0], &v[1], &v[2]})) {
                at::Tensor out4 = at::empty({v[0].size(0), v[0].size(1), s.M, s.N}, self_t.options());
                if (run_gemm(v[0], v[1], v[2], alpha.toDouble(), has_bias ? beta.toDouble() : 0.0, act, tdt, out4))
                    return finish(out4.view({s.B, s.M, s.N}), s);
                return fallback();
            }
        }
    }
    at::Tensor a = batched_view(self_t, s.batch_shape, s.M, s.K, s.B);
    at::Tensor b = batched_view(other_t, s.batch_shape, s.K, s.N, s.B);
    at::Tensor out = at::empty({s.B, s.M, s.N}, a.options());
    if (s.M == 0 || s.N == 0 || s.B == 0) return finish(out, s);
    at::Tensor bias;
    if (has_bias) bias = batched_view(bias_t, s.batch_shape, s.M, s.N, s.B);
    if (s.K == 0) {
        at::Tensor r = has_bias ? (bias * beta) : out.zero_();
        return finish(apply_activation(r, act), s);
    }
    if (negative_strides({&a, &b, &bias})) {
        TVKB_FALLBACK("A matmul operand with negative strides. Falling back to CPU.");
        return fallback();
    }
    if (!run_gemm(a, b, bias, alpha.toDouble(), has_bias ? beta.toDouble() : 0.0, act, tdt, out)) return fallback();
    return finish(out, s);
}

// The CPU's checks, with the CPU's messages (torch's mm / addmm meta
// functions; the reference's check_matrix_product, matmul.cpp:600-606, keeps
// the same rule: the device rejects exactly what the CPU rejects).
void check_matrix_product(const char* name, const at::Tensor& mat1, const at::Tensor& mat2) {
    if (std::strcmp(name, "mm") == 0) {
        TORCH_CHECK(mat1.dim() == 2, "self must be a matrix");
        TORCH_CHECK(mat2.dim() == 2, "mat2 must be a matrix");
    } else {
        TORCH_CHECK(mat1.dim() == 2, "mat1 must be a matrix, got ", mat1.dim(), "-D tensor");
        TORCH_CHECK(mat2.dim() == 2, "mat2 must be a matrix, got ", mat2.dim(), "-D tensor");
    }
    TORCH_CHECK(mat1.size(1) == mat2.size(0), "mat1 and mat2 shapes cannot be multiplied (", mat1.size(0), "x",
                mat1.size(1), " and ", mat2.size(0), "x", mat2.size(1), ")");
}

at::Tensor mm_vk(const at::Tensor& self, const at::Tensor& other) {
    check_matrix_product("mm", self, other);
    return dispatch_matmul(self, other, {}, 1, 0, ACT_NONE,
                           [&]() { return at::mm(self.cpu(), other.cpu()).to(self.device()); });
}

// aten::matmul on the device: torch's composite reshapes batched operands to
// [B, M, K] first, which copies views whose batch dims do not merge
// (head-strided q/k/v); here they keep their strides (two batch dimensions).
// Broadcasting, 1-D operands and the result shape follow torch.matmul.
at::Tensor matmul_vk(const at::Tensor& self, const at::Tensor& other) {
    TORCH_CHECK(self.dim() != 0 && other.dim() != 0, "both arguments to matmul need to be at least 1D, but they are ",
                self.dim(), "D and ", other.dim(), "D");
    return dispatch_matmul(self, other, {}, 1, 0, ACT_NONE,
                           [&]() { return at::matmul(self.cpu(), other.cpu()).to(self.device()); });
}

// Autograd: the composite (whose reshape and bmm record their own backward)
// whenever a gradient is needed; the device kernel otherwise.
at::Tensor matmul_autograd_vk(const at::Tensor& self, const at::Tensor& other) {
    if (at::GradMode::is_enabled() && (self.requires_grad() || other.requires_grad())) return at::native::matmul(self, other);
    at::AutoDispatchBelowADInplaceOrView guard;
    return matmul_vk(self, other);
}

at::Tensor bmm_vk(const at::Tensor& self, const at::Tensor& other) {
    TORCH_CHECK(self.dim() == 3, "batch1 must be a 3D tensor");
    TORCH_CHECK(other.dim() == 3, "batch2 must be a 3D tensor");
    TORCH_CHECK(self.device() == other.device(), "Expected all tensors to be on the same device, but found at least two devices, ",
                self.device(), " and ", other.device(), "!");
    TORCH_CHECK(self.scalar_type() == other.scalar_type(), "expected scalar type ", self.scalar_type(), " but found ",
                other.scalar_type());
    TORCH_CHECK(other.size(0) == self.size(0) && other.size(1) == self.size(2),
                "Expected size for first two dimensions of batch2 tensor to be: [", self.size(0), ", ", self.size(2),
                "] but got: [", other.size(0), ", ", other.size(1), "].");
    return dispatch_matmul(self, other, {}, 1, 0, ACT_NONE,
                           [&]() { return at::bmm(self.cpu(), other.cpu()).to(self.device()); });
}

at::Tensor addmm_vk(const at::Tensor& input, const at::Tensor& mat1, const at::Tensor& mat2, const at::Scalar& beta,
                 const at::Scalar& alpha) {
    for (const at::Tensor* t : {&mat1, &mat2})
        TORCH_CHECK(t->device() == input.device(), "Expected all tensors to be on the same device, but found at least two devices, ",
                    input.device(), " and ", t->device(), "!");
    check_matrix_product("addmm", mat1, mat2);
    return dispatch_matmul(mat1, mat2, input, alpha, beta, ACT_NONE, [&]() {
        return at::addmm(input.cpu(), mat1.cpu(), mat2.cpu(), beta, alpha).to(mat1.device());
    });
}

at::Tensor baddbmm_vk(const at::Tensor& input, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                   const at::Scalar& alpha) {
    TORCH_CHECK(input.scalar_type() == b1.scalar_type() && b1.scalar_type() == b2.scalar_type(),
                "Input dtypes must be the same, got: input ", input.dtype().name(), ", batch1: ", b1.dtype().name(),
                ", batch2: ", b2.dtype().name());
    return dispatch_matmul(b1, b2, input, alpha, beta, ACT_NONE, [&]() {
        return at::baddbmm(input.cpu(), b1.cpu(), b2.cpu(), beta, alpha).to(b1.device());
    });
}

at::Tensor addmm_activation_vk(const at::Tensor& input, const at::Tensor& mat1, const at::Tensor& mat2, const at::Scalar& beta,
                            const at::Scalar& alpha, bool use_gelu) {
    return dispatch_matmul(mat1, mat2, input, alpha, beta, use_gelu ? ACT_GELU : ACT_RELU, [&]() {
        return at::_addmm_activation(input.cpu(), mat1.cpu(), mat2.cpu(), beta, alpha, use_gelu).to(mat1.device());
    });
}

// resize-and-copy into an out= tensor (src/api/ops/helpers.h:363-378)
at::Tensor& fill_out(at::Tensor& out, const at::Tensor& res) {
    TORCH_CHECK(!res.is_privateuseone() || out.is_privateuseone(), "Expected out tensor to have device ", res.device(),
                ", but got ", out.device(), " instead");
    TORCH_CHECK(at::canCast(res.scalar_type(), out.scalar_type()), "result type ", res.scalar_type(),
                " can't be cast to the desired output type ", out.scalar_type());
    if (res.is_same(out)) return out;
    if (at::native::resize_output(out, res.sizes()) && res.is_non_overlapping_and_dense() && out.strides() != res.strides())
        out.as_strided_(res.sizes(), res.strides());
    out.copy_(res);
    return out;
}

at::Tensor& mm_out_vk(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) { return fill_out(out, mm_vk(self, other)); }
at::Tensor& bmm_out_vk(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) {
    TORCH_CHECK(out.device() == self.device(), "Expected out tensor to have device ", self.device(), ", but got ",
                out.device(), " instead");
    return fill_out(out, bmm_vk(self, other));
}
at::Tensor& addmm_out_vk(const at::Tensor& input, const at::Tensor& m1, const at::Tensor& m2, const at::Scalar& beta,
                      const at::Scalar& alpha, at::Tensor& out) {
    return fill_out(out, addmm_vk(input, m1, m2, beta, alpha));
}
at::Tensor& baddbmm_out_vk(const at::Tensor& input, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                        const at::Scalar& alpha, at::Tensor& out) {
    return fill_out(out, baddbmm_vk(input, b1, b2, beta, alpha));
}
at::Tensor& addmm_activation_out_vk(const at::Tensor& input, const at::Tensor& m1, const at::Tensor& m2, const at::Scalar& beta,
                                 const at::Scalar& alpha, bool use_gelu, at::Tensor& out) {
    return fill_out(out, addmm_activation_vk(input, m1, m2, beta, alpha, use_gelu));
}

// addbmm: sum_b b1[b] @ b2[b] as one mm on permuted operands
// (src/api/decompositions.cpp:1114-1139)
at::Tensor addbmm_vk(const at::Tensor& input, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                  const at::Scalar& alpha) {
    TORCH_CHECK(b1.dim() == 3, "batch1 must be a 3D tensor");
    TORCH_CHECK(b2.dim() == 3, "batch2 must be a 3D tensor");
    TORCH_CHECK(b1.size(0) == b2.size(0), "batch1 and batch2 must have same number of batches, got ", b1.size(0), " and ",
                b2.size(0));
    TORCH_CHECK(b1.size(2) == b2.size(1), "Incompatible matrix sizes for bmm (", b1.size(1), "x", b1.size(2), " and ",
                b2.size(1), "x", b2.size(2), ")");
    TORCH_CHECK(input.scalar_type() == b1.scalar_type(), "self and mat2 must have the same dtype, but got ",
                input.scalar_type(), " and ", b1.scalar_type());
    const int64_t B = b1.size(0), M = b1.size(1), K = b1.size(2), N = b2.size(2);
    at::Tensor a = b1.permute({1, 0, 2}).reshape({M, B * K});
    at::Tensor b = b2.reshape({B * K, N});
    return dispatch_matmul(a, b, input, alpha, beta, ACT_NONE, [&]() {
        return at::addbmm(input.cpu(), b1.cpu(), b2.cpu(), beta, alpha).to(b1.device());
    });
}

at::Tensor& addbmm_out_vk(const at::Tensor& input, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                          const at::Scalar& alpha, at::Tensor& out) {
    return fill_out(out, addbmm_vk(input, b1, b2, beta, alpha));
}

// in-place variants write the computed result back into self, which must
// already have the result's shape (src/api/ops/helpers.h:389-397)
at::Tensor& write_back(at::Tensor& self, const at::Tensor& res) {
    TORCH_CHECK(at::canCast(res.scalar_type(), self.scalar_type()), "result type ", res.scalar_type(),
                " can't be cast to the desired output type ", self.scalar_type());
    TORCH_CHECK(res.sizes() == self.sizes(), "output with shape ", self.sizes(), " doesn't match the broadcast shape ",
                res.sizes());
    if (!res.is_same(self)) self.copy_(res);
    return self;
}

at::Tensor& addbmm_inplace_vk(at::Tensor& self, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                              const at::Scalar& alpha) {
    return write_back(self, addbmm_vk(self, b1, b2, beta, alpha));
}

// mm.dtype / mm.dtype_out (src/api/decompositions.cpp:1146-1157): the output
// keeps the inputs' dtype, or is float32 for float16/bfloat16 inputs, which
// is the float32 product of the widened operands (every float16/bfloat16
// value is exact in float32, so only the accumulation differs from the
// inputs' own product: it runs in the float32 kernel's sequential order)
at::Tensor mm_dtype_vk(const at::Tensor& self, const at::Tensor& mat2, at::ScalarType out_dtype) {
    const at::ScalarType dt = self.scalar_type();
    TORCH_CHECK(out_dtype == dt || (out_dtype == at::kFloat && (dt == at::kHalf || dt == at::kBFloat16)),
                "out_dtype must be the same as input dtype or fp32 for fp16/bf16 inputs");
    if (out_dtype == dt) return mm_vk(self, mat2);
    return mm_vk(self.to(at::kFloat), mat2.to(at::kFloat));
}

at::Tensor& mm_dtype_out_vk(const at::Tensor& self, const at::Tensor& mat2, at::ScalarType out_dtype, at::Tensor& out) {
    return fill_out(out, mm_dtype_vk(self, mat2, out_dtype));
}

// addmv: out = beta*self + alpha*(mat @ vec), with torch's addmv meta checks
// and messages. The product runs as the one-row GEMM
// out^T[1, M] = vec^T[1, K] . mat^T[K, M] (self broadcast along the row as
// the bias), the M <= 16 streaming shape of tvk_gemm; no operand is copied.
// The reference computes it as mm(mat, vec.unsqueeze(1)) in float32 for
// float16/bfloat16 (src/api/decompositions.cpp:109-124); here the float32
// accumulation and the epilogue round once to the dtype.
at::Tensor addmv_vk(const at::Tensor& self, const at::Tensor& mat, const at::Tensor& vec, const at::Scalar& beta,
                    const at::Scalar& alpha) {
    TORCH_CHECK(mat.dim() == 2 && vec.dim() == 1 && self.dim() <= 1, "vector + matrix @ vector expected, got ", self.dim(),
                ", ", mat.dim(), ", ", vec.dim());
    TORCH_CHECK(mat.size(1) == vec.size(0) && (mat.size(0) == self.numel() || self.numel() == 1),
                "size mismatch, got input (", self.dim() == 0 ? 1 : self.size(0), "), mat (", mat.size(0), "x", mat.size(1),
                "), vec (", vec.size(0), ")");
    TORCH_CHECK(mat.scalar_type() == vec.scalar_type(), "expected scalar type ", mat.scalar_type(), " but found ",
                vec.scalar_type());
    for (const at::Tensor* t : {&self, &vec})
        TORCH_CHECK(t->device() == mat.device(), "Expected all tensors to be on the same device, but found at least two devices, ",
                    mat.device(), " and ", t->device(), "!");
    const int64_t M = mat.size(0);
    at::Tensor bias = self.dim() == 0 ? self.reshape({1}) : self;
    at::Tensor r = dispatch_matmul(vec.unsqueeze(0), mat.t(), bias, alpha, beta, ACT_NONE, [&]() {
        return at::addmv(self.cpu(), mat.cpu(), vec.cpu(), beta, alpha).to(mat.device()).unsqueeze(0);
    });
    return r.reshape({M});
}

at::Tensor& addmv_out_vk(const at::Tensor& self, const at::Tensor& mat, const at::Tensor& vec, const at::Scalar& beta,
                         const at::Scalar& alpha, at::Tensor& out) {
    TORCH_CHECK(out.scalar_type() == mat.scalar_type(), "Expected out tensor to have dtype ", mat.scalar_type(), ", but got ",
                out.scalar_type(), " instead");
    TORCH_CHECK(out.device() == mat.device(), "Expected out tensor to have device ", mat.device(), ", but got ", out.device(),
                " instead");
    return fill_out(out, addmv_vk(self, mat, vec, beta, alpha));
}

at::Tensor& addmv_inplace_vk(at::Tensor& self, const at::Tensor& mat, const at::Tensor& vec, const at::Scalar& beta,
                             const at::Scalar& alpha) {
    return write_back(self, addmv_vk(self, mat, vec, beta, alpha));
}

// 1 / x of a float32 scalar on the device (tvk_binary's IEEE division).
at::Tensor device_reciprocal(const at::Tensor& x) {
    at::Tensor one = at::scalar_tensor(1.0, x.options().dtype(at::kFloat));
    at::Tensor v = x.reshape({}).to(at::kFloat);
    at::Tensor out = at::empty({}, one.options());
    tvk_binary_desc d;
    std::memset(&d, 0, sizeof(d));
    d.op = TVK_BIN_DIV;
    d.dtype = TVK_F32;
    d.ndim = 0;
    d.a = one.data_ptr();
    d.b = v.data_ptr();
    d.out = out.data_ptr();
    d.alpha = 1.0;
    d.stream = stream_of(out);
    check_status(tvk_binary(&d), "tvk_binary");
    return out;
}

// _scaled_mm (+ .out): torch's emulated float8 product, as the reference
// computes it on its device (scaled_mm_out_vulkan, src/api/ops/matmul.cpp:706-747,
// torch's own checks and messages): the float8 operands are decoded to
// float32 and multiplied by their scales (one scale each, or a row of A by a
// column of B), multiplied in float32, the bias added, the product
// multiplied by 1 / scale_result when the target is a float8 type, and
// rounded to the output's dtype. Every step runs on the device.
at::Tensor& scaled_mm_out_vk(const at::Tensor& mat1, const at::Tensor& mat2, const at::Tensor& scale_a,
                             const at::Tensor& scale_b, const std::optional<at::Tensor>& bias,
                             const std::optional<at::Tensor>& scale_result, std::optional<at::ScalarType> out_dtype,
                             bool /* use_fast_accum */, at::Tensor& out) {
    TORCH_CHECK_VALUE(!out_dtype || *out_dtype == out.scalar_type(), "out_dtype must match output matrix type");
    TORCH_CHECK(mat1.dim() == 2, "mat1 must be a matrix");
    TORCH_CHECK(mat2.dim() == 2, "mat2 must be a matrix");
    TORCH_CHECK(mat1.size(1) == mat2.size(0), "mat_a and mat_b shapes cannot be multiplied (", mat1.size(0), "x",
                mat1.size(1), " and ", mat2.size(0), "x", mat2.size(1), ")");
    TORCH_CHECK_VALUE(at::isFloat8Type(mat1.scalar_type()) && at::isFloat8Type(mat2.scalar_type()),
                      "mat1 and mat2 must be fp8 types, got: ", mat1.scalar_type(), mat2.scalar_type());
    const bool tensorwise = scale_a.numel() == 1 && scale_b.numel() == 1;
    const bool rowwise = scale_a.dim() == 2 && scale_b.dim() == 2 && scale_a.size(0) == mat1.size(0) &&
                         scale_a.size(1) == 1 && scale_b.size(0) == 1 && scale_b.size(1) == mat2.size(1);
    TORCH_CHECK_VALUE(tensorwise || rowwise, "Invalid scaling configuration");
    TORCH_CHECK_VALUE(scale_a.scalar_type() == at::kFloat, "scale_a must have Float elements");
    TORCH_CHECK_VALUE(scale_b.scalar_type() == at::kFloat, "scale_b must have Float elements");
    TORCH_CHECK(!scale_result || (scale_result->numel() == 1 && scale_result->scalar_type() == at::kFloat),
                "scale_result must be a float scalar");
    TORCH_CHECK(!bias || bias->numel() == mat2.size(1), "Bias must be size ", mat2.size(1), " but got ", bias->numel());
    bool ok8 = false;
    copy_dtype_of(mat1.scalar_type(), ok8);
    bool ok8b = false;
    copy_dtype_of(mat2.scalar_type(), ok8b);
    auto on_dev = [&](const at::Tensor& t) { return t.device() == mat1.device(); };
    if (!ok8 || !ok8b || !on_dev(mat2) || !on_dev(scale_a) || !on_dev(scale_b) || (bias && !on_dev(*bias)) ||
        (scale_result && !on_dev(*scale_result))) {
        TVKB_FALLBACK("A _scaled_mm of ", mat1.scalar_type(), " operands or with host tensors. Falling back to CPU.");
        std::optional<at::Tensor> bc, rc;
        if (bias) bc = bias->cpu();
        if (scale_result) rc = scale_result->cpu();
        at::Tensor r = at::_scaled_mm(mat1.cpu(), mat2.cpu(), scale_a.cpu(), scale_b.cpu(), bc, rc, out_dtype, false);
        at::native::resize_output(out, r.sizes());
        out.copy_(r);
        return out;
    }
    at::native::resize_output(out, {mat1.size(0), mat2.size(1)});
    const at::ScalarType target = out_dtype.value_or(at::kBFloat16);
    at::Tensor a = at::mul(mat1.to(at::kFloat), tensorwise ? scale_a.reshape({}) : scale_a);
    at::Tensor b = at::mul(mat2.to(at::kFloat), tensorwise ? scale_b.reshape({}) : scale_b);
    at::Tensor product = at::mm(a, b);
    if (bias) product = at::add(product, *bias);
    if (scale_result && (target == at::kFloat8_e4m3fn || target == at::kFloat8_e5m2))
        product = at::mul(product, device_reciprocal(*scale_result));
    out.copy_(product);
    return out;
}

at::Tensor scaled_mm_vk(const at::Tensor& mat1, const at::Tensor& mat2, const at::Tensor& scale_a, const at::Tensor& scale_b,
                        const std::optional<at::Tensor>& bias, const std::optional<at::Tensor>& scale_result,
                        std::optional<at::ScalarType> out_dtype, bool use_fast_accum) {
    at::Tensor out = at::empty({0}, mat1.options().dtype(out_dtype.value_or(mat1.scalar_type())));
    return scaled_mm_out_vk(mat1, mat2, scale_a, scale_b, bias, scale_result, out_dtype, use_fast_accum, out);
}

}  // namespace
}  // namespace tvkb

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
    m.impl("matmul", &tvkb::matmul_vk);
    m.impl("mm", &tvkb::mm_vk);
    m.impl("mm.out", &tvkb::mm_out_vk);
    m.impl("bmm", &tvkb::bmm_vk);
    m.impl("bmm.out", &tvkb::bmm_out_vk);
    m.impl("addmm", &tvkb::addmm_vk);
    m.impl("addmm.out", &tvkb::addmm_out_vk);
    m.impl("baddbmm", &tvkb::baddbmm_vk);
    m.impl("baddbmm.out", &tvkb::baddbmm_out_vk);
    m.impl("_addmm_activation", &tvkb::addmm_activation_vk);
    m.impl("_addmm_activation.out", &tvkb::addmm_activation_out_vk);
    m.impl("addbmm", &tvkb::addbmm_vk);
    m.impl("addbmm.out", &tvkb::addbmm_out_vk);
    m.impl("addbmm_", &tvkb::addbmm_inplace_vk);
    m.impl("mm.dtype", &tvkb::mm_dtype_vk);
    m.impl("mm.dtype_out", &tvkb::mm_dtype_out_vk);
    m.impl("addmv", &tvkb::addmv_vk);
    m.impl("addmv.out", &tvkb::addmv_out_vk);
    m.impl("addmv_", &tvkb::addmv_inplace_vk);
    m.impl("_scaled_mm", &tvkb::scaled_mm_vk);
    m.impl("_scaled_mm.out", &tvkb::scaled_mm_out_vk);
}

TORCH_LIBRARY_IMPL(aten, AutogradPrivateUse1, m) {
    m.impl("matmul", &tvkb::matmul_autograd_vk);
}
