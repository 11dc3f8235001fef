// tvk_gemm for float64 and the integer types (F64, I64, I32, I16, I8, U8).
//
// Reference semantics: the reference runs these matmuls on its device with
// the dtype itself as the accumulate type (Accum = double / int64_t /
// int32_t / ... / uint8_t, src/shaders/core/dtype.slang:117-219), alpha and
// beta pushed in that type (src/vulkan/builders.h:119-140), each output
// accumulated over k in sequence by the SIMD tile
// (src/shaders/helpers/gemm_simd.slang:219-239) and the same
// v = act(acc*alpha + bias*beta) epilogue (:67-99).
//   - float64: fma over k = 0..K-1 in order for every output, so the result
//     is the sequential-order one bit for bit; the epilogue rounds acc*alpha
//     and bias*beta separately, then their sum.
//   - integers: two's-complement wraparound in the type's width. Sums and
//     products modulo 2^bits do not depend on the order of the terms, so the
//     kernel accumulates in 32 bits (64 for I64) and truncates once: the bits
//     are those of accumulating in the type itself.
//
// Kernel: 64x64 output tiles, 256 threads each owning a 4x4 grid of outputs
// (rows ty + 16i, columns tx + 16j, so a quarter-wave's loads and stores run
// along 16 consecutive columns). 16-k slices of A and B are staged in LDS in
// the accumulate type; operands may have any element strides.
#include "gemm_common.h"

#include <algorithm>

namespace tvk {
namespace {

constexpr int W_T = 64, W_BK = 16, W_LD = W_T + 1;

template <int DT> struct wide;
template <> struct wide<TVK_F64> { typedef double T; typedef double Acc; };
template <> struct wide<TVK_I64> { typedef int64_t T; typedef uint64_t Acc; };
template <> struct wide<TVK_I32> { typedef int32_t T; typedef uint32_t Acc; };
template <> struct wide<TVK_I16> { typedef int16_t T; typedef uint32_t Acc; };
template <> struct wide<TVK_I8> { typedef int8_t T; typedef uint32_t Acc; };
template <> struct wide<TVK_U8> { typedef uint8_t T; typedef uint32_t Acc; };

struct WideArgs {
    const void* a;
    const void* b;
    const void* bias;
    void* c;
    int64_t sa[3], sb[3], sbias[3], sc[3];
    int64_t M, N, K;
    int tiles_n;
    int a_kfast, b_kfast;        // the operand's k stride is 1: its loads run along k
    int has_bias, act;
    double alpha_f, beta_f;      // float64
    uint64_t alpha_i, beta_i;    // integers: the scalars as two's-complement bits
    int64_t bh;                  // second batch dimension (tvk_gemm_desc.batch_inner), > 1 when present
    int64_t sa_h, sb_h, sbias_h, sc_h;
};

// Element offset of batch bz with outer stride s0 and inner stride sh.
__device__ inline int64_t wide_boff(const WideArgs& p, int64_t bz, int64_t s0, int64_t sh) {
    return p.bh > 1 ? (bz / p.bh) * s0 + (bz % p.bh) * sh : bz * s0;
}

// An element in the accumulate type: signed types sign-extend, so the low
// bits of every product and sum are the type's own.
template <int DT>
__device__ inline typename wide<DT>::Acc load_acc(const void* base, int64_t off) {
    typedef typename wide<DT>::T T;
    typedef typename wide<DT>::Acc Acc;
    const T v = static_cast<const T*>(base)[off];
    if constexpr (DT == TVK_F64) return v;
    else if constexpr (DT == TVK_U8) return (Acc)v;
    else return (Acc)(int64_t)v;
}

template <int DT>
__device__ inline typename wide<DT>::T finish(typename wide<DT>::Acc acc, const WideArgs& p, typename wide<DT>::Acc bv) {
    typedef typename wide<DT>::T T;
    typedef typename wide<DT>::Acc Acc;
    if constexpr (DT == TVK_F64) {
#pragma clang fp contract(off)
        double v = acc * p.alpha_f;
        if (p.has_bias) {
            const double t = bv * p.beta_f;
            v = v + t;
        }
        if (p.act == TVK_ACT_RELU) v = v > 0.0 ? v : (v != v ? v : 0.0);
        else if (p.act == TVK_ACT_GELU) v = 0.5 * v * (1.0 + erf(v * 0.7071067811865476));
        return v;
    } else {
        Acc v = acc * (Acc)p.alpha_i;
        if (p.has_bias) v += bv * (Acc)p.beta_i;
        T r = (T)v;   // truncation to the type's width (two's complement)
        if (p.act == TVK_ACT_RELU && r < (T)0) r = (T)0;
        return r;
    }
}

template <int DT>
__global__ __launch_bounds__(256) void gemm_wide_kernel(WideArgs p) {
    typedef typename wide<DT>::T T;
    typedef typename wide<DT>::Acc Acc;
    __shared__ Acc As[W_BK][W_LD];   // [k][m]
    __shared__ Acc Bs[W_BK][W_LD];   // [k][n]
    const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const int64_t tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    const int64_t m0 = tm * W_T, n0 = tn * W_T;
    const int64_t bz = blockIdx.y;
    const char* A = static_cast<const char*>(p.a) + wide_boff(p, bz, p.sa[0], p.sa_h) * (int64_t)sizeof(T);
    const char* B = static_cast<const char*>(p.b) + wide_boff(p, bz, p.sb[0], p.sb_h) * (int64_t)sizeof(T);

    Acc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (Acc)0;

    for (int64_t k0 = 0; k0 < p.K; k0 += W_BK) {
        // 64 x 16 elements of each operand, 4 per thread, consecutive threads
        // along the operand's contiguous dimension; zeros past the edges
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = tid + 256 * r;
            int kk = p.a_kfast ? e % W_BK : e / W_T, mm = p.a_kfast ? e / W_BK : e % W_T;
            int64_t gk = k0 + kk, gm = m0 + mm;
            As[kk][mm] = (gm < p.M && gk < p.K) ? load_acc<DT>(A, gm * p.sa[1] + gk * p.sa[2]) : (Acc)0;
            kk = p.b_kfast ? e % W_BK : e / W_T;
            mm = p.b_kfast ? e / W_BK : e % W_T;
            gk = k0 + kk;
            const int64_t gn = n0 + mm;
            Bs[kk][mm] = (gn < p.N && gk < p.K) ? load_acc<DT>(B, gk * p.sb[1] + gn * p.sb[2]) : (Acc)0;
        }
        __syncthreads();
        const int kn = (int)std::min<int64_t>(W_BK, p.K - k0);
        for (int kk = 0; kk < kn; ++kk) {
            Acc av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (DT == TVK_F64) acc[i][j] = fma(av[i], bv[j], acc[i][j]);
                    else acc[i][j] += av[i] * bv[j];
                }
        }
        __syncthreads();
    }

    T* C = static_cast<T*>(p.c) + wide_boff(p, bz, p.sc[0], p.sc_h);
    const char* X = p.has_bias ? static_cast<const char*>(p.bias) + wide_boff(p, bz, p.sbias[0], p.sbias_h) * (int64_t)sizeof(T) : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty + 16 * i;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx + 16 * j;
            if (n >= p.N) continue;
            const Acc bv = p.has_bias ? load_acc<DT>(X, m * p.sbias[1] + n * p.sbias[2]) : (Acc)0;
            C[m * p.sc[1] + n * p.sc[2]] = finish<DT>(acc[i][j], p, bv);
        }
    }
}

template <int DT>
tvk_status launch_wide(const tvk_gemm_desc& d, WideArgs w) {
    const int64_t tiles_m = (d.M + W_T - 1) / W_T, tiles_n = (d.N + W_T - 1) / W_T;
    if (tiles_m * tiles_n > (int64_t)0x7fffffff) return fail(TVK_ERR_UNSUPPORTED, "tvk_gemm: too many output tiles");
    w.tiles_n = (int)tiles_n;
    const hipStream_t s = resolve_stream(d.stream);
    const size_t es = sizeof(typename wide<DT>::T);
    // batch chunks of whole inner batches, so each chunk starts at an outer index
    const int64_t bh = w.bh > 1 ? w.bh : 1, step = 65535 / bh * bh;
    for (int64_t b0 = 0; b0 < d.batch; b0 += step) {
        const int nb = (int)std::min<int64_t>(step, d.batch - b0);
        const int64_t bo = b0 / bh;
        WideArgs q = w;
        q.a = static_cast<const char*>(d.a) + (size_t)(bo * d.a_stride[0]) * es;
        q.b = static_cast<const char*>(d.b) + (size_t)(bo * d.b_stride[0]) * es;
        q.c = static_cast<char*>(d.c) + (size_t)(bo * d.c_stride[0]) * es;
        if (q.has_bias) q.bias = static_cast<const char*>(d.bias) + (size_t)(bo * d.bias_stride[0]) * es;
        hipLaunchKernelGGL(gemm_wide_kernel<DT>, dim3((unsigned)(tiles_m * tiles_n), (unsigned)nb), dim3(256), 0, s, q);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_gemm: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

}  // namespace

bool gemm_wide_dtype(int dtype) {
    return dtype == TVK_F64 || dtype == TVK_I64 || dtype == TVK_I32 || dtype == TVK_I16 || dtype == TVK_I8 || dtype == TVK_U8;
}

const char* gemm_wide_name(int dtype) { return dtype == TVK_F64 ? "gemm_wide_f64" : "gemm_wide_int"; }

tvk_status gemm_wide_run(const tvk_gemm_desc& d) {
    if (d.dtype != TVK_F64 && d.activation == TVK_ACT_GELU)
        return fail(TVK_ERR_INVALID, "tvk_gemm: gelu is only defined for floating point products");
    WideArgs w{};
    w.a = d.a; w.b = d.b; w.c = d.c;
    w.has_bias = d.bias != nullptr && d.beta != 0.0;
    w.bias = w.has_bias ? d.bias : nullptr;
    for (int i = 0; i < 3; ++i) {
        w.sa[i] = d.a_stride[i];
        w.sb[i] = d.b_stride[i];
        w.sc[i] = d.c_stride[i];
        w.sbias[i] = w.has_bias ? d.bias_stride[i] : 0;
    }
    w.M = d.M; w.N = d.N; w.K = d.K;
    w.bh = d.batch_inner > 1 ? d.batch_inner : 1;
    w.sa_h = d.a_stride_inner; w.sb_h = d.b_stride_inner; w.sc_h = d.c_stride_inner;
    w.sbias_h = w.has_bias ? d.bias_stride_inner : 0;
    w.a_kfast = d.a_stride[2] == 1 && !(d.a_stride[1] == 1 && d.M > 1 && d.K == 1);
    w.b_kfast = d.b_stride[1] == 1 && !(d.b_stride[2] == 1 && d.N > 1 && d.K == 1);
    w.act = d.activation;
    w.alpha_f = d.alpha;
    w.beta_f = d.beta;
    // integer scalars: the reference converts them to the accumulate type
    w.alpha_i = (uint64_t)(int64_t)d.alpha;
    w.beta_i = (uint64_t)(int64_t)d.beta;
    switch (d.dtype) {
    case TVK_F64: return launch_wide<TVK_F64>(d, w);
    case TVK_I64: return launch_wide<TVK_I64>(d, w);
    case TVK_I32: return launch_wide<TVK_I32>(d, w);
    case TVK_I16: return launch_wide<TVK_I16>(d, w);
    case TVK_I8: return launch_wide<TVK_I8>(d, w);
    default: return launch_wide<TVK_U8>(d, w);
    }
}

}  // namespace tvk
