/*
 * gemm_oracle.c - CPU restatement of the reference's matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path links or calls this
 * file; tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it
 * as the checker.
 *
 * What it restates (reference file:line):
 *   - the SIMD tile GEMM's per-output order: operands are converted to the
 *     float32 accumulate type on load, every output accumulates over
 *     k = 0..K-1 in sequence (src/shaders/helpers/gemm_simd.slang:144-242,
 *     accumulate at :219-239; conversion AccumMatrix :46-64)
 *   - LinearEpilogue: v = acc*alpha; if HAS_BIAS: v = v + bias*beta; act(v)
 *     (src/shaders/helpers/gemm_simd.slang:67-99); gelu is the erf form
 *     (src/shaders/core/dtype.slang:737); relu is max(v, 0)
 *     (src/shaders/helpers/unary_ops.slang:10)
 *   - has_bias = bias defined and beta != 0 (src/api/ops/matmul.cpp:259)
 *   - alpha/beta are float32 (pushed in the accumulate type,
 *     src/vulkan/builders.h:119-140)
 *   - one rounding to the storage type: half(v) / BFloat16(v), round to
 *     nearest even (src/shaders/core/dtype.slang:255-282)
 *   - K == 0: act(beta*bias) or zeros (src/api/ops/matmul.cpp:284-288)
 *
 * Whether the reference's driver contracts `acc += a*b` into a fused
 * multiply-add is decided by the Vulkan driver's compiler, not by the
 * reference's source; both forms are offered (fma_mode 1: fmaf, 0: a rounded
 * product then a rounded add). Build with -ffp-contract=off so the compiler
 * does not change the chosen form.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2 };
enum { OR_ACT_NONE = 0, OR_ACT_RELU = 1, OR_ACT_GELU = 2 };

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float32 -> IEEE binary16, round to nearest even, with subnormals, overflow
 * to infinity and quiet NaN. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t s = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return s | (a > 0x7f800000u ? (uint16_t)(0x7e00u | ((a >> 13) & 0x3ffu)) : 0x7c00u);
    if (a >= 0x477ff000u) return s | 0x7c00u; /* >= 65520 rounds to infinity */
    if (a >= 0x38800000u) {                   /* normal half */
        uint32_t m = a + 0xfffu + ((a >> 13) & 1u);
        return s | (uint16_t)((m - 0x38000000u) >> 13);
    }
    uint32_t e = a >> 23;
    if (e < 102) return s;                    /* below 2^-25: rounds to zero */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - e;                 /* value / 2^-24 = mant >> shift */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return s | (uint16_t)q;
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return bits_f32(s | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bits_f32(s);
        /* subnormal: m * 2^-24, exact in float32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return s ? -v : v;
    }
    return bits_f32(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

static inline float load_elem(int dt, const void* p, int64_t i) {
    switch (dt) {
    case OR_F32: return ((const float*)p)[i];
    case OR_F16: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    default: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
    }
}

static inline void store_elem(int dt, void* p, int64_t i, float v) {
    switch (dt) {
    case OR_F32: ((float*)p)[i] = v; break;
    case OR_F16: ((uint16_t*)p)[i] = oracle_f32_to_f16(v); break;
    default: ((uint16_t*)p)[i] = oracle_f32_to_bf16(v); break;
    }
}

float oracle_gelu(float v) { return 0.5f * v * (1.0f + erff(v * 0.7071067811865476f)); }

static inline float epilogue(float acc, float alpha, int has_bias, float bias, float beta, int act) {
    float v = acc * alpha;
    if (has_bias) {
        float t = bias * beta;
        v = v + t;
    }
    if (act == OR_ACT_RELU) v = v > 0.0f ? v : (isnan(v) ? v : 0.0f);
    else if (act == OR_ACT_GELU) v = oracle_gelu(v);
    return v;
}

/* C[b,m,n] = act(alpha * sum_k A[b,m,k] B[b,k,n] + beta * bias[b,m,n]).
 * Strides are in elements: [batch, row, col]. Returns 0, or -1 on bad input.
 * The k loop is the outer loop of each output row, so every output still
 * sees its products in k order 0..K-1 (the order is per output, not per row). */
int oracle_gemm(int dtype, int act, int fma_mode, int64_t batch, int64_t M, int64_t N, int64_t K,
                const void* a, const int64_t* sa, const void* b, const int64_t* sb,
                const void* bias, const int64_t* sbias, void* c, const int64_t* sc,
                double alpha_d, double beta_d, float* scratch_row) {
    if (dtype < OR_F32 || dtype > OR_BF16 || act < 0 || act > 2) return -1;
    if (batch < 0 || M < 0 || N < 0 || K < 0) return -1;
    const float alpha = (float)alpha_d, beta = (float)beta_d;
    const int has_bias = bias != 0 && beta_d != 0.0;
    for (int64_t bi = 0; bi < batch; ++bi) {
        for (int64_t m = 0; m < M; ++m) {
            float* acc = scratch_row;
            for (int64_t n = 0; n < N; ++n) acc[n] = 0.0f;
            const int64_t arow = bi * sa[0] + m * sa[1];
            for (int64_t k = 0; k < K; ++k) {
                const float av = load_elem(dtype, a, arow + k * sa[2]);
                const int64_t brow = bi * sb[0] + k * sb[1];
                if (fma_mode) {
                    if (dtype == OR_F32 && sb[2] == 1) {
                        const float* bp = (const float*)b + brow;
                        for (int64_t n = 0; n < N; ++n) acc[n] = fmaf(av, bp[n], acc[n]);
                    } else {
                        for (int64_t n = 0; n < N; ++n) acc[n] = fmaf(av, load_elem(dtype, b, brow + n * sb[2]), acc[n]);
                    }
                } else {
                    for (int64_t n = 0; n < N; ++n) {
                        float prod = av * load_elem(dtype, b, brow + n * sb[2]);
                        acc[n] = acc[n] + prod;
                    }
                }
            }
            for (int64_t n = 0; n < N; ++n) {
                float bv = has_bias ? load_elem(dtype, bias, bi * sbias[0] + m * sbias[1] + n * sbias[2]) : 0.0f;
                store_elem(dtype, c, bi * sc[0] + m * sc[1] + n * sc[2], epilogue(acc[n], alpha, has_bias, bv, beta, act));
            }
        }
    }
    return 0;
}

/* One row range [m_begin, m_end) of batch `bi`, for callers that parallelise
 * over rows (each caller thread passes its own scratch row of N floats). */
int oracle_gemm_rows(int dtype, int act, int fma_mode, int64_t bi, int64_t m_begin, int64_t m_end, int64_t N, int64_t K,
                     const void* a, const int64_t* sa, const void* b, const int64_t* sb,
                     const void* bias, const int64_t* sbias, void* c, const int64_t* sc,
                     double alpha_d, double beta_d, float* scratch_row) {
    /* shift the batch into the base offsets and run the rows as a batch of one */
    int64_t sa1[3] = {0, sa[1], sa[2]}, sb1[3] = {0, sb[1], sb[2]}, sbias1[3] = {0, sbias[1], sbias[2]}, sc1[3] = {0, sc[1], sc[2]};
    size_t es = dtype == OR_F32 ? 4 : 2;
    const char* a1 = (const char*)a + (size_t)(bi * sa[0] + m_begin * sa[1]) * es;
    const char* b1 = (const char*)b + (size_t)(bi * sb[0]) * es;
    const char* bias1 = bias ? (const char*)bias + (size_t)(bi * sbias[0] + m_begin * sbias[1]) * es : 0;
    char* c1 = (char*)c + (size_t)(bi * sc[0] + m_begin * sc[1]) * es;
    return oracle_gemm(dtype, act, fma_mode, 1, m_end - m_begin, N, K, a1, sa1, b1, sb1, bias1, sbias1, c1, sc1,
                       alpha_d, beta_d, scratch_row);
}

/* ---------------------------------------------------------------------------
 * float64 and integer products.
 *
 * The reference runs these on its device too: the accumulate type of a
 * matmul is the dtype itself for float64 and for every integer type
 * (Accum = double / int64_t / int32_t / int16_t / int8_t / uint8_t,
 * src/shaders/core/dtype.slang:117-219), alpha and beta are pushed in that
 * type (src/vulkan/builders.h:119-140), and the SIMD tile accumulates each
 * output over k in sequence (src/shaders/helpers/gemm_simd.slang:219-239).
 *   - float64: fma over k = 0..K-1 per output, then v = acc*alpha;
 *     v = v + bias*beta (two roundings), act; gelu in its erf form.
 *   - integers: two's-complement arithmetic in the type's width, so every
 *     product and sum wraps modulo 2^bits; alpha and beta are integers
 *     (torch rejects fractional ones for integer inputs) converted to the
 *     type; relu is max(v, 0) in the type; there is no gelu for integers.
 * Integer sums modulo 2^bits do not depend on the order of the terms, so the
 * k order matters only for float64.
 * Dtype codes follow tvk_dtype: F64 = 3, I64 = 4, I32 = 5, I16 = 6, I8 = 7,
 * U8 = 8.
 * ------------------------------------------------------------------------- */
enum { OR_F64 = 3, OR_I64 = 4, OR_I32 = 5, OR_I16 = 6, OR_I8 = 7, OR_U8 = 8 };

/* an integer element as its two's-complement bits in 64 bits */
static inline uint64_t load_int(int dt, const void* p, int64_t i) {
    switch (dt) {
    case OR_I64: return (uint64_t)((const int64_t*)p)[i];
    case OR_I32: return (uint64_t)(int64_t)((const int32_t*)p)[i];
    case OR_I16: return (uint64_t)(int64_t)((const int16_t*)p)[i];
    case OR_I8: return (uint64_t)(int64_t)((const int8_t*)p)[i];
    default: return (uint64_t)((const uint8_t*)p)[i];
    }
}

/* the value truncated to the type (modulo 2^bits) */
static inline void store_int(int dt, void* p, int64_t i, uint64_t v) {
    switch (dt) {
    case OR_I64: ((int64_t*)p)[i] = (int64_t)v; break;
    case OR_I32: ((int32_t*)p)[i] = (int32_t)(uint32_t)v; break;
    case OR_I16: ((int16_t*)p)[i] = (int16_t)(uint16_t)v; break;
    case OR_I8: ((int8_t*)p)[i] = (int8_t)(uint8_t)v; break;
    default: ((uint8_t*)p)[i] = (uint8_t)v; break;
    }
}

/* relu in the type: negative values of the signed types become 0 */
static inline uint64_t relu_int(int dt, uint64_t v) {
    switch (dt) {
    case OR_I64: return (int64_t)v < 0 ? 0 : v;
    case OR_I32: return (int32_t)(uint32_t)v < 0 ? 0 : v;
    case OR_I16: return (int16_t)(uint16_t)v < 0 ? 0 : v;
    case OR_I8: return (int8_t)(uint8_t)v < 0 ? 0 : v;
    default: return v;
    }
}

double oracle_gelu64(double v) { return 0.5 * v * (1.0 + erf(v * 0.7071067811865476)); }

/* Rows [m_begin, m_end) of batch `bi` of a float64 or integer product
 * (strides in elements: [batch, row, col]). Returns 0, or -1 on bad input. */
int oracle_gemm_wide_rows(int dtype, int act, int64_t bi, int64_t m_begin, int64_t m_end, int64_t N, int64_t K,
                          const void* a, const int64_t* sa, const void* b, const int64_t* sb,
                          const void* bias, const int64_t* sbias, void* c, const int64_t* sc,
                          double alpha_d, double beta_d) {
    if (dtype < OR_F64 || dtype > OR_U8 || act < 0 || act > 2) return -1;
    if (dtype != OR_F64 && act == OR_ACT_GELU) return -1;
    if (m_begin < 0 || m_end < m_begin || N < 0 || K < 0) return -1;
    const int has_bias = bias != 0 && beta_d != 0.0;
    for (int64_t m = m_begin; m < m_end; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            const int64_t ai = bi * sa[0] + m * sa[1], bj = bi * sb[0] + n * sb[2];
            const int64_t ci = bi * sc[0] + m * sc[1] + n * sc[2];
            const int64_t xi = bi * sbias[0] + m * sbias[1] + n * sbias[2];
            if (dtype == OR_F64) {
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k)
                    acc = fma(((const double*)a)[ai + k * sa[2]], ((const double*)b)[bj + k * sb[1]], acc);
                double v = acc * alpha_d;
                if (has_bias) {
                    double t = ((const double*)bias)[xi] * beta_d;
                    v = v + t;
                }
                if (act == OR_ACT_RELU) v = v > 0.0 ? v : (isnan(v) ? v : 0.0);
                else if (act == OR_ACT_GELU) v = oracle_gelu64(v);
                ((double*)c)[ci] = v;
            } else {
                uint64_t acc = 0;
                for (int64_t k = 0; k < K; ++k) acc += load_int(dtype, a, ai + k * sa[2]) * load_int(dtype, b, bj + k * sb[1]);
                uint64_t v = acc * (uint64_t)(int64_t)alpha_d;
                if (has_bias) v += load_int(dtype, bias, xi) * (uint64_t)(int64_t)beta_d;
                if (act == OR_ACT_RELU) v = relu_int(dtype, v);
                store_int(dtype, c, ci, v);
            }
        }
    }
    return 0;
}
