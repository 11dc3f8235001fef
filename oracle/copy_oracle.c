/*
 * copy_oracle.c - CPU restatement of the reference's element conversion.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path links or calls this
 * file; tests/ use it as the checker of tvk_copy.
 *
 * What it restates (reference file:line):
 *   - castValue<Src, Dst>(v) = v.widen().narrow<Dst>()
 *     (src/shaders/core/cast.slang:49-52): signed integers widen to int64,
 *     uint8 to uint64, float16/bfloat16/float32 to float, float64 to double
 *     (src/shaders/core/dtype.slang:122,136,150,164,220,234,248,263,278);
 *   - narrowing is one conversion from the wide value: intN_t(v), uint8_t(v),
 *     float(v), double(v), half(v) (also from double: one rounding,
 *     dtype.slang:264-267) and BFloat16(float(v)) (dtype.slang:279-282);
 *   - with a bool on either side the value is (src != 0) ? 1 : 0, built
 *     through castFromI64 (src/shaders/ops/cast.slang:29-33).
 * A float that is NaN or outside an integer target's range is undefined in
 * the reference (SPIR-V OpConvertFToS/U); this restatement saturates and maps
 * NaN to 0, the convention the device kernel documents.
 *
 * The float64 -> float16 rounding here works on the bits of the double
 * directly (not through float32), so it checks the device's round-to-odd
 * route independently.
 *
 * float8 (torch's float8_e4m3fn and float8_e5m2): the reference has no shader
 * type for them and converts through float32 with c10's own conversions
 * (float8_tables / copy_float8_vulkan_to_vulkan,
 * src/api/tensor/transfer.cpp:129-226), so the semantics are the CPU's: the
 * code's exact value as a float, and from a float (other types convert to
 * float first) the nearest code, ties to the even code, with e4m3fn's NaN
 * for NaN, infinities and |x| >= 480 (or a rounding onto the 0x7F slot past
 * 448), and e5m2's infinity for |x| >= 65536 (or a rounding onto the 0x7C
 * slot past 57344), NaN -> 0x7F. This restatement decodes from the fields
 * with ldexp and encodes by searching every code's value for the nearest one
 * (a different method from the device's bit arithmetic); the tests pin both
 * against torch's own CPU conversion.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { C_F32 = 0, C_F16 = 1, C_BF16 = 2, C_F64 = 3, C_I64 = 4, C_I32 = 5, C_I16 = 6, C_I8 = 7, C_U8 = 8, C_BOOL = 9,
       C_F8E4M3FN = 10, C_F8E5M2 = 11 };
enum { W_I = 0, W_U = 1, W_F = 2, W_D = 3 };

/* shared with gemm_oracle.c */
uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float f);
float oracle_bf16_to_f32(uint16_t b);

typedef struct {
    int fam;
    int64_t i;
    uint64_t u;
    float f;
    double d;
} wide_t;

static int elem_size(int dt) {
    switch (dt) {
    case C_F64: case C_I64: return 8;
    case C_F32: case C_I32: return 4;
    case C_F16: case C_BF16: case C_I16: return 2;
    default: return 1;
    }
}

/* The value of a float8 code (NaN payloads as the CPU's conversion leaves
 * them: e4m3fn 0x7FF00000; e5m2 goes through float16, payload m << 21 with
 * the quiet bit set). */
float oracle_f8_decode(int dt, uint8_t c) {
    int neg = (c & 0x80) != 0;
    int e4 = dt == C_F8E4M3FN;
    int eb = e4 ? 4 : 5, mb = e4 ? 3 : 2, bias = e4 ? 7 : 15;
    int e = (c & 0x7f) >> mb, m = c & ((1 << mb) - 1);
    double v;
    if (e4 && e == 15 && m == 7) {
        uint32_t bits = 0x7FF00000u | (neg ? 0x80000000u : 0u);
        float f;
        memcpy(&f, &bits, 4);
        return f;
    }
    if (!e4 && e == 31) {
        /* the float16 route quiets a signaling NaN: the quiet bit is set */
        uint32_t bits = (m ? 0x7FC00000u : 0x7F800000u) | ((uint32_t)m << 21) | (neg ? 0x80000000u : 0u);
        float f;
        memcpy(&f, &bits, 4);
        return f;
    }
    (void)eb;
    if (e == 0) v = ldexp((double)m, 1 - bias - mb);
    else v = ldexp((double)((1 << mb) + m), e - bias - mb);
    return (float)(neg ? -v : v);
}

/* The float8 code of a float: the nearest of the codes 0..top (top being the
 * slot past the largest finite value: e4m3fn's NaN code 0x7F, valued 480 for
 * the search, e5m2's infinity 0x7C, valued 65536), ties to the even code. */
uint8_t oracle_f8_encode(int dt, float f) {
    int e4 = dt == C_F8E4M3FN;
    uint8_t sign = signbit(f) ? 0x80 : 0x00;
    if (f != f) return sign | 0x7f;
    double a = fabs((double)f);
    if (e4 && a >= 480.0) return sign | 0x7f;
    if (!e4 && a >= 65536.0) return sign | 0x7c;
    int top = e4 ? 0x7f : 0x7c;
    int best = 0;
    double best_d = a;
    for (int k = 1; k <= top; ++k) {
        double v = k == top ? (e4 ? 480.0 : 65536.0) : (double)oracle_f8_decode(dt, (uint8_t)k);
        double dd = fabs(a - v);
        if (dd < best_d || (dd == best_d && (k & 1) == 0)) {
            best = k;
            best_d = dd;
        }
    }
    return sign | (uint8_t)best;
}

static wide_t widen(int dt, const unsigned char* p) {
    wide_t w;
    memset(&w, 0, sizeof(w));
    switch (dt) {
    case C_F32: w.fam = W_F; memcpy(&w.f, p, 4); break;
    case C_F16: { uint16_t h; memcpy(&h, p, 2); w.fam = W_F; w.f = oracle_f16_to_f32(h); break; }
    case C_BF16: { uint16_t h; memcpy(&h, p, 2); w.fam = W_F; w.f = oracle_bf16_to_f32(h); break; }
    case C_F64: w.fam = W_D; memcpy(&w.d, p, 8); break;
    case C_I64: { int64_t v; memcpy(&v, p, 8); w.fam = W_I; w.i = v; break; }
    case C_I32: { int32_t v; memcpy(&v, p, 4); w.fam = W_I; w.i = v; break; }
    case C_I16: { int16_t v; memcpy(&v, p, 2); w.fam = W_I; w.i = v; break; }
    case C_I8: { int8_t v; memcpy(&v, p, 1); w.fam = W_I; w.i = v; break; }
    case C_F8E4M3FN: case C_F8E5M2: w.fam = W_F; w.f = oracle_f8_decode(dt, p[0]); break;
    default: w.fam = W_U; w.u = p[0]; break; /* U8, BOOL */
    }
    return w;
}

static int is_nonzero(const wide_t* w) {
    switch (w->fam) {
    case W_I: return w->i != 0;
    case W_U: return w->u != 0;
    case W_F: return w->f != 0.0f;
    default: return w->d != 0.0;
    }
}

static double as_double(const wide_t* w) {
    switch (w->fam) {
    case W_I: return (double)w->i;
    case W_U: return (double)w->u;
    case W_F: return (double)w->f;
    default: return w->d;
    }
}

static float as_float(const wide_t* w) {
    switch (w->fam) {
    case W_I: return (float)w->i;
    case W_U: return (float)w->u;
    case W_F: return w->f;
    default: return (float)w->d;
    }
}

/* float64 -> binary16, round to nearest even, from the double's bits. */
uint16_t oracle_f64_to_f16(double d) {
    uint64_t x;
    memcpy(&x, &d, 8);
    uint16_t s = (uint16_t)((x >> 48) & 0x8000u);
    uint64_t a = x & 0x7fffffffffffffffull;
    int e = (int)(a >> 52);
    uint64_t m = a & 0xfffffffffffffull;
    if (e == 0x7ff) return s | (m ? (uint16_t)(0x7e00u | (uint16_t)(m >> 42)) : 0x7c00u);
    if (e == 0) return s; /* float64 subnormals are far below 2^-25 */
    /* value = (2^52 + m) * 2^(e - 1075); in units of 2^-24 (half's subnormal quantum):
     * q = (2^52 + m) * 2^(e - 1075 + 24). Normal halves have a larger quantum. */
    int ue = e - 1023;                   /* unbiased exponent */
    if (ue >= 16) return s | 0x7c00u;    /* >= 65536 */
    int qexp = ue < -14 ? -24 : ue - 10; /* quantum exponent of the result */
    int shift = 1075 - e + qexp;         /* value / 2^qexp = (2^52 + m) >> shift */
    uint64_t mant = m | (1ull << 52);
    uint64_t q, rem, half;
    if (shift >= 64) return s;
    q = mant >> shift;
    rem = mant & ((1ull << shift) - 1);
    half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    /* q is the magnitude in units of 2^qexp */
    if (qexp == -24) return s | (uint16_t)q; /* subnormal (q may reach 1024: the smallest normal) */
    /* normal: q in [1024, 2048]; 2048 carries into the next binade */
    int he = ue + 15;
    if (q == 2048) { q = 1024; he++; }
    if (he >= 31) return s | 0x7c00u;
    return s | (uint16_t)((he << 10) | (q & 0x3ffu));
}

static int64_t sat_int(double v, int bits) {
    double lo = -ldexp(1.0, bits - 1);
    if (v != v) return 0;
    if (v <= lo) return (int64_t)lo;
    if (v >= -lo) return bits == 64 ? INT64_MAX : (int64_t)(-lo) - 1;
    return (int64_t)v;
}

static void narrow(int dt, const wide_t* w, unsigned char* p) {
    switch (dt) {
    case C_F32: { float f = as_float(w); memcpy(p, &f, 4); break; }
    case C_F64: { double d = as_double(w); memcpy(p, &d, 8); break; }
    case C_F16: {
        uint16_t h = w->fam == W_D ? oracle_f64_to_f16(w->d)
                   : w->fam == W_F ? oracle_f32_to_f16(w->f)
                   : oracle_f64_to_f16(as_double(w)); /* integers: exact in double up to 2^53 */
        memcpy(p, &h, 2);
        break;
    }
    case C_BF16: { uint16_t h = oracle_f32_to_bf16(as_float(w)); memcpy(p, &h, 2); break; }
    case C_I64: case C_I32: case C_I16: case C_I8: {
        int bits = 8 * elem_size(dt);
        int64_t v;
        if (w->fam == W_I) v = w->i;
        else if (w->fam == W_U) v = (int64_t)w->u;
        else v = sat_int(as_double(w), bits);
        /* two's-complement wrap to the target width */
        if (dt == C_I64) { memcpy(p, &v, 8); }
        else if (dt == C_I32) { int32_t t = (int32_t)(uint32_t)(uint64_t)v; memcpy(p, &t, 4); }
        else if (dt == C_I16) { int16_t t = (int16_t)(uint16_t)(uint64_t)v; memcpy(p, &t, 2); }
        else { int8_t t = (int8_t)(uint8_t)(uint64_t)v; memcpy(p, &t, 1); }
        break;
    }
    case C_U8: {
        uint8_t t;
        if (w->fam == W_I) t = (uint8_t)(uint64_t)w->i;
        else if (w->fam == W_U) t = (uint8_t)w->u;
        else {
            double v = as_double(w);
            t = !(v > 0.0) ? 0 : v >= 255.0 ? 255 : (uint8_t)v;
        }
        p[0] = t;
        break;
    }
    case C_F8E4M3FN: case C_F8E5M2: p[0] = oracle_f8_encode(dt, as_float(w)); break;
    default: p[0] = (unsigned char)is_nonzero(w); break; /* BOOL */
    }
}

/* dst[i] = castValue(src[i]) for i < n, both arrays dense. */
int oracle_cast(int sdt, const void* src, int ddt, void* dst, int64_t n) {
    if (sdt < C_F32 || sdt > C_F8E5M2 || ddt < C_F32 || ddt > C_F8E5M2) return 1;
    const unsigned char* s = (const unsigned char*)src;
    unsigned char* d = (unsigned char*)dst;
    int ss = elem_size(sdt), ds = elem_size(ddt);
    for (int64_t i = 0; i < n; ++i) {
        wide_t w = widen(sdt, s + i * ss);
        if (sdt == C_BOOL || ddt == C_BOOL) {
            int nz = is_nonzero(&w);
            memset(&w, 0, sizeof(w));
            w.fam = W_I;
            w.i = nz;
        }
        narrow(ddt, &w, d + i * ds);
    }
    return 0;
}
