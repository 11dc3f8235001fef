// Element conversion between every tvk_dtype, shared by the copy, reduce and
// element-wise kernels: the reference's castValue
// (src/shaders/core/cast.slang:49-52, src/shaders/core/dtype.slang:122-282).
// The source widens to int64 (signed integers), uint64 (U8, BOOL), float
// (F16, BF16, F32, the float8 types) or double (F64); the destination is built from that one
// wide value. With a bool on either side the value is (src != 0) ? 1 : 0
// (src/shaders/ops/cast.slang:29-33).
#pragma once

#include "tvk_common.h"

#include <cmath>
#include <limits>

namespace tvk {

constexpr int kMaxDims = TVK_COPY_MAX_DIMS;
constexpr int DYN = -1;   // dtype taken from the kernel arguments

enum { FAM_I = 0, FAM_U = 1, FAM_F = 2, FAM_D = 3 };

__host__ __device__ constexpr bool is_f8(int dt) { return dt == TVK_F8E4M3FN || dt == TVK_F8E5M2; }

__host__ __device__ constexpr int family(int dt) {
    return dt == TVK_F64 ? FAM_D
         : (dt == TVK_F32 || dt == TVK_F16 || dt == TVK_BF16 || is_f8(dt)) ? FAM_F
         : (dt == TVK_U8 || dt == TVK_BOOL) ? FAM_U
         : FAM_I;
}

struct Wide {
    int64_t i;
    uint64_t u;
    float f;
    double d;
};

// float8 (torch's float8_e4m3fn and float8_e5m2). The reference converts
// them with c10's own routines, through float32 (transfer.cpp:129-226), so
// these match the CPU bit for bit.
//
// Decoding is exact: the code's fields placed into a float32. NaN codes get
// the payload the CPU's conversion gives them: e5m2 goes through float16 on
// the CPU, which widens the payload (m << 21) and sets the quiet bit;
// e4m3fn's single NaN per sign becomes 0x7FF00000.
__device__ __forceinline__ float f8_to_f32(uint8_t c, int dt) {
    const uint32_t sign = (uint32_t)(c & 0x80) << 24;
    uint32_t bits;
    if (dt == TVK_F8E4M3FN) {
        const uint32_t e = (c >> 3) & 15, m = c & 7;
        if (e == 15 && m == 7) bits = 0x7FF00000u;
        else if (e == 0) return __builtin_bit_cast(float, sign | __builtin_bit_cast(uint32_t, (float)m * 0x1p-9f));
        else bits = ((e + 120) << 23) | (m << 20);
    } else {
        const uint32_t e = (c >> 2) & 31, m = c & 3;
        if (e == 31) bits = (m ? 0x7FC00000u : 0x7F800000u) | (m << 21);
        else if (e == 0) return __builtin_bit_cast(float, sign | __builtin_bit_cast(uint32_t, (float)m * 0x1p-16f));
        else bits = ((e + 112) << 23) | (m << 21);
    }
    return __builtin_bit_cast(float, sign | bits);
}

// Encoding: round to nearest even onto the 8-bit grid, on the float's bits
// (integer arithmetic only, so no flush of float32 subnormals can interfere).
//   e4m3fn: |x| >= 480 (NaN and infinities included) is NaN; below that a
//           magnitude rounding past 448 lands on the NaN code 0x7F too.
//   e5m2:   NaN is 0x7F; |x| >= 65536 is infinity; below that a magnitude
//           rounding past 57344 lands on the infinity code 0x7C.
__device__ __forceinline__ uint8_t f32_to_f8(float x, int dt) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
    const uint32_t a = u & 0x7FFFFFFFu;
    const bool e4 = dt == TVK_F8E4M3FN;
    if (e4) {
        if (a >= 0x43F00000u) return sign | 0x7F;
    } else {
        if (a > 0x7F800000u) return sign | 0x7F;
        if (a >= 0x47800000u) return sign | 0x7C;
    }
    const int bias = e4 ? 7 : 15, mb = e4 ? 3 : 2;
    const int e = (int)(a >> 23);
    if (e >= 128 - bias) {   // a normal 8-bit value: rebias, round the mantissa
        const int sh = 23 - mb;
        uint32_t t = a - ((uint32_t)(127 - bias) << 23);
        t += ((1u << (sh - 1)) - 1) + ((t >> sh) & 1);
        return sign | (uint8_t)(t >> sh);
    }
    // subnormal 8-bit range: a / 2^(1 - bias - mb) rounded to an integer
    // (reaching 2^mb gives the smallest normal code, as it should)
    const int s = 151 - bias - mb - e;
    if (e == 0 || s > 24) return sign;   // below half the smallest step
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t q = mant >> s;
    const uint32_t r = mant & ((1u << s) - 1), h = 1u << (s - 1);
    if (r > h || (r == h && (q & 1))) ++q;
    return sign | (uint8_t)q;
}

__device__ __forceinline__ Wide load_wide(const char* p, int dt) {
    Wide w{0, 0, 0.0f, 0.0};
    switch (dt) {
        case TVK_F32: w.f = *reinterpret_cast<const float*>(p); break;
        case TVK_F16: w.f = (float)*reinterpret_cast<const _Float16*>(p); break;
        case TVK_BF16: w.f = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p)); break;
        case TVK_F64: w.d = *reinterpret_cast<const double*>(p); break;
        case TVK_I64: w.i = *reinterpret_cast<const int64_t*>(p); break;
        case TVK_I32: w.i = *reinterpret_cast<const int32_t*>(p); break;
        case TVK_I16: w.i = *reinterpret_cast<const int16_t*>(p); break;
        case TVK_I8: w.i = *reinterpret_cast<const int8_t*>(p); break;
        case TVK_F8E4M3FN: case TVK_F8E5M2: w.f = f8_to_f32(*reinterpret_cast<const uint8_t*>(p), dt); break;
        default: w.u = *reinterpret_cast<const uint8_t*>(p); break;   // U8, BOOL
    }
    return w;
}

__device__ __forceinline__ bool nonzero(const Wide& w, int fam) {
    switch (fam) {
        case FAM_I: return w.i != 0;
        case FAM_U: return w.u != 0;
        case FAM_F: return w.f != 0.0f;   // NaN != 0
        default: return w.d != 0.0;
    }
}

__device__ __forceinline__ float wide_to_f32(const Wide& w, int fam) {
    switch (fam) {
        case FAM_I: return (float)w.i;
        case FAM_U: return (float)w.u;
        case FAM_F: return w.f;
        default: return (float)w.d;
    }
}

__device__ __forceinline__ double wide_to_f64(const Wide& w, int fam) {
    switch (fam) {
        case FAM_I: return (double)w.i;
        case FAM_U: return (double)w.u;
        case FAM_F: return (double)w.f;
        default: return w.d;
    }
}

// float64 -> float16 in one rounding (the reference's half(double)): round to
// odd into float32 (24 bits >= 11 + 2), then round to nearest even into
// float16, which gives the correctly rounded result (Boldo and Melquiond,
// "When double rounding is odd", 2005).
__device__ __forceinline__ _Float16 f64_to_f16(double d) {
    float f = (float)d;
    if (f != f || (double)f == d) return (_Float16)f;
    uint32_t bits = __builtin_bit_cast(uint32_t, f);
    if (fabs((double)f) > fabs(d)) bits -= 1;   // the magnitude went up: one step back toward zero
    bits |= 1u;                                 // inexact: odd last bit
    return (_Float16)__builtin_bit_cast(float, bits);
}

__device__ __forceinline__ _Float16 wide_to_f16(const Wide& w, int fam) {
    if (fam == FAM_D) return f64_to_f16(w.d);
    // integers: exact in float32 up to 2^24, and every larger magnitude is
    // past float16's range either way, so one rounding results
    return (_Float16)wide_to_f32(w, fam);
}

// Float to integer, saturating at the target's range, NaN -> 0 (out of range
// is undefined in the reference; in range this is truncation toward zero).
template <typename I>
__device__ __forceinline__ I float_to_int(double v) {
    constexpr double lo = (double)std::numeric_limits<I>::min();   // -2^(bits-1), exact in double
    if (v != v) return 0;
    if (v <= lo) return std::numeric_limits<I>::min();
    if (v >= -lo) return std::numeric_limits<I>::max();
    return (I)v;
}

template <typename I>
__device__ __forceinline__ I wide_to_int(const Wide& w, int fam) {
    switch (fam) {
        case FAM_I: return (I)w.i;
        case FAM_U: return (I)w.u;
        case FAM_F: return float_to_int<I>((double)w.f);
        default: return float_to_int<I>(w.d);
    }
}

__device__ __forceinline__ uint8_t wide_to_u8(const Wide& w, int fam) {
    switch (fam) {
        case FAM_I: return (uint8_t)w.i;
        case FAM_U: return (uint8_t)w.u;
        default: {
            const double v = fam == FAM_F ? (double)w.f : w.d;
            if (!(v > 0.0)) return 0;
            if (v >= 255.0) return 255;
            return (uint8_t)v;
        }
    }
}

__device__ __forceinline__ void store_narrow(char* p, int dt, const Wide& w, int fam) {
    switch (dt) {
        case TVK_F32: *reinterpret_cast<float*>(p) = wide_to_f32(w, fam); break;
        case TVK_F16: *reinterpret_cast<_Float16*>(p) = wide_to_f16(w, fam); break;
        case TVK_BF16: *reinterpret_cast<uint16_t*>(p) = f32_to_bf16_bits(wide_to_f32(w, fam)); break;
        case TVK_F64: *reinterpret_cast<double*>(p) = wide_to_f64(w, fam); break;
        case TVK_I64: *reinterpret_cast<int64_t*>(p) = wide_to_int<int64_t>(w, fam); break;
        case TVK_I32: *reinterpret_cast<int32_t*>(p) = wide_to_int<int32_t>(w, fam); break;
        case TVK_I16: *reinterpret_cast<int16_t*>(p) = wide_to_int<int16_t>(w, fam); break;
        case TVK_I8: *reinterpret_cast<int8_t*>(p) = wide_to_int<int8_t>(w, fam); break;
        case TVK_U8: *reinterpret_cast<uint8_t*>(p) = wide_to_u8(w, fam); break;
        case TVK_F8E4M3FN: case TVK_F8E5M2: *reinterpret_cast<uint8_t*>(p) = f32_to_f8(wide_to_f32(w, fam), dt); break;
        default: *reinterpret_cast<uint8_t*>(p) = nonzero(w, fam) ? 1 : 0; break;   // BOOL
    }
}

// dst = castValue<Src, Dst>(src). With compile-time dtypes every switch folds.
__device__ __forceinline__ void convert(const char* sp, int sdt, char* dp, int ddt) {
    Wide w = load_wide(sp, sdt);
    int fam = family(sdt);
    if (sdt == TVK_BOOL || ddt == TVK_BOOL) {
        w.i = nonzero(w, fam) ? 1 : 0;
        fam = FAM_I;
    }
    store_narrow(dp, ddt, w, fam);
}

template <int SDT, int DDT>
struct Dts {
    int s, d;
    __device__ __forceinline__ Dts(int rs, int rd) : s(SDT == DYN ? rs : SDT), d(DDT == DYN ? rd : DDT) {}
};

// Division by a runtime constant: q = (hi32(n * m) + n) >> s (exact for every
// 32-bit n; the sum is taken in 64 bits).
struct Div32 {
    uint32_t d, m, s;
};

inline Div32 make_div(uint32_t d) {
    Div32 r{d, 0, 0};
    uint32_t s = 0;
    while (s < 32 && (uint64_t(1) << s) < d) ++s;
    r.s = s;
    r.m = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
    return r;
}

__device__ __forceinline__ uint32_t div32(uint32_t n, const Div32& v) {
    const uint32_t t = __umulhi(n, v.m);
    return (uint32_t)(((uint64_t)t + n) >> v.s);
}

}  // namespace tvk
