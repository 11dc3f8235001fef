// Element conversion between every tvk_dtype, shared by the copy, reduce and
// element-wise kernels: the reference's castValue
// (src/shaders/core/cast.slang:49-52, src/shaders/core/dtype.slang:122-282).
// The source widens to int64 (signed integers), uint64 (U8, BOOL), float
// (F16, BF16, F32) or double (F64); the destination is built from that one
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

__host__ __device__ constexpr int family(int dt) {
    return dt == TVK_F64 ? FAM_D
         : (dt == TVK_F32 || dt == TVK_F16 || dt == TVK_BF16) ? FAM_F
         : (dt == TVK_U8 || dt == TVK_BOOL) ? FAM_U
         : FAM_I;
}

struct Wide {
    int64_t i;
    uint64_t u;
    float f;
    double d;
};

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
