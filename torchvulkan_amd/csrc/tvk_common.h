// Shared definitions of the gfx950 dense-contraction library: status/error
// plumbing, element types and the float32 <-> float16/bfloat16 conversions the
// kernels and the host agree on.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/tvk_hip.h"

namespace tvk {

// Thread-local last error (tvk_last_error).
void set_error(const std::string& msg);
void clear_error();

inline tvk_status fail(tvk_status code, const std::string& msg) {
    set_error(msg);
    return code;
}

#define TVK_HIP_CHECK(expr)                                                      \
    do {                                                                         \
        hipError_t _e = (expr);                                                  \
        if (_e != hipSuccess)                                                    \
            return ::tvk::fail(TVK_ERR_DEVICE, std::string(#expr " failed: ") +  \
                                                   hipGetErrorString(_e));       \
    } while (0)

// Library stream of a device (created lazily); defined in runtime.hip.
hipStream_t device_stream(int device);

// A lease of library scratch memory (split-K partials, repacked operands,
// convolution partials) for the kernels one call queues on one stream of the
// current device. The lease ends when the object is destroyed, after the
// call's launches. A buffer is only ever leased again for the same stream, so
// stream order puts this call's kernels before the next holder's; buffers are
// freed only after the device has drained, never while a lease holds them
// (scratch_pool.h).
class Scratch {
public:
    Scratch() = default;
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    ~Scratch() { release(); }
    // At least `bytes` of device memory, 256-byte aligned, for kernels queued
    // on `stream`; NULL when it cannot be allocated. One lease per object: a
    // second call ends the first lease.
    void* get(size_t bytes, hipStream_t stream);
    void release();

private:
    void* lease_ = nullptr;
    int device_ = -1;
    hipStream_t stream_ = nullptr;
};

// Split-K tile counters for kernels queued on `stream` of the current device:
// `count` words, zero now and left zero by every kernel that uses them (the
// last workgroup of a tile resets its counter). One array per stream, so
// stream order alone separates two launches' use of it; allocated and zeroed
// on the stream at its first use and kept until the process ends. NULL when
// count exceeds the array, the allocation fails, or the stream is being
// captured before its first use (callers then reduce in a second launch).
unsigned* split_counters(hipStream_t stream, int64_t count);

// A NULL stream handle is HIP's default (null) stream, as in every HIP library.
inline hipStream_t resolve_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ constexpr size_t dtype_size(int32_t dt) {
    switch (dt) {
        case TVK_F64: case TVK_I64: return 8;
        case TVK_F32: case TVK_I32: return 4;
        case TVK_F16: case TVK_BF16: case TVK_I16: return 2;
        default: return 1;   // I8, U8, BOOL
    }
}

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Store of a kernel result that the kernel itself does not read back:
// non-temporal, so the line streams through the L2 instead of staying there
// dirty, which leaves the end-of-kernel write-back less to do (measured 1.3 us
// off a 17 us stride-1 convolution launch whose output is 16.8 MB).
template <class V>
__device__ inline void st_nt(V* p, V v) { __builtin_nontemporal_store(v, p); }
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element storage as raw 16-bit patterns for the 16-bit types.
struct bf16_raw { uint16_t bits; };

// float32 -> bfloat16, round to nearest even; NaN stays a quiet NaN. This is
// the same rounding c10::BFloat16's float constructor performs.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// Element type traits used by the kernels: load as float, store from float.
template <int DT> struct elem;
template <> struct elem<TVK_F32> {
    typedef float T;
    __device__ static inline float to_f32(T v) { return v; }
    __device__ static inline T from_f32(float v) { return v; }
};
template <> struct elem<TVK_F16> {
    typedef half_t T;
    __device__ static inline float to_f32(T v) { return (float)v; }
    __device__ static inline T from_f32(float v) { return (half_t)v; }  // v_cvt_f16_f32: RNE
};
template <> struct elem<TVK_BF16> {
    typedef uint16_t T;
    __device__ static inline float to_f32(T v) { return bf16_bits_to_f32(v); }
    __device__ static inline T from_f32(float v) { return f32_to_bf16_bits(v); }
};

}  // namespace tvk
