// Measurement aids (no counterpart in the reference).
//
// tvk_calibrate_mfma: the sustained float16 MFMA rate of this device with data
// that toggles like a GEMM's (tvk_calibrate_mfma). The dense-peak figure
// (2.5 PFLOP/s) assumes operands that barely toggle; with random operands the
// part is power-limited, and that lower ceiling is what a GEMM's MFMA pipe
// can reach at all. The GEMM kernels' roofline reports carry both.
//
// Kernel: every wave holds four pairs of float16 A/B fragments (random:
// uniform in [-1, 1) from a per-lane hash; or all zeros, the operands that
// toggle nothing) and issues v_mfma_f32_16x16x32_f16 over sixteen independent
// accumulators, 64 MFMAs per loop trip (one scalar add, compare and branch per
// 64 MFMAs), cycling through the fragment pairs so consecutive MFMAs see
// different operands. No memory traffic inside the loop; the accumulators are
// summed and stored at the end so nothing is removed. A grid of 256 CUs x 4
// SIMDs x `waves_per_simd` waves (`waves_per_simd` workgroups of 256 threads
// per CU), timed with HIP events around the launch. Random against zero
// operands separates the pipe's issue limit from the part's power limit.
//
// tvk_calibrate_hbm: the read bandwidth a plain streaming kernel reaches, the
// practical ceiling of an HBM-bound kernel that reads each byte once (the
// M <= 16 GEMM streaming B). Three windows of `window_bytes` are read in
// rotation, one a launch, so that with windows above ~90 MB the window read
// next has left the 256 MB Infinity Cache since it was last read (the same
// rotation the skinny-GEMM benchmark uses for its B operands). Kernel: 512
// workgroups of 256 threads (two a CU), each thread four 16-byte loads in
// flight, grid-strided; the loaded words are folded into one value that is
// stored only if it matches a constant, so nothing is removed.
#include "tvk_common.h"

#include <string>

namespace tvk {
namespace {

__device__ inline uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// eight float16 values uniform in [-1, 1) from a seed
__device__ inline half8 rand_frag(uint32_t seed) {
    half8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t r = mix32(seed * 8u + (uint32_t)i);
        v[i] = (_Float16)((float)(r >> 8) * (2.0f / 16777216.0f) - 1.0f);
    }
    return v;
}

__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int iterations, int zeros, float* out) {
    const uint32_t id = blockIdx.x * 256u + threadIdx.x;
    half8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = rand_frag(id * 16u + (uint32_t)i);
        b[i] = rand_frag(id * 16u + 8u + (uint32_t)i);
        if (zeros) {
#pragma unroll
            for (int e = 0; e < 8; ++e) a[i][e] = b[i][e] = (_Float16)0.0f;
        }
    }
    f32x4 acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // 64 MFMAs a trip, four per accumulator; every fragment index is a
    // constant, so the fragments stay in registers
    for (int it = 0; it < iterations; it += 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j % 4], b[(j / 4 + r) % 4], acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    out[id] = s;
}

// The same flops a trip on v_mfma_f32_32x32x16_f16: 32 MFMAs over eight
// 32x32 accumulators (the larger instruction reads half the A/B register
// bytes per flop; whether that buys clock under the power limit is what this
// form measures).
__global__ __launch_bounds__(256) void mfma32_ceiling_kernel(int iterations, int zeros, float* out) {
    const uint32_t id = blockIdx.x * 256u + threadIdx.x;
    half8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = rand_frag(id * 16u + (uint32_t)i);
        b[i] = rand_frag(id * 16u + 8u + (uint32_t)i);
        if (zeros) {
#pragma unroll
            for (int e = 0; e < 8; ++e) a[i][e] = b[i][e] = (_Float16)0.0f;
        }
    }
    f32x16 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    for (int it = 0; it < iterations; it += 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j % 4], b[(j / 4 + r) % 4], acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    out[id] = s;
}

__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* p, int64_t n16, uint32_t* out) {
    uint32_t acc = 0;
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= a.x ^ b.y ^ c.z ^ d.w;
    }
    for (; i < n16; i += stride) acc ^= p[i].x;
    if (acc == 0x9e3779b9u) out[0] = acc;
}

}  // namespace
}  // namespace tvk

using namespace tvk;

extern "C" tvk_status tvk_calibrate_hbm(int device, size_t window_bytes, int iterations, double* gbps, double* ms) {
    if (!gbps || !ms) return fail(TVK_ERR_INVALID, "tvk_calibrate_hbm: gbps or ms is NULL");
    if (window_bytes < 4096 || window_bytes % 16 != 0 || window_bytes > (size_t(8) << 30) || iterations < 1)
        return fail(TVK_ERR_INVALID, "tvk_calibrate_hbm: window_bytes must be a multiple of 16 in [4 KiB, 8 GiB] and iterations positive");
    int cur = 0;
    TVK_HIP_CHECK(hipGetDevice(&cur));
    TVK_HIP_CHECK(hipSetDevice(device));
    tvk_status st = TVK_OK;
    char* buf = nullptr;
    uint32_t* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipStream_t s = nullptr;
    do {
        if (hipMalloc(&buf, 3 * window_bytes) != hipSuccess || hipMalloc(&out, 16) != hipSuccess) {
            st = fail(TVK_ERR_OOM, "tvk_calibrate_hbm: out of memory");
            break;
        }
        if (hipStreamCreate(&s) != hipSuccess || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
            st = fail(TVK_ERR_DEVICE, "tvk_calibrate_hbm: stream or event creation failed");
            break;
        }
        if (hipMemsetAsync(buf, 0x3c, 3 * window_bytes, s) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_hbm: fill failed"); break; }
        const int64_t n16 = (int64_t)(window_bytes / 16);
        auto window = [&](int i) { return reinterpret_cast<const u32x4*>(buf + (size_t)(i % 3) * window_bytes); };
        for (int i = 0; i < 6; ++i) hipLaunchKernelGGL(hbm_read_kernel, dim3(512), dim3(256), 0, s, window(i), n16, out);   // warm-up
        if (hipEventRecord(e0, s) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_hbm: event record failed"); break; }
        for (int i = 0; i < iterations; ++i) hipLaunchKernelGGL(hbm_read_kernel, dim3(512), dim3(256), 0, s, window(i), n16, out);
        if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) {
            st = fail(TVK_ERR_DEVICE, std::string("tvk_calibrate_hbm: ") + hipGetErrorString(hipGetLastError()));
            break;
        }
        float t = 0.0f;
        if (hipEventElapsedTime(&t, e0, e1) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_hbm: elapsed time failed"); break; }
        *ms = t / iterations;
        *gbps = (double)window_bytes / ((double)*ms * 1e-3) / 1e9;
    } while (false);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) {
        (void)hipStreamSynchronize(s);
        (void)hipStreamDestroy(s);
    }
    if (out) (void)hipFree(out);
    if (buf) (void)hipFree(buf);
    (void)hipSetDevice(cur);
    return st;
}

extern "C" tvk_status tvk_calibrate_mfma_operands(int device, int waves_per_simd, int iterations, int operands, double* tflops,
                                                  double* ms) {
    if (!tflops || !ms) return fail(TVK_ERR_INVALID, "tvk_calibrate_mfma: tflops or ms is NULL");
    if (operands < 0 || operands > 3)
        return fail(TVK_ERR_INVALID, "tvk_calibrate_mfma: operands must be 0 (random) or 1 (zeros), +2 for the 32x32x16 form");
    if (waves_per_simd < 1 || waves_per_simd > 4 || iterations < 1)
        return fail(TVK_ERR_INVALID, "tvk_calibrate_mfma: waves_per_simd must be 1..4 and iterations positive");
    int cur = 0;
    TVK_HIP_CHECK(hipGetDevice(&cur));
    TVK_HIP_CHECK(hipSetDevice(device));
    hipDeviceProp_t prop;
    tvk_status st = TVK_OK;
    float* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipStream_t s = nullptr;
    do {
        if (hipGetDeviceProperties(&prop, device) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_mfma: no device properties"); break; }
        const int blocks = prop.multiProcessorCount * waves_per_simd;   // 4 waves a workgroup: one per SIMD
        if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) { st = fail(TVK_ERR_OOM, "tvk_calibrate_mfma: out of memory"); break; }
        if (hipStreamCreate(&s) != hipSuccess || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
            st = fail(TVK_ERR_DEVICE, "tvk_calibrate_mfma: stream or event creation failed");
            break;
        }
        auto kern = operands >= 2 ? mfma32_ceiling_kernel : mfma_ceiling_kernel;
        const int zeros = operands & 1;
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, s, iterations / 8 + 4, zeros, out);   // warm-up
        if (hipEventRecord(e0, s) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_mfma: event record failed"); break; }
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, s, iterations, zeros, out);
        if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) {
            st = fail(TVK_ERR_DEVICE, std::string("tvk_calibrate_mfma: ") + hipGetErrorString(hipGetLastError()));
            break;
        }
        float t = 0.0f;
        if (hipEventElapsedTime(&t, e0, e1) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_mfma: elapsed time failed"); break; }
        const double steps = (double)((iterations + 3) / 4 * 4);
        const double flops = (double)blocks * 4.0 * 16.0 * steps * 16.0 * 16.0 * 32.0 * 2.0;
        *ms = t;
        *tflops = flops / ((double)t * 1e-3) / 1e12;
    } while (false);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (out) (void)hipFree(out);
    (void)hipSetDevice(cur);
    return st;
}

extern "C" tvk_status tvk_calibrate_mfma(int device, int waves_per_simd, int iterations, double* tflops, double* ms) {
    return tvk_calibrate_mfma_operands(device, waves_per_simd, iterations, 0, tflops, ms);
}
