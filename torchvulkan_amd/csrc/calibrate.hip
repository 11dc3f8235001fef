// Measurement aid: the sustained float16 MFMA rate of this device with data
// that toggles like a GEMM's (tvk_calibrate_mfma). The dense-peak figure
// (2.5 PFLOP/s) assumes operands that barely toggle; with random operands the
// part is power-limited, and that lower ceiling is what a GEMM's MFMA pipe
// can reach at all. The GEMM kernels' roofline reports carry both.
//
// Kernel: every wave holds four pairs of random float16 A/B fragments
// (uniform in [-1, 1), from a per-lane hash) and issues
// v_mfma_f32_16x16x32_f16 in a loop over eight independent accumulators,
// cycling through the fragment pairs so consecutive MFMAs see different
// operands. No memory traffic inside the loop; the accumulators are summed
// and stored at the end so nothing is removed. A grid of 256 CUs x 4 SIMDs x
// `waves_per_simd` waves (`waves_per_simd` workgroups of 256 threads per CU),
// timed with HIP events around the launch.
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

__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int iterations, float* out) {
    const uint32_t id = blockIdx.x * 256u + threadIdx.x;
    half8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = rand_frag(id * 16u + (uint32_t)i);
        b[i] = rand_frag(id * 16u + 8u + (uint32_t)i);
    }
    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // four steps a trip, so every fragment index is a constant (the fragments
    // stay in registers)
    for (int it = 0; it < iterations; it += 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j % 4], b[(j + r) % 4], acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    out[id] = s;
}

}  // namespace
}  // namespace tvk

using namespace tvk;

extern "C" tvk_status tvk_calibrate_mfma(int device, int waves_per_simd, int iterations, double* tflops, double* ms) {
    if (!tflops || !ms) return fail(TVK_ERR_INVALID, "tvk_calibrate_mfma: tflops or ms is NULL");
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
        hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(blocks), dim3(256), 0, s, iterations / 8 + 4, out);   // warm-up
        if (hipEventRecord(e0, s) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_mfma: event record failed"); break; }
        hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(blocks), dim3(256), 0, s, iterations, out);
        if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) {
            st = fail(TVK_ERR_DEVICE, std::string("tvk_calibrate_mfma: ") + hipGetErrorString(hipGetLastError()));
            break;
        }
        float t = 0.0f;
        if (hipEventElapsedTime(&t, e0, e1) != hipSuccess) { st = fail(TVK_ERR_DEVICE, "tvk_calibrate_mfma: elapsed time failed"); break; }
        const double steps = (double)((iterations + 3) / 4 * 4);
        const double flops = (double)blocks * 4.0 * 8.0 * steps * 16.0 * 16.0 * 32.0 * 2.0;
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
