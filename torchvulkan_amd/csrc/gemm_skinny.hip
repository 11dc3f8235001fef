// M <= 16 GEMM as an HBM stream over B (the decode-like shapes of the path:
// C5 "skinny" [16,4096]x[4096,14336] and small-batch linears).
//
// With M <= 16 the product is bound by reading B once: 2*K*N bytes against
// 2*M*K*N flops. A workgroup owns CW (64) columns, one 128-byte line of each
// row of B, and all of K; its eight waves take 64-row blocks of K in turn and
// reduce their partial sums in LDS at the end, so no
// workgroup ever waits for another (a cross-XCD handoff would need an L2
// write-back per workgroup). Per 32 k a wave issues v_mfma_f32_16x16x32 per 16
// columns against the 16 rows of A. B stored k-contiguous ([N][K], a transposed
// weight view) is loaded straight into MFMA operands; B stored n-contiguous
// ([K][N]) is written to a wave-private LDS tile as it arrives and read back
// along k.
//
// Epilogue semantics are the reference's (src/shaders/helpers/gemm_simd.slang:67-99).
#include "gemm_common.h"

namespace tvk {
namespace {

constexpr int SK_NW = 8;      // waves per workgroup (K split over them)
constexpr int SK_CW = 64;     // columns per workgroup: 128-byte rows of B
constexpr int SK_NG = SK_CW / 16;
constexpr int SK_KSTEP = 32;  // k per MFMA
constexpr int SK_U = 2;       // k steps per wave iteration
constexpr int SK_KI = SK_U * SK_KSTEP;
constexpr int SK_LDW = SK_CW + 8;  // LDS row (halfs) of the [k][col] transpose tile

template <int DT>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int DT, bool BKM, bool VEC>
__global__ __launch_bounds__(64 * SK_NW) void gemm_skinny_kernel(GemmArgs p) {
    constexpr int TILE_H = SK_KI * SK_LDW;              // halfs per wave
    constexpr int RED_F = SK_NW * 16 * (SK_CW + 4);     // floats
    constexpr int TILE_BYTES = BKM ? 0 : SK_NW * TILE_H * 2;
    constexpr int BYTES = TILE_BYTES > RED_F * 4 ? TILE_BYTES : RED_F * 4;
    __shared__ __attribute__((aligned(16))) unsigned char smem[BYTES];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    // strips are dealt to the 8 XCDs round robin by block id: give each XCD a
    // contiguous run of strips (neighbouring strips share DRAM rows of B)
    int strip = blockIdx.x;
    if (gridDim.x % 8 == 0) strip = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
    const int n0 = strip * SK_CW, b = blockIdx.z;

    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a) + (int64_t)b * p.sa[0];
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.b) + (int64_t)b * p.sb[0];
    const int64_t a_bytes = 2 * ((int64_t)(p.M - 1) * p.sa[1] + (int64_t)(p.K - 1) * p.sa[2] + 1);
    const int64_t b_bytes = 2 * ((int64_t)(p.N - 1) * p.sb[2] + (int64_t)(p.K - 1) * p.sb[1] + 1);
    __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)min(a_bytes, (int64_t)0x7fffffff), 0x00020000);
    __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)B, 0, (int)min(b_bytes, (int64_t)0x7fffffff), 0x00020000);

    const int j = lane % 16, g = lane / 16;
    // n-contiguous B: lane loads 8 columns (chunk lane%8) of rows lane/8 + 8q
    const int tc = (lane % 8) * 8, tr = lane / 8;
    uint16_t* tile = reinterpret_cast<uint16_t*>(smem) + wave * TILE_H;

    f32x4 acc[SK_NG];
#pragma unroll
    for (int e = 0; e < SK_NG; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // The waves of the workgroup take 64-row blocks of B in turn (block
    // wave, wave+8, ...), so at any time they sweep neighbouring rows
    // together. The loads of a wave's next block are in flight while the
    // current one is transposed and multiplied (two register sets).
    u32x4 av[2][SK_U], bv[2][SK_U][SK_NG];
    auto issue = [&](int set, int k0) {
#pragma unroll
        for (int u = 0; u < SK_U; ++u) {
            const int kk = k0 + u * SK_KSTEP + g * 8;
            av[set][u] = load_chunk<VEC>(ra, j < p.M, (int64_t)j * p.sa[1] + (int64_t)kk * p.sa[2], p.sa[2], p.K - kk);
            if constexpr (BKM) {
#pragma unroll
                for (int e = 0; e < SK_NG; ++e) {
                    const int n = n0 + 16 * e + j;
                    bv[set][u][e] = load_chunk<VEC>(rb, n < p.N, (int64_t)n * p.sb[2] + (int64_t)kk * p.sb[1], p.sb[1], p.K - kk);
                }
            } else {
                const int n = n0 + tc;
#pragma unroll
                for (int q = 0; q < SK_NG; ++q) {
                    const int kr = k0 + u * SK_KSTEP + tr + 8 * q;
                    bv[set][u][q] = load_chunk<VEC>(rb, kr < p.K, (int64_t)kr * p.sb[1] + (int64_t)n * p.sb[2], p.sb[2], p.N - n);
                }
            }
        }
    };
    auto consume = [&](int set) {
        if constexpr (!BKM) {
            // rows arrive n-contiguous: park them in the wave's [k][col] tile,
            // then gather 8 k of one column per lane
#pragma unroll
            for (int u = 0; u < SK_U; ++u)
#pragma unroll
                for (int q = 0; q < SK_NG; ++q)
                    *reinterpret_cast<u32x4*>(tile + (u * SK_KSTEP + tr + 8 * q) * SK_LDW + tc) = bv[set][u][q];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < SK_U; ++u)
#pragma unroll
                for (int e = 0; e < SK_NG; ++e) {
                    const uint16_t* src = tile + (u * SK_KSTEP + g * 8) * SK_LDW + 16 * e + j;
                    uint32_t h[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) h[i] = src[i * SK_LDW];
                    bv[set][u][e] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
                }
            __builtin_amdgcn_wave_barrier();
        }
#pragma unroll
        for (int u = 0; u < SK_U; ++u)
#pragma unroll
            for (int e = 0; e < SK_NG; ++e) acc[e] = mfma16<DT>(av[set][u], bv[set][u][e], acc[e]);
    };
    const int kstride = SK_NW * SK_KI;
    int k0 = wave * SK_KI;
    if (k0 < p.K) issue(0, k0);
    while (k0 < p.K) {
        if (k0 + kstride < p.K) issue(1, k0 + kstride);
        consume(0);
        k0 += kstride;
        if (k0 >= p.K) break;
        if (k0 + kstride < p.K) issue(0, k0 + kstride);
        consume(1);
        k0 += kstride;
    }

    // reduce the waves' partial sums (16x16 accumulator layout: lane holds
    // column lane%16, rows (lane/16)*4 + r)
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int e = 0; e < SK_NG; ++e)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * 16 + g * 4 + r) * (SK_CW + 4) + 16 * e + j] = acc[e][r];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < (16 * SK_CW) / (64 * SK_NW); ++q) {
        const int idx = tid + 64 * SK_NW * q;
        const int m = idx / SK_CW, cl = idx % SK_CW;
        float v = red[m * (SK_CW + 4) + cl];
#pragma unroll
        for (int w = 1; w < SK_NW; ++w) v += red[(w * 16 + m) * (SK_CW + 4) + cl];
        const int n = n0 + cl;
        if (m < p.M && n < p.N) store_out<DT>(p, b, m, n, v);
    }
}

}  // namespace

bool skinny_applies(int64_t M, int64_t N, int64_t K, int64_t batch) {
    return M >= 1 && M <= 16 && N >= 64 && K >= 64 && batch <= 65535;
}

const char* skinny_name(bool b_kmajor) { return b_kmajor ? "gemm16_skinny_bk" : "gemm16_skinny_bn"; }

hipError_t launch_skinny(int dtype, const GemmArgs& p, bool b_kmajor, bool vec, hipStream_t s) {
    const int strips = (p.N + SK_CW - 1) / SK_CW;
    dim3 grid(strips, 1, p.batch);
#define TVK_SK(D, BKM, V) hipLaunchKernelGGL((gemm_skinny_kernel<D, BKM, V>), grid, dim3(64 * SK_NW), 0, s, p)
    if (dtype == TVK_F16) {
        if (b_kmajor) { if (vec) TVK_SK(TVK_F16, true, true); else TVK_SK(TVK_F16, true, false); }
        else { if (vec) TVK_SK(TVK_F16, false, true); else TVK_SK(TVK_F16, false, false); }
    } else {
        if (b_kmajor) { if (vec) TVK_SK(TVK_BF16, true, true); else TVK_SK(TVK_BF16, true, false); }
        else { if (vec) TVK_SK(TVK_BF16, false, true); else TVK_SK(TVK_BF16, false, false); }
    }
#undef TVK_SK
    return hipGetLastError();
}

}  // namespace tvk
