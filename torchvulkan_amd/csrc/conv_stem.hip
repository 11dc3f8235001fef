// 2-D convolution on gfx950 for few input channels (a network's stem: 3
// colour channels, 3x3 taps), float16/bfloat16, groups == 1. The channel-rich
// kernels stage 32-channel k stages of a channels-last copy; with 3 channels a
// whole reduction is one 32-k MFMA step (c, kh, kw <= 32 values), so these
// kernels gather straight from NCHW and skip the copy:
//   forward     y[p][co] = sum_k patch(x, p)[k] * W[co][k]: one 16x16x32 MFMA
//               per 16x16 output block, k = (c, kh, kw) zero-filled past K;
//               y written NCHW through an LDS tile (16-byte stores)
//   grad weight dW[co][k] = sum_p dy[co][p] * patch(x, p)[k]: the pixels are
//               the reduction, 32 a step; dy rows are the A operand read as
//               16-byte loads, the x patches the B operand; float32 partials
//               per workgroup, summed in workgroup order by a second kernel
//   grad input  (stride 1, 3x3, dilation 1, at most 4 input channels)
//               dx[c][i] = sum_{co,t} dy[co][i + off(t)] * W[co][c][t] with
//               v_dot2 over output-channel pairs: a workgroup stages a halo of
//               dy rows (channel pairs interleaved) in LDS and each thread sums
//               one input pixel for every input channel
//
// Reference semantics (file:line under the reference tree): the sums of
// src/shaders/helpers/conv.slang:198-511 and src/api/ops/conv.cpp:1014-1060
// (the same as conv.hip's kernels) with another k order inside each output's
// reduction, which the float16/bfloat16 tolerance allows; bias is added in
// float32 before the one rounding (src/shaders/conv_simd.slang:8-19).
#include "tvk_common.h"
#include "gemm_common.h"

#include <algorithm>
#include <cstring>
#include <string>

namespace tvk {
namespace {

struct SmallArgs {
    const void* x;
    const void* w;
    const void* bias;
    const void* dy;
    void* out;        // y (forward), dx (grad input), dW or nothing (grad weight with partials)
    float* part;      // grad weight: [split][cout * K]
    int n, cin, H, W, cout, kh, kw, sh, sw, ph, pw, dh, dw, Ho, Wo;
    int K;            // cin * kh * kw (<= 32)
    int M;            // forward: output pixels n * Ho * Wo
    int split;        // grad weight: workgroups along the pixels (partials when > 1)
    int has_bias;
    int vec_out;      // forward: Ho * Wo % 8 == 0 and y 16-byte aligned
    // grad input tile: TR input rows a workgroup, halo HR x HC, ncp output-channel pairs
    int tr, hr, hc, ncp, row_blocks;
};

constexpr int S_CP = 16;   // grad input: output-channel pairs per LDS chunk

template <int DT>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ inline u32x4 pack8(const uint16_t (&v)[8]) {
    return u32x4{v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16), v[4] | ((uint32_t)v[5] << 16),
                 v[6] | ((uint32_t)v[7] << 16)};
}

// k -> (channel plane offset, row tap offset, column tap offset); plane -1 past K
__device__ inline void fill_ktab(const SmallArgs& p, int (*ktab)[32]) {
    const int k = threadIdx.x;
    if (k >= 32) return;
    const int T = p.kh * p.kw;
    if (k < p.K) {
        const int c = k / T, t = k - c * T, a = t / p.kw, b = t - a * p.kw;
        ktab[0][k] = c * p.H * p.W;
        ktab[1][k] = a * p.dh;
        ktab[2][k] = b * p.dw;
    } else {
        ktab[0][k] = -1;
        ktab[1][k] = 0;
        ktab[2][k] = 0;
    }
}

// One 256-pixel x 64-channel output tile: 4 waves of 64 pixels, 4x4 MFMAs each.
template <int DT>
__global__ __launch_bounds__(256) void conv_small_fwd_kernel(SmallArgs p) {
    typedef typename elem<DT>::T T;
    constexpr int LROW = 256 + 8;
    __shared__ int ktab[3][32];
    __shared__ __attribute__((aligned(16))) uint16_t tile[64 * LROW];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16;
    const int m0 = blockIdx.x * 256, n0 = blockIdx.y * 64;
    const int HW = p.H * p.W, HWo = p.Ho * p.Wo;
    fill_ktab(p, ktab);
    __syncthreads();
    int kc[8], ka[8], kb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        kc[e] = ktab[0][g * 8 + e];
        ka[e] = ktab[1][g * 8 + e];
        kb[e] = ktab[2][g * 8 + e];
    }
    const uint16_t* x = static_cast<const uint16_t*>(p.x);
    const uint16_t* w = static_cast<const uint16_t*>(p.w);
    // B: W[co][k] is the NCHW weight itself ([co][c][kh][kw] = [co][K])
    u32x4 fb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int co = n0 + j * 16 + lane % 16;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int k = g * 8 + e;
            v[e] = (co < p.cout && k < p.K) ? w[co * p.K + k] : (uint16_t)0;
        }
        fb[j] = pack8(v);
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // rows past M gather a valid pixel; they are never stored
        const int m = min(m0 + wave * 64 + i * 16 + lane % 16, p.M - 1);
        const int img = m / HWo, o = m - img * HWo;
        const int oh = o / p.Wo, ow = o - oh * p.Wo;
        const int ih0 = oh * p.sh - p.ph, iw0 = ow * p.sw - p.pw;
        const uint16_t* xb = x + img * p.cin * HW;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int ih = ih0 + ka[e], iw = iw0 + kb[e];
            v[e] = (kc[e] >= 0 && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W) ? xb[kc[e] + ih * p.W + iw]
                                                                                                  : (uint16_t)0;
        }
        const u32x4 fa = pack8(v);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<DT>(fa, fb[j], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    }
    // [channel][pixel] tile, then 16-byte stores along each channel plane
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ch = j * 16 + lane % 16;
        float bv = 0.0f;
        if (p.has_bias && n0 + ch < p.cout) bv = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[n0 + ch]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint16_t h[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[i][j][r];
                if (p.has_bias) {
#pragma clang fp contract(off)
                    v = v + bv;
                }
                h[r] = __builtin_bit_cast(uint16_t, elem<DT>::from_f32(v));
            }
            const int px = wave * 64 + i * 16 + g * 4;
            *reinterpret_cast<u32x2*>(tile + ch * LROW + px) = u32x2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
        }
    }
    __syncthreads();
    uint16_t* y = static_cast<uint16_t*>(p.out);
    for (int idx = tid; idx < 64 * 32; idx += 256) {
        const int ch = idx / 32, pc = idx % 32;
        const int co = n0 + ch, pix = m0 + pc * 8;
        if (co >= p.cout || pix >= p.M) continue;
        const uint16_t* src = tile + ch * LROW + pc * 8;
        if (p.vec_out) {
            // 8 pixels of one image (Ho * Wo % 8 == 0): one 16-byte store
            const int img = pix / HWo, o = pix - img * HWo;
            st_nt(reinterpret_cast<u32x4*>(y + ((int64_t)img * p.cout + co) * HWo + o), *reinterpret_cast<const u32x4*>(src));
        } else {
            for (int e = 0; e < 8 && pix + e < p.M; ++e) {
                const int img = (pix + e) / HWo, o = pix + e - img * HWo;
                y[((int64_t)img * p.cout + co) * HWo + o] = src[e];
            }
        }
    }
}

// Forward, stride 1, dilation 1, output width Wo in 8..256 dividing 256: a
// workgroup computes TR = 256 / Wo whole output rows of one image x 64
// output channels. The input rows it reads (with zeros for the padding) and
// the weight block go to LDS with coalesced loads first, so the patch gather
// is 8 LDS reads a fragment and needs no bounds checks. LDS: x as
// [c][TR + kh - 1][W + 16] (image column iw at iw + 8), weights as [64][40]
// (80-byte rows: the 16 lanes of a fragment read hit distinct banks).
template <int DT>
__global__ __launch_bounds__(256) void conv_small_fwd_rows_kernel(SmallArgs p) {
    typedef typename elem<DT>::T T;
    constexpr int LROW = 256 + 8, WROW = 40;
    __shared__ int ktab[32];
    __shared__ __attribute__((aligned(16))) uint16_t ws[64 * WROW];
    __shared__ __attribute__((aligned(16))) uint16_t xs[8192];
    __shared__ __attribute__((aligned(16))) uint16_t tile[64 * LROW];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, sl = lane % 16;
    const int TR = 256 / p.Wo;
    const int rt = blockIdx.x % p.row_blocks, img = blockIdx.x / p.row_blocks;
    const int h0 = rt * TR, n0 = blockIdx.y * 64;
    const int HR = TR + p.kh - 1, RP = p.W + 16, taps = p.kh * p.kw;
    const uint16_t* x = static_cast<const uint16_t*>(p.x) + (int64_t)img * p.cin * p.H * p.W;
    const uint16_t* w = static_cast<const uint16_t*>(p.w);
    // k -> LDS offset of (c, a, b) from the pixel's row-0 column-0 slot; -1 past K
    if (tid < 32) {
        const int k = tid;
        if (k < p.K) {
            const int c = k / taps, t = k - c * taps, a = t / p.kw, b = t - a * p.kw;
            ktab[k] = (c * HR + a) * RP + b - p.pw + 8;
        } else {
            ktab[k] = -1;
        }
    }
    // every load of a phase is issued before its LDS stores (a loop that
    // stored each load as it arrived waited on every load in turn)
    {
        uint16_t wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + i * 256, co = e / 32, k = e % 32;
            const bool ok = n0 + co < p.cout && k < p.K;
            const uint16_t v = w[ok ? (n0 + co) * p.K + k : 0];
            wv[i] = ok ? v : (uint16_t)0;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + i * 256;
            ws[(e / 32) * WROW + e % 32] = wv[i];
        }
    }
    const int nx = p.cin * HR * RP;
    for (int e0 = 0; e0 < nx; e0 += 8 * 256) {
        uint16_t xv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + i * 256;
            const int col = e % RP, rest = e / RP;
            const int hr = rest % HR, c = rest / HR;
            const int ih = h0 - p.ph + hr, iw = col - 8;
            const bool ok = e < nx && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
            const uint16_t v = x[ok ? ((int64_t)c * p.H + ih) * p.W + iw : 0];
            xv[i] = ok ? v : (uint16_t)0;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + i * 256;
            if (e < nx) xs[e] = xv[i];
        }
    }
    float bvs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p.has_bias) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int co = n0 + j * 16 + sl;
            const float v = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[min(co, p.cout - 1)]);
            bvs[j] = co < p.cout ? v : 0.0f;
        }
    }
    __syncthreads();
    int ko[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ko[e] = ktab[g * 8 + e];
    u32x4 fb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u32x4*>(ws + (j * 16 + sl) * WROW + g * 8);
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = wave * 64 + i * 16 + sl;
        const int base = (q / p.Wo) * RP + q % p.Wo;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = ko[e] >= 0 ? xs[base + ko[e]] : (uint16_t)0;
        const u32x4 fa = pack8(v);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<DT>(fa, fb[j], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ch = j * 16 + sl;
        const float bv = bvs[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint16_t h[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[i][j][r];
                if (p.has_bias) {
#pragma clang fp contract(off)
                    v = v + bv;
                }
                h[r] = __builtin_bit_cast(uint16_t, elem<DT>::from_f32(v));
            }
            const int px = wave * 64 + i * 16 + g * 4;
            *reinterpret_cast<u32x2*>(tile + ch * LROW + px) = u32x2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
        }
    }
    __syncthreads();
    // the tile's 256 pixels are contiguous in each output plane (whole rows)
    uint16_t* y = static_cast<uint16_t*>(p.out);
    const int HWo = p.Ho * p.Wo, pix0 = h0 * p.Wo;
    for (int idx = tid; idx < 64 * 32; idx += 256) {
        const int ch = idx / 32, pc = idx % 32;
        if (n0 + ch >= p.cout || pix0 + pc * 8 >= HWo) continue;
        st_nt(reinterpret_cast<u32x4*>(y + ((int64_t)img * p.cout + n0 + ch) * HWo + pix0 + pc * 8), *reinterpret_cast<const u32x4*>(tile + ch * LROW + pc * 8));
    }
}

// Grad weight: workgroup b sums pixel chunks b, b + split, ... of 512 pixels
// (4 waves x 4 steps of 32, each wave its own 128 pixels), for 16 * NI (64)
// output channels (grid y) x the 32 (zero-padded) k. Ho * Wo % 8 == 0 so a
// lane's 8 pixels lie in one image and start 16-byte aligned. (32-channel
// blocks, twice the workgroups, measured slower on the C4 stem: 12.8 against
// 10.7 us.)
template <int DT, int NI = 4>
__global__ __launch_bounds__(256) void conv_small_wgrad_kernel(SmallArgs p) {
    typedef typename elem<DT>::T T;
    constexpr int CB = 16 * NI;
    __shared__ int ktab[3][32];
    __shared__ float red[4][CB * 33];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16;
    const int n0 = blockIdx.y * CB;
    const int HW = p.H * p.W, HWo = p.Ho * p.Wo, P = p.n * HWo;
    fill_ktab(p, ktab);
    __syncthreads();
    // B columns: k = j * 16 + lane % 16
    int kc[2], ka[2], kb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        kc[j] = ktab[0][j * 16 + lane % 16];
        ka[j] = ktab[1][j * 16 + lane % 16];
        kb[j] = ktab[2][j * 16 + lane % 16];
    }
    const uint16_t* x = static_cast<const uint16_t*>(p.x);
    const uint16_t* dy = static_cast<const uint16_t*>(p.dy);
    f32x4 acc[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = blockIdx.x * 512; base < P; base += p.split * 512) {
        u32x4 fa[4][NI], fb[4][2];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int p0 = base + wave * 128 + s * 32 + g * 8;
            const bool live = p0 < P;   // P % 8 == 0: a lane's 8 pixels are all in or all out
            const int img = live ? p0 / HWo : 0, o = live ? p0 - img * HWo : 0;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int co = min(n0 + i * 16 + lane % 16, p.cout - 1);
                fa[s][i] = live ? *reinterpret_cast<const u32x4*>(dy + ((int64_t)img * p.cout + co) * HWo + o)
                                : u32x4{0u, 0u, 0u, 0u};
            }
            int oh = o / p.Wo, ow = o - oh * p.Wo;
            uint16_t v[2][8];
            const uint16_t* xb = x + img * p.cin * HW;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int ih0 = oh * p.sh - p.ph, iw0 = ow * p.sw - p.pw;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int ih = ih0 + ka[j], iw = iw0 + kb[j];
                    v[j][e] = (live && kc[j] >= 0 && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
                                  ? xb[kc[j] + ih * p.W + iw]
                                  : (uint16_t)0;
                }
                if (++ow == p.Wo) {
                    ow = 0;
                    ++oh;
                }
            }
            fb[s][0] = pack8(v[0]);
            fb[s][1] = pack8(v[1]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma16<DT>(fa[s][i], fb[s][j], acc[i][j]);
    }
    // the 4 waves' sums, added in wave order
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(i * 16 + g * 4 + r) * 33 + j * 16 + lane % 16] = acc[i][j][r];
    __syncthreads();
    for (int q = tid; q < CB * 32; q += 256) {
        const int cl = q / 32, k = q % 32, co = n0 + cl;
        if (co >= p.cout || k >= p.K) continue;
        const int at = cl * 33 + k;
        const float v = ((red[0][at] + red[1][at]) + red[2][at]) + red[3][at];
        if (p.split > 1) p.part[(int64_t)blockIdx.x * p.cout * p.K + co * p.K + k] = v;
        else reinterpret_cast<T*>(p.out)[co * p.K + k] = elem<DT>::from_f32(v);
    }
}

// The same grad weight where each 512-pixel chunk is whole rows of one image
// (stride 1, padding 1, 3x3, at most 3 input channels, W = 16, 32 or 64): the
// chunk's TR + 2 input rows of every channel go to LDS first (one aligned
// 16-byte load a thread, rows padded by 8 zero columns each side), and a
// lane's 8 pixels of one (channel, tap) come back as one 16-byte LDS read,
// shifted by one element with its neighbour for the side taps, instead of 8
// bounds-checked 2-byte global gathers. Same products, sums and partials as
// conv_small_wgrad_kernel.
__device__ inline u32x4 shift_in_low(u32x4 a, uint32_t prev) {   // {prev, a0 .. a6}
    return u32x4{(prev & 0xffffu) | (a.x << 16), (a.x >> 16) | (a.y << 16), (a.y >> 16) | (a.z << 16), (a.z >> 16) | (a.w << 16)};
}
__device__ inline u32x4 shift_in_high(u32x4 a, uint32_t next) {  // {a1 .. a7, next}
    return u32x4{(a.x >> 16) | (a.y << 16), (a.y >> 16) | (a.z << 16), (a.z >> 16) | (a.w << 16), (a.w >> 16) | (next << 16)};
}

template <int DT, int W>
__global__ __launch_bounds__(256) void conv_small_wgrad_rows_kernel(SmallArgs p) {
    typedef typename elem<DT>::T T;
    constexpr int NI = 4, CB = 16 * NI, TR = 512 / W, PITCH = W + 16, ROWS = 3 * (TR + 2);
    __shared__ __attribute__((aligned(16))) uint16_t xs[ROWS * PITCH];
    __shared__ float red[4][CB * 33];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16;
    const int n0 = blockIdx.y * CB;
    const int HW = p.H * W, P = p.n * HW;
    // this lane's B columns k = j * 16 + lane % 16: channel c, tap (a, b); k >= K are zeros
    int krow[2], kb[2];
    bool kon[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int k = j * 16 + lane % 16, c = k / 9, t = k % 9;
        kon[j] = k < p.K;
        krow[j] = kon[j] ? c * (TR + 2) + t / 3 : 0;   // (k >= K: an in-range row, the value is dropped)
        kb[j] = kon[j] ? t % 3 : 1;
    }
    // the column pads of every row, once (the fills write only the data columns)
    for (int e = tid; e < ROWS * 16; e += 256) {
        const int r = e / 16, q = e % 16;
        xs[r * PITCH + (q < 8 ? q : W + q)] = 0;
    }
    const uint16_t* x = static_cast<const uint16_t*>(p.x);
    const uint16_t* dy = static_cast<const uint16_t*>(p.dy);
    f32x4 acc[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = blockIdx.x * 512; base < P; base += p.split * 512) {
        const int img = base / HW, oh0 = (base - img * HW) / W;
        // dy of the chunk first, so its latency overlaps the row fill
        u32x4 fa[4][NI];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int o = base - img * HW + wave * 128 + s * 32 + g * 8;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int co = min(n0 + i * 16 + lane % 16, p.cout - 1);
                fa[s][i] = *reinterpret_cast<const u32x4*>(dy + ((int64_t)img * p.cout + co) * HW + o);
            }
        }
        __syncthreads();   // the previous chunk's LDS reads are done
        for (int e = tid; e < p.cin * (TR + 2) * (W / 8); e += 256) {
            const int q = e % (W / 8), r = e / (W / 8), c = r / (TR + 2), ih = oh0 - 1 + r % (TR + 2);
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (ih >= 0 && ih < p.H) v = *reinterpret_cast<const u32x4*>(x + ((int64_t)img * p.cin + c) * HW + ih * W + q * 8);
            *reinterpret_cast<u32x4*>(xs + r * PITCH + 8 + q * 8) = v;
        }
        __syncthreads();
        u32x4 fb[4][2];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int o = base - img * HW + wave * 128 + s * 32 + g * 8, oh = o / W, ow = o - oh * W;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint16_t* rp = xs + (krow[j] + oh - oh0) * PITCH + 8 + ow;
                const u32x4 a = *reinterpret_cast<const u32x4*>(rp);
                u32x4 v = a;
                if (kb[j] == 0) v = shift_in_low(a, rp[-1]);
                else if (kb[j] == 2) v = shift_in_high(a, rp[8]);
                fb[s][j] = kon[j] ? v : u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma16<DT>(fa[s][i], fb[s][j], acc[i][j]);
    }
    // the 4 waves' sums, added in wave order
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(i * 16 + g * 4 + r) * 33 + j * 16 + lane % 16] = acc[i][j][r];
    __syncthreads();
    for (int q = tid; q < CB * 32; q += 256) {
        const int cl = q / 32, k = q % 32, co = n0 + cl;
        if (co >= p.cout || k >= p.K) continue;
        const int at = cl * 33 + k;
        const float v = ((red[0][at] + red[1][at]) + red[2][at]) + red[3][at];
        if (p.split > 1) p.part[(int64_t)blockIdx.x * p.cout * p.K + co * p.K + k] = v;
        else reinterpret_cast<T*>(p.out)[co * p.K + k] = elem<DT>::from_f32(v);
    }
}

// out[e] = sum over s of part[s][e], in s order within each of SG groups
// (group q: s = q, q + SG, ...), the group sums added in group order.
template <int DT>
__global__ __launch_bounds__(256) void small_split_reduce_kernel(const float* part, void* out, int count, int split, int sg) {
    typedef typename elem<DT>::T T;
    __shared__ float red[256];
    const int L = 256 / sg, q = threadIdx.x / L, l = threadIdx.x % L;
    const int e = blockIdx.x * L + l;
    float v = 0.0f;
    if (e < count) {
        // eight planes' loads in flight before their adds (still in split order)
        int s = q;
        for (; s + 7 * sg < split; s += 8 * sg) {
            float w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = part[(int64_t)(s + u * sg) * count + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) v += w[u];
        }
        for (; s < split; s += sg) v += part[(int64_t)s * count + e];
    }
    red[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x < L && e < count) {
        float t = red[l];
        for (int k = 1; k < sg; ++k) t += red[k * L + l];
        reinterpret_cast<T*>(out)[e] = elem<DT>::from_f32(t);
    }
}

// Grad input, stride 1, 3x3 taps, dilation 1: workgroup = TR input rows (all
// W columns) of one image; threads = pixels. Output-channel pairs are staged
// S_CP at a time as a halo of dy, [pair][HR][HC] dwords (channel 2q in the low
// half, zero outside dy); the weights as [pair][tap][4 input channels] dwords.
// Every global load of a phase is issued before its LDS stores (a loop that
// stored each load as it arrived waited on every load in turn), and each halo
// element is written exactly once per chunk (rows outside dy and the columns
// left and right of it as zeros), so no separate clearing pass is needed.
constexpr int S_DT = 4;   // grad input: dy copy tasks a thread per batch of loads

template <int DT, int NC>
__global__ __launch_bounds__(256) void conv_small_dgrad_kernel(SmallArgs p) {
    typedef typename elem<DT>::T T;
    __shared__ __attribute__((aligned(16))) uint32_t dyh[S_CP * 768];
    __shared__ __attribute__((aligned(16))) uint32_t wq[128 * 9 * 4];
    const int tid = threadIdx.x;
    const int img = blockIdx.x / p.row_blocks, h0 = (blockIdx.x - img * p.row_blocks) * p.tr;
    const int HR = p.hr, HC = p.hc, HRC = HR * HC;
    const int r_lo = h0 + p.ph - 2, c_lo = p.pw - 2;   // dy row / column of halo (0, 0)
    const uint16_t* w = static_cast<const uint16_t*>(p.w);
    const uint16_t* dy = static_cast<const uint16_t*>(p.dy);
    const int HWo = p.Ho * p.Wo;
    // weight pairs: wq[(q * 9 + t) * 4 + c] = W[2q][c][t] | W[2q+1][c][t] << 16
    const int nw = p.ncp * 36;
    for (int e0 = 0; e0 < nw; e0 += 8 * 256) {
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + i * 256;
            const int c = e % 4, t = (e / 4) % 9, q = e / 36;
            const bool ok = e < nw && c < p.cin, okh = ok && 2 * q + 1 < p.cout;
            const uint16_t l = w[ok ? ((2 * q) * p.cin + c) * 9 + t : 0];
            const uint16_t h = w[okh ? ((2 * q + 1) * p.cin + c) * 9 + t : 0];
            lo[i] = ok ? l : 0u;
            hi[i] = okh ? h : 0u;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + i * 256;
            if (e < nw) wq[e] = lo[i] | (hi[i] << 16);
        }
    }
    const int tr = tid / p.W, iw = tid - tr * p.W;
    const bool live = tr < p.tr && h0 + tr < p.H;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    const int nq = p.Wo / 8;                              // 16-byte chunks per dy row
    const int left = max(0, -c_lo), right = max(0, HC - (p.Wo - c_lo));   // zero columns either side of dy
    const int ncopy = S_CP * HR * nq, nedge = S_CP * HR;
    u32x4 lo[S_DT], hi[S_DT];
    // loads of copy tasks e0 + tid + i * 256 of the chunk at pair q0
    auto load = [&](int q0, int e0) {
#pragma unroll
        for (int i = 0; i < S_DT; ++i) {
            const int e = e0 + tid + i * 256;
            const int cq = e % nq, rest = e / nq, hr = rest % HR, cp = rest / HR;
            const int co = 2 * (q0 + cp), oh = r_lo + hr;
            const bool ok = e < ncopy && co < p.cout && (unsigned)oh < (unsigned)p.Ho;
            const bool okh = ok && co + 1 < p.cout;
            const int64_t off = ((int64_t)img * p.cout + co) * HWo + oh * p.Wo + cq * 8;
            lo[i] = *reinterpret_cast<const u32x4*>(dy + (ok ? off : 0));
            hi[i] = *reinterpret_cast<const u32x4*>(dy + (okh ? off + HWo : 0));
            if (!ok) lo[i] = u32x4{0u, 0u, 0u, 0u};
            if (!okh) hi[i] = u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store = [&](int e0) {
#pragma unroll
        for (int i = 0; i < S_DT; ++i) {
            const int e = e0 + tid + i * 256;
            if (e >= ncopy) break;
            const int cq = e % nq, rest = e / nq, hr = rest % HR, cp = rest / HR;
            uint32_t* row = dyh + cp * HRC + hr * HC;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int hc = cq * 8 + k - c_lo;
                const uint32_t l = lo[i][k / 2], h = hi[i][k / 2];
                const uint32_t v = (k % 2 == 0) ? ((l & 0xffffu) | (h << 16)) : ((l >> 16) | (h & 0xffff0000u));
                if ((unsigned)hc < (unsigned)HC) row[hc] = v;
            }
        }
    };
    for (int q0 = 0; q0 < p.ncp; q0 += S_CP) {
        // halo rows of 8 dy columns (rows outside dy as zeros); keeping the
        // next chunk's loads in flight during this one's products measured
        // slower (16.4 -> 18.3 us on the C4 stem)
        for (int e0 = 0; e0 < ncopy; e0 += S_DT * 256) {
            load(q0, e0);
            store(e0);
        }
        // the columns left and right of dy
        for (int e = tid; e < nedge; e += 256) {
            uint32_t* row = dyh + (e / HR) * HRC + (e % HR) * HC;
            for (int k = 0; k < left; ++k) row[k] = 0u;
            for (int k = HC - right; k < HC; ++k) row[k] = 0u;
        }
        __syncthreads();
        if (live) {
            const int ncp = min(S_CP, p.ncp - q0);
            for (int cp = 0; cp < ncp; ++cp) {
                const uint32_t* hb = dyh + cp * HRC + tr * HC + iw;
                const u32x4* wb = reinterpret_cast<const u32x4*>(wq) + (q0 + cp) * 9;
#pragma unroll
                for (int a = 0; a < 3; ++a)
#pragma unroll
                    for (int b = 0; b < 3; ++b) {
                        // input (h0 + tr, iw) meets dy (h0 + tr + ph - a, iw + pw - b): halo (tr + 2 - a, iw + 2 - b)
                        const uint32_t v = hb[(2 - a) * HC + 2 - b];
                        const u32x4 wv = wb[a * 3 + b];
                        // scalar copies: hipcc reads element 0 for a bit cast
                        // of an indexed vector element in this unrolled loop
                        const uint32_t wc[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                        for (int c = 0; c < NC; ++c) {
                            if constexpr (DT == TVK_F16)
                                acc[c] = __builtin_amdgcn_fdot2(__builtin_bit_cast(_Float16 __attribute__((ext_vector_type(2))), v),
                                                                __builtin_bit_cast(_Float16 __attribute__((ext_vector_type(2))), wc[c]),
                                                                acc[c], false);
                            else
                                acc[c] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(__bf16 __attribute__((ext_vector_type(2))), v),
                                                                         __builtin_bit_cast(__bf16 __attribute__((ext_vector_type(2))), wc[c]),
                                                                         acc[c], false);
                        }
                    }
            }
        }
        __syncthreads();
    }
    if (!live) return;
    T* dx = static_cast<T*>(p.out);
    const int HWi = p.H * p.W;
#pragma unroll
    for (int c = 0; c < NC; ++c) dx[((int64_t)img * p.cin + c) * HWi + (h0 + tr) * p.W + iw] = elem<DT>::from_f32(acc[c]);
}

// Grad input, stride 1, 3x3, padding 1, 64 output channels, at most 16 input
// channels, as a product on the MFMA pipe: dx[c][p] = sum over k = (tap,
// output channel) of W[k][c] * dy[k][p + shift(tap)], one 16x16x32 MFMA per
// 16 pixels and 32 k (the c rows past c_in are zero). A workgroup takes
// TR = 256 / W whole input rows of one image. The dy halo [TR + 2][W + 2]
// [64 channels] is staged once in LDS (NCHW rows loaded 16 bytes at a time and
// transposed in registers, 128-byte pixel rows); each pixel-fragment read is
// one ds_read_b128. The 18 A fragments (the weights of all k) stay in
// registers for the whole tile. Lane column j of a fragment takes pixel
// pi(j): {0-3} -> 0-3, {4-11} -> 8-15, {12-15} -> 4-7, so the 16 lanes that
// gfx950 serves together (j {0-3, 12-15} of one lane group and j {4-11} of
// the next) read pixels 0-7 at one chunk and 8-15 at the next; with the
// chunk XOR 2 * ((pixel >> 1) & 3) they cover the 64 banks for any shift.
constexpr int SM_HALO = 396 * 128;   // (TR + 2) * (W + 2) pixels <= 396 (W = 64) x 128 bytes

__device__ inline int sm_swz(int hp) { return ((hp >> 1) & 3) * 2; }

template <int DT>
__global__ __launch_bounds__(256) void conv_small_dgrad_mfma_kernel(SmallArgs p) {
    typedef typename elem<DT>::T T;
    __shared__ __attribute__((aligned(16))) char halo[SM_HALO];
    __shared__ __attribute__((aligned(16))) uint16_t ws[64 * 16 * 9];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, j = lane % 16;
    const int W = p.W, TR = 256 / W, HC = W + 2, HR = TR + 2;
    const int img = blockIdx.x / p.row_blocks, h0 = (blockIdx.x - img * p.row_blocks) * TR;
    const uint16_t* w = static_cast<const uint16_t*>(p.w);
    const uint16_t* dy = static_cast<const uint16_t*>(p.dy);
    const int HW = p.H * W;

    // weights [64][cin][9] as they are, eight loads a thread in flight
    const int nw = 64 * p.cin * 9;
    for (int e0 = 0; e0 < nw; e0 += 8 * 256) {
        uint16_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + i * 256;
            v[i] = w[e < nw ? e : 0];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + i * 256;
            if (e < nw) ws[e] = v[i];
        }
    }

    // dy halo: task = (8 columns, 8 channels, halo row): eight 16-byte loads
    // (one per channel), an 8x8 transpose, eight 16-byte stores (one per
    // pixel). (Rows before channels, so that a load instruction reads a
    // channel's rows as one run, measured the same.)
    const int ncq = W / 8, ntask = HR * ncq * 8;
    u32x4 ld[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int e = tid + u * 256;
        const int cq = e % ncq, rest = e / ncq, cg = rest % 8, hr = rest / 8;
        const int oh = h0 - 1 + hr;
        const bool ok = e < ntask && (unsigned)oh < (unsigned)p.H;
        const int64_t off = ((int64_t)img * 64 + cg * 8) * HW + (int64_t)(ok ? oh : 0) * W + cq * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ld[u][i] = ok ? *reinterpret_cast<const u32x4*>(dy + off + (int64_t)i * HW) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int e = tid + u * 256;
        if (e >= ntask) break;
        const int cq = e % ncq, rest = e / ncq, cg = rest % 8, hr = rest / 8;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t v[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t lo = ld[u][2 * m][k / 2], hi = ld[u][2 * m + 1][k / 2];
                v[m] = (k % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
            }
            const int hp = hr * HC + cq * 8 + k + 1;
            *reinterpret_cast<u32x4*>(halo + hp * 128 + ((cg ^ sm_swz(hp)) * 16)) = u32x4{v[0], v[1], v[2], v[3]};
        }
    }
    // halo columns 0 and W + 1 (outside dy) are zero
    for (int e = tid; e < HR * 2 * 8; e += 256) {
        const int hp = (e / 16) * HC + ((e / 8) % 2 ? W + 1 : 0);
        *reinterpret_cast<u32x4*>(halo + hp * 128 + (e % 8) * 16) = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    // A fragments: k step s = tap * 2 + cb; lane: c = j, channels cb * 32 + 8g .. + 7
    u32x4 af[18];
#pragma unroll
    for (int s = 0; s < 18; ++s) {
        const int t = s / 2, cb = s % 2;
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int co = cb * 32 + g * 8 + e;
            h[e] = j < p.cin ? ws[(co * p.cin + j) * 9 + t] : 0u;
        }
        af[s] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
    const int pj = j < 4 ? j : (j < 12 ? j + 4 : j - 8);
    int hb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = wave * 64 + i * 16 + pj, r = q / W, col = q - r * W;
        hb[i] = (r + 2) * HC + col + 2;   // halo pixel of tap (0, 0): input (r, col) meets dy (r + 1 - a, col + 1 - b)
    }
    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 18; ++s) {
        const int t = s / 2, cb = s % 2, a = t / 3, b = t % 3;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hp = hb[i] - a * HC - b;
            const u32x4 bf = *reinterpret_cast<const u32x4*>(halo + hp * 128 + (((cb * 4 + g) ^ sm_swz(hp)) * 16));
            acc[i] = mfma16<DT>(af[s], bf, acc[i]);
        }
    }
    // lane: pixel pi(j) of each block, channels 4g .. 4g + 3
    T* dx = static_cast<T*>(p.out);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = wave * 64 + i * 16 + pj, r = q / W, col = q - r * W;
        if (h0 + r >= p.H) continue;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int c = g * 4 + m;
            if (c < p.cin) dx[((int64_t)img * p.cin + c) * HW + (int64_t)(h0 + r) * W + col] = elem<DT>::from_f32(acc[i][m]);
        }
    }
}

bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

SmallArgs small_args(const tvk_conv_desc& d) {
    SmallArgs p;
    memset(&p, 0, sizeof(p));
    p.x = d.x; p.w = d.weight; p.bias = d.bias; p.dy = d.y;
    p.n = (int)d.n; p.cin = (int)d.c_in; p.H = (int)d.h; p.W = (int)d.w; p.cout = (int)d.c_out;
    p.kh = (int)d.kh; p.kw = (int)d.kw; p.sh = (int)d.stride[0]; p.sw = (int)d.stride[1];
    p.ph = (int)d.padding[0]; p.pw = (int)d.padding[1]; p.dh = (int)d.dilation[0]; p.dw = (int)d.dilation[1];
    p.Ho = (int)d.h_out; p.Wo = (int)d.w_out;
    p.K = p.cin * p.kh * p.kw;
    return p;
}

// forward by whole output rows: stride 1, dilation 1, Wo a power of two in
// 8..256, the padding inside the 8 spare columns each side of a staged row,
// and the staged rows within 16 KB
bool fwd_rows_applies(const tvk_conv_desc& d) {
    if (d.stride[0] != 1 || d.stride[1] != 1 || d.dilation[0] != 1 || d.dilation[1] != 1) return false;
    const int64_t wo = d.w_out;
    if (wo < 8 || wo > 256 || (wo & (wo - 1)) != 0 || !al16(d.y)) return false;
    if (d.padding[1] > 8 || wo - 1 + d.kw - 1 - d.padding[1] >= d.w + 8) return false;
    return d.c_in * (256 / wo + d.kh - 1) * (d.w + 16) <= 8192;
}

// grad input on the MFMA pipe: 3x3 stride 1 padding 1, 64 output channels,
// W in {8, 16, 32, 64}, dy 16-byte aligned
bool dgrad_mfma_applies(const tvk_conv_desc& d) {
    if (d.kh != 3 || d.kw != 3 || d.stride[0] != 1 || d.stride[1] != 1 || d.dilation[0] != 1 || d.dilation[1] != 1) return false;
    if (d.padding[0] != 1 || d.padding[1] != 1 || d.c_out != 64 || d.c_in > 16) return false;
    return (d.w == 8 || d.w == 16 || d.w == 32 || d.w == 64) && al16(d.y);
}

// grad input tile: rows per workgroup and the halo it stages
void dgrad_tile(const tvk_conv_desc& d, int& tr, int& hr, int& hc) {
    tr = std::max<int>(1, 256 / (int)d.w);
    hr = tr + 2;
    hc = (int)d.w + 2;
}

}  // namespace

bool conv_small_applies(const tvk_conv_desc& d, int mode) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return false;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return false;
    // channel-rich convolutions keep the channels-last ring
    if (d.c_in * d.kh * d.kw > 32 || d.c_in >= 32) return false;
    // 32-bit element offsets
    const int64_t big = std::max({d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out});
    if (big >= (int64_t(1) << 30)) return false;
    if (mode == 0) return true;
    if (mode == 2) return (d.h_out * d.w_out) % 8 == 0 && al16(d.y);
    // grad input: the stride-1 3x3 kernels
    if (d.kh != 3 || d.kw != 3 || d.stride[0] != 1 || d.stride[1] != 1 || d.dilation[0] != 1 || d.dilation[1] != 1) return false;
    if (dgrad_mfma_applies(d)) return true;
    if (d.c_in > 4 || d.c_out > 256 || d.w > 256 || d.w_out % 8 != 0 || !al16(d.y)) return false;
    int tr, hr, hc;
    dgrad_tile(d, tr, hr, hc);
    return hr * hc <= 768;
}

tvk_status conv_small_run(const tvk_conv_desc& d, int mode, const char* who) {
    SmallArgs p = small_args(d);
    hipStream_t s = resolve_stream(d.stream);
    Scratch scratch;
    const bool f16 = d.dtype == TVK_F16;
    if (mode == 0) {
        p.out = d.y;
        p.M = p.n * p.Ho * p.Wo;
        p.has_bias = d.bias ? 1 : 0;
        p.vec_out = (p.Ho * p.Wo) % 8 == 0 && al16(d.y);
        if (fwd_rows_applies(d)) {
            p.row_blocks = (p.Ho + 256 / p.Wo - 1) / (256 / p.Wo);
            const dim3 grid((unsigned)(p.n * p.row_blocks), (unsigned)((p.cout + 63) / 64));
            if (f16) hipLaunchKernelGGL(conv_small_fwd_rows_kernel<TVK_F16>, grid, dim3(256), 0, s, p);
            else hipLaunchKernelGGL(conv_small_fwd_rows_kernel<TVK_BF16>, grid, dim3(256), 0, s, p);
        } else {
            const dim3 grid((unsigned)((p.M + 255) / 256), (unsigned)((p.cout + 63) / 64));
            if (f16) hipLaunchKernelGGL(conv_small_fwd_kernel<TVK_F16>, grid, dim3(256), 0, s, p);
            else hipLaunchKernelGGL(conv_small_fwd_kernel<TVK_BF16>, grid, dim3(256), 0, s, p);
        }
    } else if (mode == 2) {
        const int64_t P = (int64_t)p.n * p.Ho * p.Wo;
        const int ny = (p.cout + 63) / 64;
        // 512-pixel chunks; at most 1024 workgroups along the pixels
        p.split = (int)std::max<int64_t>(1, std::min<int64_t>((P + 511) / 512, 1024));
        p.out = d.weight;
        const int count = p.cout * p.K;
        if (p.split > 1) {
            p.part = static_cast<float*>(scratch.get((size_t)p.split * count * sizeof(float), s));
            if (!p.part) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the grad-weight partials");
        }
        const dim3 grid((unsigned)p.split, (unsigned)ny);
        // whole-row chunks of a stride-1 3x3 padding-1 stem: input rows staged in LDS
        const bool rows = d.kh == 3 && d.kw == 3 && d.stride[0] == 1 && d.stride[1] == 1 && d.padding[0] == 1 &&
                          d.padding[1] == 1 && d.dilation[0] == 1 && d.dilation[1] == 1 && d.c_in <= 3 &&
                          (p.W == 16 || p.W == 32 || p.W == 64) && p.H % (512 / p.W) == 0 && al16(d.x);
#define TVK_SWR(W_)                                                                                          \
    do {                                                                                                     \
        if (f16) hipLaunchKernelGGL((conv_small_wgrad_rows_kernel<TVK_F16, W_>), grid, dim3(256), 0, s, p); \
        else hipLaunchKernelGGL((conv_small_wgrad_rows_kernel<TVK_BF16, W_>), grid, dim3(256), 0, s, p);    \
    } while (0)
        if (rows && p.W == 16) TVK_SWR(16);
        else if (rows && p.W == 32) TVK_SWR(32);
        else if (rows) TVK_SWR(64);
        else if (f16) hipLaunchKernelGGL((conv_small_wgrad_kernel<TVK_F16, 4>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((conv_small_wgrad_kernel<TVK_BF16, 4>), grid, dim3(256), 0, s, p);
#undef TVK_SWR
        if (p.split > 1) {
            int sg = 1;
            while (sg < 16 && sg * 2 <= p.split && (int64_t)count * sg / 256 < 512) sg *= 2;
            const int L = 256 / sg;
            const dim3 rgrid((unsigned)((count + L - 1) / L));
            if (f16) hipLaunchKernelGGL(small_split_reduce_kernel<TVK_F16>, rgrid, dim3(256), 0, s, p.part, d.weight, count, p.split, sg);
            else hipLaunchKernelGGL(small_split_reduce_kernel<TVK_BF16>, rgrid, dim3(256), 0, s, p.part, d.weight, count, p.split, sg);
        }
    } else if (dgrad_mfma_applies(d)) {
        p.out = d.x;
        p.tr = 256 / p.W;
        p.row_blocks = (p.H + p.tr - 1) / p.tr;
        const dim3 grid((unsigned)(p.n * p.row_blocks));
        if (f16) hipLaunchKernelGGL(conv_small_dgrad_mfma_kernel<TVK_F16>, grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL(conv_small_dgrad_mfma_kernel<TVK_BF16>, grid, dim3(256), 0, s, p);
    } else {
        p.out = d.x;
        dgrad_tile(d, p.tr, p.hr, p.hc);
        p.ncp = (p.cout + 1) / 2;
        p.row_blocks = (p.H + p.tr - 1) / p.tr;
        const dim3 grid((unsigned)(p.n * p.row_blocks));
#define TVK_SD(NC_)                                                                                 \
    do {                                                                                          \
        if (f16) hipLaunchKernelGGL((conv_small_dgrad_kernel<TVK_F16, NC_>), grid, dim3(256), 0, s, p);  \
        else hipLaunchKernelGGL((conv_small_dgrad_kernel<TVK_BF16, NC_>), grid, dim3(256), 0, s, p);     \
    } while (0)
        switch (p.cin) {
        case 1: TVK_SD(1); break;
        case 2: TVK_SD(2); break;
        case 3: TVK_SD(3); break;
        default: TVK_SD(4); break;
        }
#undef TVK_SD
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

}  // namespace tvk
