// 2-D convolution on gfx950 as a channels-last implicit GEMM over the
// direct-to-LDS ring of gemm_dma.hip: float16/bfloat16, groups == 1, channel
// counts in multiples of 32 (the layers of the path's ResNet config; other
// convolutions keep the element-gather kernels of conv.hip).
//
// Reference semantics (file:line under the reference tree): the same sums as
// conv.hip's kernels (src/shaders/helpers/conv.slang:198-511,
// src/api/ops/conv.cpp:1014-1060) with a different k order inside the
// reduction (tap-major, channel-minor), which the fp16/bf16 tolerance allows;
// the strided grad-input runs as stride^2 sub-pixel phases, each a dense GEMM
// over the taps that reach it, as the reference's subpixel_split does
// (src/api/ops/conv.cpp:364-382, src/shaders/helpers/conv.slang:135-172,364-432).
//
// Layouts. The activation that is gathered goes to NHWC in the library
// workspace first (one transpose pass), so that 8 consecutive channels are one
// 16-byte load, with a zero border wide enough for every tap of every row
// pixel: the loads need no bounds checks, and each lane's offsets are set
// once, a stage adding one uniform tap and channel offset. The weight is
// permuted to tap-major order.
//   forward     C[p][co] = sum_{t,c} x_nhwc[pix(p) + off(t)][c] * Wf[co][t][c]
//               p = output pixel (n, oh, ow); y is written NCHW
//   grad input  C[p][c]  = sum_{t,co} dy_nhwc[pix(p) + off(t)][co] * Wd[c][t][co]
//               p = input pixel of one sub-pixel phase; dx is written NCHW
//   grad weight C[(t,c)][co] = sum_p x_nhwc[pix(p) + off(t)][c] * dy[n][co][o(p)]
//               K = output pixels, split into float32 partials reduced in split
//               order into dW[co][c][t]
// Tiles are 256 rows (pixels, or (tap, channel) for grad weight) x BN columns
// (output channels) with BN = 64, 128 or 256, a 4-stage ring of 32-k stages,
// v_mfma_f32_16x16x32 on 64-column wave tiles.
#include "tvk_common.h"
#include "gemm_common.h"
#include "convert.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <type_traits>

namespace tvk {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
#define TVK_LDS __attribute__((address_space(3)))

constexpr int V_BK = 32, V_NS = 4;
constexpr int V_MAXTAPS = 16;

struct ConvRing {
    const void* act;     // gathered activation, padded NHWC (x, or dy for grad input)
    const void* wt;      // permuted weight [N][T][Cs] (forward / grad input)
    const void* dyc;     // grad weight: dy, NCHW
    const void* bias;    // forward
    void* out;           // y / dx NCHW (forward, grad input); dW (grad weight, no split)
    float* part;         // grad weight partials [split][M][N]
    // gather geometry: the activation is [n][Hs][Ws][Cs], Hs and Ws including the
    // zero border; every row pixel and tap lands inside it
    int Hs, Ws, Cs;
    // rows: pixels of an [n][Hp][Wp] grid (forward / grad input)
    int Hp, Wp;
    int M, N, K;         // GEMM sizes
    int ntap;            // taps in this launch (a sub-pixel phase may use a subset)
    int wt_taps;         // taps per row of the permuted weight
    int tap_h[V_MAXTAPS], tap_w[V_MAXTAPS], tap_k[V_MAXTAPS];   // row offsets and weight tap of each k tap
    int tap_off[V_MAXTAPS], wt_off[V_MAXTAPS];   // forward / grad input: byte offsets of each k tap in act and wt
    int pix_sh, pix_sw, pix_bh, pix_bw;   // row pixel (i, j) -> source origin (i*sh + bh, j*sw + bw), border included
    Div32 wdiv;          // grad weight: division by the output width
    // output placement (forward / grad input): pixel (i, j) -> (i*osh + orh, j*osw + orw) of [n][N][Ho][Wo]
    int Ho, Wo, osh, osw, orh, orw;
    // grad weight: output pixels per image, width; k per split; taps for the dW order
    int HWo, Wd, kh_kw, k_chunk, split;
    int has_bias;
    int act_bytes, wt_bytes, dyc_bytes;
};

// One launch covers up to 4 problems in grid z: the sub-pixel phases of a
// stride-2 grad input (forward and grad weight use ph[0])
constexpr int V_MAXPH = 4;
struct ConvRingSet {
    ConvRing ph[V_MAXPH];
};

__device__ inline i32x4 v_rsrc(const void* p, int64_t bytes) {
    const uint64_t a = (uint64_t)p;
    return i32x4{(int)(uint32_t)a, (int)((a >> 32) & 0xffff), (int)min(bytes, (int64_t)0x7fffffff), 0x00020000};
}
__device__ inline void v_dma16(i32x4 r, uint32_t lds_addr, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voff), "s"(r) : "memory");
}
template <int N>
__device__ inline void v_wait() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }

__device__ inline int swz_km(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }
__device__ inline int swz_mn(int kr) { return (kr & 3) * 2; }

template <int DT>
__device__ inline f32x4 vmfma(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 16x16x32 fragment of a k-contiguous tile (rows of 64 bytes, XOR chunk swizzle)
__device__ inline u32x4 frag_km(uint32_t base, int row_base, int lane) {
    const int row = row_base + lane % 16;
    return *(const TVK_LDS u32x4*)(uintptr_t)(base + row * 64 + (((lane / 16) ^ swz_km(row)) * 16));
}
// 16x16x32 fragment of an m-contiguous tile (k-rows of 512 bytes): transposed reads
__device__ inline u32x4 frag_mn(uint32_t base, int col_base, int lane) {
    const int g = lane / 16, s = lane % 16;
    const int col = col_base + (s % 4) * 4;
    const int chunk = col / 8, within = (col % 8) * 2;
    u32x4 out;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const int kr = g * 8 + rr * 4 + s / 4;
        TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(base + kr * 512 + ((chunk ^ swz_mn(kr)) * 16) + within);
        const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
        out[rr * 2] = w.x;
        out[rr * 2 + 1] = w.y;
    }
    return out;
}

// waves of a BM x BN tile: 64x64 wave tiles, except 256x256 (8 waves of 128x64)
constexpr int ring_waves(int bm, int bn) { return bm == 256 ? (bn == 64 ? 4 : 8) : 2 * (bn / 64); }

// MODE 0: rows are pixels (forward, grad input; grid z = sub-pixel phase);
// MODE 1: grad weight (grid z = k split).
template <int DT, int MODE, int BM, int BN>
__global__ __launch_bounds__(64 * ring_waves(BM, BN)) void conv_ring_kernel(ConvRingSet set) {
    static_assert(MODE == 0 || BM == 256, "grad weight uses 256-row tiles");
    constexpr int V_BM = BM;
    constexpr int NW = ring_waves(BM, BN);
    constexpr int WN = BN / 64, WMW = NW / WN;       // waves along N and M
    constexpr int WTM = V_BM / WMW;                  // wave tile rows (x 64 columns)
    constexpr int FM = WTM / 16, FN = 4;
    constexpr int OPA = V_BM * V_BK * 2;
    constexpr int OPB = BN * V_BK * 2;
    constexpr int STB = OPA + OPB;
    constexpr int DA = (OPA / 1024) / NW, DB = (OPB / 1024) / NW, DS = DA + DB;
    static_assert(DB >= 1 && DA >= 1, "every wave loads both operands");
    constexpr int LROW = V_BM + 8;                   // epilogue tile row (halfs)
    constexpr int LDS_BYTES = V_NS * STB > BN * LROW * 2 ? V_NS * STB : BN * LROW * 2;
    __shared__ __attribute__((aligned(1024))) char lds_raw[LDS_BYTES];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds_raw);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int wm = wave / WN, wn = wave % WN;
    const ConvRing& p = set.ph[MODE == 0 ? blockIdx.z : 0];
    const int m0 = blockIdx.x * V_BM, n0 = blockIdx.y * BN;
    if (m0 >= p.M) return;   // this phase has fewer row tiles than the grid
    const int z = blockIdx.z;
    const int kb = MODE == 1 ? z * p.k_chunk : 0;
    const int klen = MODE == 1 ? min(p.k_chunk, p.K - kb) : p.K;
    const int nk = klen / V_BK;

    const i32x4 ra = v_rsrc(p.act, p.act_bytes);
    const i32x4 rb = v_rsrc(MODE == 1 ? p.dyc : p.wt, MODE == 1 ? p.dyc_bytes : p.wt_bytes);

    // ---- per-lane, per-load constants ----
    // Rows past M (pixels, or (tap, channel) rows) and columns past N read a
    // valid row instead; their results are never stored.
    // A (MODE 0): KM tile, 16 rows per block; a_off = byte offset of the row
    //   pixel's origin and the lane's 8 channels, a stage adds its tap and channel
    // A (MODE 1): MN tile, 2 k-rows per block; a_off = element offset of the
    //   lane's (tap, channel) chunk, a stage adds its output pixel's position
    int a_off[DA], a_kr[DA];
#pragma unroll
    for (int q = 0; q < DA; ++q) {
        const int blk = wave * DA + q;
        if constexpr (MODE == 0) {
            const int row = blk * 16 + lane / 4;
            const int pix = min(m0 + row, p.M - 1);
            const int hw = p.Hp * p.Wp;
            const int img = pix / hw, r = pix - img * hw;
            const int i = r / p.Wp, j = r - i * p.Wp;
            const int ih = i * p.pix_sh + p.pix_bh, iw = j * p.pix_sw + p.pix_bw;
            a_off[q] = (((img * p.Hs + ih) * p.Ws + iw) * p.Cs + ((lane % 4) ^ swz_km(row)) * 8) * 2;
            a_kr[q] = 0;
        } else {
            const int kr = blk * 2 + lane / 32;
            const int m = min(m0 + (((lane % 32) ^ swz_mn(kr)) * 8), p.M - 8);
            const int t = m / p.Cs, c = m - t * p.Cs;
            a_off[q] = (p.tap_h[t] * p.Ws + p.tap_w[t]) * p.Cs + c;
            a_kr[q] = kr;
        }
    }
    // B: KM tile, 16 rows (output channels) per block; byte offset of the lane's row and chunk
    int b_off[DB];
#pragma unroll
    for (int q = 0; q < DB; ++q) {
        const int blk = wave * DB + q;
        const int row = blk * 16 + lane / 4;
        const int n = min(n0 + row, p.N - 1);
        const int bc = ((lane % 4) ^ swz_km(row)) * 8;
        if constexpr (MODE == 0) b_off[q] = (n * p.wt_taps * p.Cs + bc) * 2;
        else b_off[q] = (n * p.HWo + bc) * 2;
    }

    // MODE 0: stages run tap-major, channel-minor in issue order
    int it = 0, ic0 = 0;
    auto issue = [&](int s) {
        if (s >= nk) return;
        const uint32_t slot = lds0 + (uint32_t)((s % V_NS) * STB);
        if constexpr (MODE == 0) {
            const int aoff = p.tap_off[it] + ic0 * 2, woff = p.wt_off[it] + ic0 * 2;
#pragma unroll
            for (int q = 0; q < DA; ++q) v_dma16(ra, slot + (uint32_t)((wave * DA + q) * 1024), (uint32_t)(a_off[q] + aoff));
#pragma unroll
            for (int q = 0; q < DB; ++q) v_dma16(rb, slot + OPA + (uint32_t)((wave * DB + q) * 1024), (uint32_t)(b_off[q] + woff));
            ic0 += V_BK;
            if (ic0 == p.Cs) {
                ic0 = 0;
                ++it;
            }
        } else {
            // the stage's 32 output pixels lie in one image (HWo % 32 == 0)
            const int k0 = kb + s * V_BK;
            const int img = k0 / p.HWo, o0 = k0 - img * p.HWo;
            const int ibase = img * p.Hs;
#pragma unroll
            for (int q = 0; q < DA; ++q) {
                const int o = o0 + a_kr[q];
                const int oh = (int)div32((uint32_t)o, p.wdiv), ow = o - oh * p.Wd;
                const int off = ((ibase + oh * p.pix_sh) * p.Ws + ow * p.pix_sw) * p.Cs + a_off[q];
                v_dma16(ra, slot + (uint32_t)((wave * DA + q) * 1024), (uint32_t)off * 2);
            }
            const int dyoff = ((img * p.N) * p.HWo + o0) * 2;
#pragma unroll
            for (int q = 0; q < DB; ++q) v_dma16(rb, slot + OPA + (uint32_t)((wave * DB + q) * 1024), (uint32_t)(b_off[q] + dyoff));
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto read_a = [&](uint32_t st, int i) {
        if constexpr (MODE == 0) return frag_km(st, wm * WTM + i * 16, lane);
        else return frag_mn(st, wm * WTM + i * 16, lane);
    };
    u32x4 fa[2][FM], fb[2][FN];
    if (nk > 0) {
#pragma unroll
        for (int s = 0; s < V_NS; ++s) issue(s);
        // stage 0 landed
        if (nk >= V_NS) v_wait<DS * (V_NS - 1)>(); else v_wait<0>();
        __syncthreads();
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[0][i] = read_a(lds0, i);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[0][j] = frag_km(lds0 + OPA, wn * 64 + j * 16, lane);
        if (nk >= V_NS) v_wait<DS * (V_NS - 2)>(); else v_wait<0>();
        __syncthreads();

        auto body = [&](int kt, auto cur_c) {
            constexpr int cur = decltype(cur_c)::value;
            // (on the last stage the reads fetch a slot no stage filled: unused)
            const uint32_t st_next = lds0 + (uint32_t)(((kt + 1) % V_NS) * STB);
#pragma unroll
            for (int q = 0; q < FM * FN; ++q) {
                const int i = q / FN, j = q % FN;
                acc[i][j] = vmfma<DT>(fa[cur][i], fb[cur][j], acc[i][j]);
                if (q % 2 == 0) {
                    const int r = q / 2;
                    if (r < FM) fa[cur ^ 1][r] = read_a(st_next, r);
                    else if (r < FM + FN) fb[cur ^ 1][r - FM] = frag_km(st_next + OPA, wn * 64 + (r - FM) * 16, lane);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            issue(kt + V_NS);
            // stage kt+2 landed (or, near the end, everything issued)
            if (kt + V_NS < nk) v_wait<DS * (V_NS - 2)>(); else v_wait<0>();
            __syncthreads();
        };
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            body(kt, std::integral_constant<int, 0>{});
            body(kt + 1, std::integral_constant<int, 1>{});
        }
        if (kt < nk) body(kt, std::integral_constant<int, 0>{});
        v_wait<0>();
        __syncthreads();
    }

    typedef typename elem<DT>::T T;
    if constexpr (MODE == 1) {
        // (tap, channel) rows x output-channel columns: partials, or dW[co][c][t]
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = n0 + wn * 64 + j * 16 + lane % 16;
                if (col >= p.N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm * WTM + i * 16 + (lane / 16) * 4 + r;
                    if (row >= p.M) continue;
                    if (p.split > 1) {
                        p.part[((int64_t)z * p.M + row) * p.N + col] = acc[i][j][r];
                    } else {
                        const int t = row / p.Cs, c = row - t * p.Cs;
                        reinterpret_cast<T*>(p.out)[((int64_t)col * p.Cs + c) * p.kh_kw + t] = elem<DT>::from_f32(acc[i][j][r]);
                    }
                }
            }
        return;
    }

    // pixels x channels -> NCHW through LDS: the tile is written as [channel][pixel]
    // (rows of 256 pixels + 8 halfs of padding), then each thread stores 8 pixels
    // of one channel at a time
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds_raw);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int ch = wn * 64 + j * 16 + lane % 16;
            const int px = wm * WTM + i * 16 + (lane / 16) * 4;
            float bv = 0.0f;
            if (p.has_bias && n0 + ch < p.N) bv = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[n0 + ch]);
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
            *reinterpret_cast<u32x2*>(tile + ch * LROW + px) = u32x2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
        }
    __syncthreads();
    T* out = reinterpret_cast<T*>(p.out);
    const int hw = p.Hp * p.Wp;
    const bool dense = p.osh == 1 && p.osw == 1 && p.Hp == p.Ho && p.Wp == p.Wo && hw % 8 == 0;
    constexpr int NT = 64 * NW;
    if (dense) {
        for (int idx = tid; idx < BN * (V_BM / 8); idx += NT) {
            const int ch = idx / (V_BM / 8), pc = idx % (V_BM / 8);
            const int co = n0 + ch;
            const int pix = m0 + pc * 8;
            if (co >= p.N || pix >= p.M) continue;
            // 8 pixels of one image row run (hw % 8 == 0): one 16-byte store
            const int img = pix / hw, o = pix - img * hw;
            st_nt(reinterpret_cast<u32x4*>(out + ((int64_t)img * p.N + co) * hw + o), *reinterpret_cast<const u32x4*>(tile + ch * LROW + pc * 8));
        }
    } else {
        // sub-pixel phases (or pixel runs that 16-byte stores do not fit): a
        // thread keeps one pixel (NT is a multiple of the tile's rows) and walks
        // the channels, so a store's 64 lanes write 64 consecutive row pixels
        static_assert(NT % V_BM == 0, "one pixel per thread");
        const int pc = tid % V_BM, pix = m0 + pc;
        if (pix < p.M) {
            const int img = pix / hw, r = pix - img * hw;
            const int i = r / p.Wp, j = r - i * p.Wp;
            const int plane = p.Ho * p.Wo;
            T* o = out + ((int64_t)img * p.N + n0) * plane + (i * p.osh + p.orh) * p.Wo + j * p.osw + p.orw;
            for (int ch = tid / V_BM; ch < BN && n0 + ch < p.N; ch += NT / V_BM)
                o[(int64_t)ch * plane] = __builtin_bit_cast(T, tile[ch * LROW + pc]);
        }
    }
}

// NCHW -> zero-bordered NHWC [n][Hs][Ws][C] for 16-bit elements, the image at
// rows pt.. and columns pl.. of each padded plane. The grid is one-dimensional:
// workgroup b < nx * cy * n takes column block b % nx of channel block
// (b / nx) % cy of image b / (nx * cy); the workgroups after those, when the
// weight is given, permute the weight for the same convolution in the same
// launch: w[co][c][t] -> wout[co][t][c] (forward) or wout[c][t][co] (grad
// input). Column block nx - 1, when the plane has a border, zeroes the border
// pixels of its channels (the rows above and below, then the columns left and
// right of each image row); the others copy 64 channels x PX pixels.
// VEC (HW % 8 == 0, C % 8 == 0): PX = 256, no LDS. A lane loads 8 pixels of 8
// channels (eight 16-byte loads; 8 lanes read 128 contiguous bytes of a channel
// row), transposes the 8x8 block of 16-bit elements in registers and stores 8
// pixels of 8 channels (8 lanes write 128 contiguous bytes of a pixel).
// Otherwise PX = 64 through an LDS tile, element accesses where the counts
// leave no 16-byte run.
struct WeightPermute {
    const uint16_t* w = nullptr;
    uint16_t* out = nullptr;
    int cout = 0, cin = 0, taps = 0, forward = 0;
};

struct NhwcArgs {
    const uint16_t* src;
    uint16_t* dst;
    int C, H, W, Hs, Ws, pt, pl;
    int nblk, nx, cy, copy_blocks;   // copy column blocks per plane (nblk, plus 1 with a border)
    WeightPermute wp;
};

__device__ inline void permute_weight(const WeightPermute& wp, int blk, int nb) {
    // weight elements number below 2^30 (checked on the host)
    const int total = wp.cout * wp.cin * wp.taps;
    for (int e = blk * 256 + (int)threadIdx.x; e < total; e += nb * 256) {
        const int t = e % wp.taps, r = e / wp.taps;
        const int c = r % wp.cin, co = r / wp.cin;
        const int o = wp.forward ? (co * wp.taps + t) * wp.cin + c : (c * wp.taps + t) * wp.cout + co;
        wp.out[o] = wp.w[e];
    }
}

__device__ inline void zero_border(const NhwcArgs& a, uint16_t* d, int c0, bool vec) {
    const int rows = a.Hs - a.H, cols = a.Ws - a.W;   // border rows (whole width), border columns per image row
    const int npix = rows * a.Ws + a.H * cols;
    for (int e = threadIdx.x; e < npix * 8; e += 256) {
        const int px = e / 8, c = c0 + (e % 8) * 8;
        if (c >= a.C) continue;
        int hp, wq;
        if (px < rows * a.Ws) {
            const int r = px / a.Ws;
            hp = r < a.pt ? r : r + a.H;
            wq = px - r * a.Ws;
        } else {
            const int q = px - rows * a.Ws, r = q / cols, k = q - r * cols;
            hp = a.pt + r;
            wq = k < a.pl ? k : k + a.W;
        }
        uint16_t* o = d + ((int64_t)hp * a.Ws + wq) * a.C + c;
        if (vec && c + 8 <= a.C) *reinterpret_cast<u32x4*>(o) = u32x4{0, 0, 0, 0};
        else
            for (int k = 0; k < 8 && c + k < a.C; ++k) o[k] = 0;
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void nchw_to_nhwc_kernel(NhwcArgs a) {
    const int b = blockIdx.x;
    if (b >= a.copy_blocks) {
        permute_weight(a.wp, b - a.copy_blocks, (int)gridDim.x - a.copy_blocks);
        return;
    }
    const int bx = b % a.nx, img = b / (a.nx * a.cy), c0 = (b / a.nx - img * a.cy) * 64;
    const int C = a.C, W = a.W, HW = a.H * a.W;
    uint16_t* d = a.dst + (int64_t)img * a.Hs * a.Ws * C;
    if (bx >= a.nblk) {
        zero_border(a, d, c0, VEC);
        return;
    }
    const uint16_t* s = a.src + (int64_t)img * C * HW;
    if constexpr (VEC) {
        const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
        const int c = c0 + (lane % 8) * 8;
        const int px = bx * 256 + wave * 64 + (lane / 8) * 8;
        if (c >= C || px >= HW) return;
        u32x4 r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = *reinterpret_cast<const u32x4*>(s + (int64_t)(c + i) * HW + px);
        int h = px / W, w = px - h * W;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // pixel px + j: channel pairs (2k, 2k + 1) packed low/high
            uint32_t v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = r[2 * k][j / 2], hi = r[2 * k + 1][j / 2];
                v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
            }
            *reinterpret_cast<u32x4*>(d + ((int64_t)(h + a.pt) * a.Ws + w + a.pl) * C + c) = u32x4{v[0], v[1], v[2], v[3]};
            if (++w == W) {
                w = 0;
                ++h;
            }
        }
    } else {
        __shared__ uint16_t tile[64][72];
        const int p0 = bx * 64;
#pragma unroll
        for (int e = threadIdx.x; e < 64 * 8; e += 256) {
            const int c = e / 8, q = (e % 8) * 8;
            if (c0 + c >= C) continue;
            for (int k = 0; k < 8; ++k)
                if (p0 + q + k < HW) tile[c][q + k] = s[(int64_t)(c0 + c) * HW + p0 + q + k];
        }
        __syncthreads();
#pragma unroll
        for (int e = threadIdx.x; e < 64 * 8; e += 256) {
            const int q = e / 8, c = (e % 8) * 8;
            const int px = p0 + q;
            if (px >= HW) continue;
            const int h = px / W, w = px - h * W;
            uint16_t* o = d + ((int64_t)(h + a.pt) * a.Ws + w + a.pl) * C + c0 + c;
            for (int k = 0; k < 8; ++k)
                if (c0 + c + k < C) o[k] = tile[c + k][q];
        }
    }
}

// grad weight: sums partials [split][(t,c)][co] into dW[co][c][t]. A
// workgroup takes E = 1024 / SG consecutive outputs: SG groups of threads each
// sum every SG-th split with 16-byte loads (group g: splits g, g + SG, ... in
// order; 4 outputs a thread), then the SG group sums are added in group order
// through LDS. (M * N % 4 == 0; SG a power of two up to 16.)
template <int DT>
__global__ __launch_bounds__(256) void wgrad_ring_reduce_kernel(const float* part, void* out, int M, int N, int Cs, int taps,
                                                                int split, int sg) {
    typedef typename elem<DT>::T T;
    __shared__ float red[1024];
    const int total = M * N;   // below 2^30 (checked on the host)
    const int L = 256 / sg, E = 1024 / sg;
    const int g = threadIdx.x / L, l = threadIdx.x % L;
    const int e0 = blockIdx.x * E + l * 4;
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (e0 < total) {
        // eight planes' loads in flight before their adds (still in split order)
        const float* src = part + e0;
        int s = g;
        for (; s + 7 * sg < split; s += 8 * sg) {
            f32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f32x4*>(src + (int64_t)(s + u * sg) * total);
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; s < split; s += sg) acc += *reinterpret_cast<const f32x4*>(src + (int64_t)s * total);
    }
    *reinterpret_cast<f32x4*>(red + g * E + l * 4) = acc;
    __syncthreads();
    for (int k = threadIdx.x; k < E; k += 256) {
        const int e = blockIdx.x * E + k;
        if (e >= total) break;
        float v = red[k];
        for (int q = 1; q < sg; ++q) v += red[q * E + k];
        const int row = e / N, co = e - row * N;
        const int t = row / Cs, c = row - t * Cs;
        reinterpret_cast<T*>(out)[((int64_t)co * Cs + c) * taps + t] = elem<DT>::from_f32(v);
    }
}

// Launches MODE 0 over set.ph[0..nph) (grid z = phase) or MODE 1 over `splits`
// k splits. 128-row tiles when 256-row tiles would leave the device under-filled.
#ifndef TVK_RING_MIN_BN
#define TVK_RING_MIN_BN 64
#endif
template <int DT, int MODE>
void launch_ring(const ConvRingSet& set, int nph, int splits, hipStream_t s) {
    const ConvRing& p0 = set.ph[0];
    int bn = p0.N <= 64 ? 64 : p0.N <= 128 ? 128 : 256;
    int max_m = 0;
    for (int i = 0; i < nph; ++i) max_m = std::max(max_m, set.ph[i].M);
    // forward / grad input: narrower columns while 128-row tiles leave the device under-filled
    if (MODE == 0)
        while (bn > TVK_RING_MIN_BN && (int64_t)((max_m + 127) / 128) * ((p0.N + bn - 1) / bn) * nph < 192) bn /= 2;
    const int ny = (p0.N + bn - 1) / bn;
    const int64_t t256 = (int64_t)((max_m + 255) / 256) * ny * (MODE == 0 ? nph : splits);
    const int bm = (MODE == 0 && t256 < 192) ? 128 : 256;
    const dim3 grid((max_m + bm - 1) / bm, ny, MODE == 0 ? nph : splits);
#define TVK_RING(BM_, BN_) hipLaunchKernelGGL((conv_ring_kernel<DT, MODE, BM_, BN_>), grid, dim3(64 * ring_waves(BM_, BN_)), 0, s, set)
    if constexpr (MODE == 0) {
        if (bm == 128) {
            if (bn == 64) TVK_RING(128, 64); else if (bn == 128) TVK_RING(128, 128); else TVK_RING(128, 256);
            return;
        }
    }
    if (bn == 64) TVK_RING(256, 64); else if (bn == 128) TVK_RING(256, 128); else TVK_RING(256, 256);
#undef TVK_RING
}

// A zero border around each image: pt/pb rows above/below, pl/pr columns left/right.
struct Border {
    int pt = 0, pb = 0, pl = 0, pr = 0;
};

void launch_nhwc(const void* src, void* dst, int n, int C, int H, int W, const Border& bd, hipStream_t s,
                 const WeightPermute& wp = WeightPermute()) {
    NhwcArgs a;
    a.src = static_cast<const uint16_t*>(src);
    a.dst = static_cast<uint16_t*>(dst);
    a.C = C; a.H = H; a.W = W;
    a.Hs = H + bd.pt + bd.pb; a.Ws = W + bd.pl + bd.pr;
    a.pt = bd.pt; a.pl = bd.pl;
    // 16-byte accesses: every channel row and pixel starts 16-byte aligned (the
    // source is, and the workspace is 256-byte aligned)
    const bool vec = (H * W) % 8 == 0 && C % 8 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
    const int px = vec ? 256 : 64;
    a.nblk = (H * W + px - 1) / px;
    const bool border = a.Hs > H || a.Ws > W;
    a.nx = a.nblk + (border ? 1 : 0);
    a.cy = (C + 63) / 64;
    a.copy_blocks = a.nx * a.cy * n;
    a.wp = wp;
    const int64_t wn = (int64_t)wp.cout * wp.cin * wp.taps;
    const int wblocks = wp.w ? (int)std::min<int64_t>((wn + 255) / 256, 1024) : 0;
    const dim3 grid((unsigned)(a.copy_blocks + wblocks));
    if (vec) hipLaunchKernelGGL(nchw_to_nhwc_kernel<true>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(nchw_to_nhwc_kernel<false>, grid, dim3(256), 0, s, a);
}

// Border that keeps rows lo + i*step + [tap_lo, tap_hi] for i in [0, count)
// (and likewise columns) inside the image after padding: the amounts by which
// the lowest index falls below 0 and the highest exceeds size - 1.
void border_for(int lo, int step, int count, int tap_lo, int tap_hi, int size, int& before, int& after) {
    before = std::max(before, -(lo + tap_lo));
    after = std::max(after, lo + (count - 1) * step + tap_hi - (size - 1));
}

// ---------------------------------------------------------------------------
// Stride-1 3x3 "same" convolution (padding 1) straight from NCHW: forward
// (source x) and grad input (source dy, taps mirrored). A workgroup computes
// TR x W output pixels (TR * W = 512, W in 8..64) x 64 output channels, 8
// waves of 64 pixels (two per SIMD, so one wave's LDS waits overlap the
// other's MFMAs). Per
// 32-channel k chunk it stages the (TR + 2) x (W + 2) source halo in LDS
// ([pixel][32 channels], 64-byte rows, the 16-byte chunks XOR-swizzled by
// hl_swz(pixel)) and the permuted weight's [9 taps][64 channels][32] rows,
// then all 9 taps read their A fragments from the halo at a shifted pixel:
// each source element crosses from L2 once per chunk instead of once per tap.
// The halo is gathered into registers (a lane: 8 channels x 8 pixels of one
// row, 16-byte loads, an in-register 8x8 transpose, 16-byte LDS stores); the
// weight rows go straight to LDS. Two stages: chunk k + 1 loads while k
// computes.
// ---------------------------------------------------------------------------
constexpr int HL_BN = 64;
constexpr int HL_PX = 512;      // output pixels a tile
constexpr int HL_A = 43008;     // halo pixels (TR + 2) * (W + 2) <= 660 (largest at W = 8 and 64) * 64 bytes, rounded up to 1 KB
constexpr int HL_B = 9 * HL_BN * 64;

// The stride-1 kernel's two tile sizes: 512 output pixels on 8 waves with
// two LDS stages (156 KB: one workgroup a CU), or 256 pixels on 4 waves with
// one stage (61 KB: two workgroups a CU, which overlap each other's loads,
// prologue and epilogue), for grids that would leave the CUs one 512-pixel
// workgroup or less each.
template <int PX>
struct HaloCfg {
    static constexpr int NT = PX, NW = PX / 64;
    static constexpr int NS = PX == 512 ? 2 : 1;
    static constexpr int A = PX == 512 ? HL_A : 25600;   // (TR + 2) * (W + 2) <= 396 pixels x 64 bytes at 256
    static constexpr int STAGE = A + HL_B;
    static constexpr int NQ = (36 + NW - 1) / NW;       // weight-row loads per wave
    static_assert(PX == 512 || PX == 256, "tile");
    static_assert(HL_BN * (PX + 8) * 2 <= NS * STAGE, "the epilogue tile fits the stages");
};

struct HaloArgs {
    const uint16_t* src;   // x (forward) or dy (grad input), NCHW [n][Cs][H][W]
    const void* wt;        // permuted weight [N][9][Cs]
    const void* bias;      // forward
    void* out;             // y or dx, NCHW [n][N][H][W]
    int Cs, N, H, W, tr, row_tiles;
    int dtap[9];           // halo pixel offset of each tap: hoff * (W + 2) + woff
    int has_bias;
    int wt_bytes;
    int ipt, nimg;         // stride-2 grad input: images a tile, batch size
    const uint16_t* wraw;  // forward on 256 threads: the weight as given, [N][Cs][3][3] (no permuted copy)
};

// 16-byte chunk swizzle of the 64-byte LDS rows (halo pixels and weight rows):
// chunk c of row r sits at c ^ hl_swz(r). A fragment read takes 16
// consecutive rows, chunk g = lane / 16; with gfx950's ds_read_b128 lane
// groups ({0-3, 12-15} of one 16 and {4-11} of the other, served together)
// flipping bit 1 of the chunk every 4 rows spreads every group over the 64
// banks for any first row, where a 4-row rotation left 2-way conflicts.
__device__ inline int hl_swz(int row) { return ((row >> 2) & 1) * 2; }

// Forward weight rows of one 32-channel chunk gathered by the conv kernel
// itself from the weight as given ([N][Cs][3][3]), in place of the permuted
// copy's LDS-DMA: thread t of 256 takes output channel t / 4 of the tile's 64
// and input channels 8 * (t % 4) .. + 7 of the chunk, whose 72 halves (8
// channels x 9 taps) are one contiguous, 16-byte aligned run: nine 16-byte
// loads, then the 8 x 9 transpose in registers (two halves a dword) and nine
// 16-byte LDS stores, one per tap row (tap * 64 + channel, the permuted
// layout's rows). Saves the permute launch of every forward call.
struct RawWeights {
    u32x4 v[9];
    __device__ inline void load(const uint16_t* w, int co, int Cs, int kc, int cg) {
        load_at(w + ((int64_t)co * Cs + kc * 32 + cg * 8) * 9);
    }
    __device__ inline void load_at(const uint16_t* run) {   // the 72-half run (16-byte aligned)
        const u32x4* src = reinterpret_cast<const u32x4*>(run);
#pragma unroll
        for (int j = 0; j < 9; ++j) v[j] = src[j];
    }
    __device__ inline uint32_t half_at(int a) const {   // half a of the 72-half run, in the low 16 bits
        const uint32_t d = v[a / 8][(a / 2) % 4];
        return (a % 2) ? (d >> 16) : (d & 0xffffu);
    }
    __device__ inline void store(char* rows, int col, int cg) const {
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            uint32_t o[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) o[m] = half_at(2 * m * 9 + t) | (half_at((2 * m + 1) * 9 + t) << 16);
            const int row = t * 64 + col;
            *reinterpret_cast<u32x4*>(rows + row * 64 + ((cg ^ hl_swz(row)) * 16)) = u32x4{o[0], o[1], o[2], o[3]};
        }
    }
    // Grad input: the run holds 8 input channels (its output columns) of one
    // output channel (a k row), and the B tile is kept k-major, [tap][32 k
    // rows][64 columns], 128-byte rows read back with transposed reads
    // (ds_read_b64_tr_b16); k row kr, 16-byte chunk cg at cg ^ hl_swz_t(kr)
    __device__ inline void store_t(char* rows, int kr, int cg) const;
    // the same with 64-byte rows (32 columns)
    __device__ inline void store_t64(char* rows, int kr, int cg) const;
};

// Chunk swizzle of the grad input's k-major weight rows (128 bytes, 8 chunks):
// a transposed fragment read takes k rows {0-3, 8-11} (+ 4) at one chunk pair,
// which this spreads over the 8 32-byte bank groups of a 256-byte window.
__device__ inline int hl_swz_t(int kr) { return (((kr >> 1) & 1) | ((kr >> 2) & 2)) * 2; }

// With 64-byte rows (four per 256-byte window) the pair of k rows kr and
// kr + 8 of a transposed read shares a window position; flipping the chunk
// pair for kr & 8 separates them.
__device__ inline int hl_swz_t64(int kr) { return ((kr >> 3) & 1) * 2; }

__device__ inline void RawWeights::store_t64(char* rows, int kr, int cg) const {
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = half_at(2 * m * 9 + t) | (half_at((2 * m + 1) * 9 + t) << 16);
        *reinterpret_cast<u32x4*>(rows + (t * 32 + kr) * 64 + ((cg ^ hl_swz_t64(kr)) * 16)) = u32x4{o[0], o[1], o[2], o[3]};
    }
}

__device__ inline void RawWeights::store_t(char* rows, int kr, int cg) const {
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = half_at(2 * m * 9 + t) | (half_at((2 * m + 1) * 9 + t) << 16);
        *reinterpret_cast<u32x4*>(rows + (t * 32 + kr) * 128 + ((cg ^ hl_swz_t(kr)) * 16)) = u32x4{o[0], o[1], o[2], o[3]};
    }
}

// 3x3 weight w[co][c][9] -> forward wout[co][t][c] or grad input
// wout[c][t][co], the reduced channel count a multiple of 8: a thread gathers
// 8 consecutive reduced channels of one (row, tap) and writes them as one
// 16-byte store.
template <bool FWD>
__global__ __launch_bounds__(256) void weight_permute9_kernel(const uint16_t* w, uint16_t* out, int cout, int cin) {
    const int rows = FWD ? cout : cin, red = FWD ? cin : cout;
    const int groups = red / 8, total = rows * 9 * groups;
    for (int e = blockIdx.x * 256 + (int)threadIdx.x; e < total; e += (int)gridDim.x * 256) {
        const int gi = e % groups, rest = e / groups;
        const int t = rest % 9, r = rest / 9;
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int c0 = gi * 8 + 2 * k;
            const uint32_t lo = FWD ? w[(r * cin + c0) * 9 + t] : w[(c0 * cin + r) * 9 + t];
            const uint32_t hi = FWD ? w[(r * cin + c0 + 1) * 9 + t] : w[((c0 + 1) * cin + r) * 9 + t];
            v[k] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x4*>(out + (r * 9 + t) * red + gi * 8) = u32x4{v[0], v[1], v[2], v[3]};
    }
}

// TB: grad input with its weight rows gathered from the weight as given
// (k-major B tile, transposed fragment reads); 256-pixel tiles only.
template <int DT, int PX, bool TB = false>
__global__ __launch_bounds__(PX) void conv_halo_kernel(HaloArgs p) {
    typedef HaloCfg<PX> G;
    constexpr int NT = G::NT, NS = G::NS, STG = G::STAGE, A_BYTES = G::A, NQ = G::NQ, NW = G::NW;
    __shared__ __attribute__((aligned(1024))) char lds[NS * STG];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64), g = lane / 16;
    const int img = blockIdx.x / p.row_tiles, h0 = (blockIdx.x - img * p.row_tiles) * p.tr;
    const int n0 = blockIdx.y * HL_BN;
    const int W = p.W, WP = W + 2, HWs = p.H * W;
    const int nk = p.Cs / 32;

    // zero halo columns 0 and W + 1 of every stage (no load writes them)
    for (int e = tid; e < (p.tr + 2) * 8; e += NT) {
        const int hr = e / 8, hc = (e / 4) % 2 ? W + 1 : 0, ch = e % 4;
        const int hp = hr * WP + hc;
#pragma unroll
        for (int st = 0; st < NS; ++st)
            *reinterpret_cast<u32x4*>(lds + st * STG + hp * 64 + ch * 16) = u32x4{0u, 0u, 0u, 0u};
    }

    // halo gather: lane -> (column group wq, channel group cg, halo row hr)
    const int nwq = W / 8;
    const int wq = tid % nwq, cg = (tid / nwq) % 4, hr = tid / (nwq * 4);
    const bool a_live = hr < p.tr + 2;
    const int ih = h0 - 1 + hr;
    const bool a_row = a_live && ih >= 0 && ih < p.H;
    const uint16_t* a_src = p.src + ((int64_t)img * p.Cs + cg * 8) * HWs + (int64_t)(a_row ? ih : 0) * W + wq * 8;
    u32x4 ar[8];
    auto load_a = [&](int kc) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ar[i] = a_row ? *reinterpret_cast<const u32x4*>(a_src + (int64_t)(kc * 32 + i) * HWs) : u32x4{0u, 0u, 0u, 0u};
    };
    auto store_a = [&](int st) {
        if (!a_live) return;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = ar[2 * k][j / 2], hi = ar[2 * k + 1][j / 2];
                v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
            }
            const int hp = hr * WP + wq * 8 + j + 1;
            *reinterpret_cast<u32x4*>(lds + st * STG + hp * 64 + ((cg ^ hl_swz(hp)) * 16)) = u32x4{v[0], v[1], v[2], v[3]};
        }
    };

    // weight rows: 36 DMA instructions of 16 rows a chunk, instruction q * NW + wave
    // (at 8 waves, waves 0-3 issue 5 and waves 4-7 issue 4); row = tap * 64 + channel
    const i32x4 rb = v_rsrc(p.wt, p.wt_bytes);
    int b_off[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int row = min(q * NW + wave, 35) * 16 + lane / 4;
        const int t = row / HL_BN, co = min(n0 + row % HL_BN, p.N - 1);
        b_off[q] = ((co * 9 + t) * p.Cs + (((lane % 4) ^ hl_swz(row)) * 8)) * 2;
    }
    auto issue_b = [&](int kc, int st) {
        const uint32_t base = lds0 + (uint32_t)(st * STG + A_BYTES);
#pragma unroll
        for (int q = 0; q < NQ; ++q)
            if (q * NW + wave < 36) v_dma16(rb, base + (uint32_t)((q * NW + wave) * 1024), (uint32_t)(b_off[q] + kc * 64));
    };

    // A fragment rows: this wave's 64 pixels of the tile, 16 per fragment
    int hp0[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = wave * 64 + i * 16 + lane % 16;
        const int r = q / W, c = q - r * W;
        hp0[i] = (r + 1) * WP + c + 1;
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // the nine taps of one chunk from stage `cur`
    auto compute = [&](int cur) {
        const char* sa = lds + cur * STG;
        const char* sb = sa + A_BYTES;
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            u32x4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int hp = hp0[i] + p.dtap[t];
                fa[i] = *reinterpret_cast<const u32x4*>(sa + hp * 64 + ((g ^ hl_swz(hp)) * 16));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (TB) {
                    // source lane s of group g points at k row 8g + 4rr + s/4, columns
                    // 4(s%4)..+3 of this fragment; the transpose hands lane s the four
                    // k values of its column
                    const int sl = lane % 16, col = j * 16 + (sl % 4) * 4;
#pragma unroll
                    for (int rr = 0; rr < 2; ++rr) {
                        const int kr = g * 8 + rr * 4 + sl / 4;
                        TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(TVK_LDS const char*)(
                            sb + (t * 32 + kr) * 128 + (((col / 8) ^ hl_swz_t(kr)) * 16) + (col % 8) * 2);
                        const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
                        fb[j][rr * 2] = w.x;
                        fb[j][rr * 2 + 1] = w.y;
                    }
                } else {
                    const int row = t * HL_BN + j * 16 + lane % 16;
                    fb[j] = *reinterpret_cast<const u32x4*>(sb + row * 64 + ((g ^ hl_swz(row)) * 16));
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = vmfma<DT>(fa[i], fb[j], acc[i][j]);
        }
    };

    static_assert(!TB || PX == 256, "the k-major weight tile is gathered on 256 threads");
    if constexpr (NS == 2) {
        issue_b(0, 0);
        load_a(0);
        store_a(0);
        v_wait<0>();
        __syncthreads();
        for (int kc = 0; kc < nk; ++kc) {
            const int cur = kc & 1;
            if (kc + 1 < nk) {
                issue_b(kc + 1, cur ^ 1);
                load_a(kc + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(cur);
            __builtin_amdgcn_sched_barrier(0);
            if (kc + 1 < nk) store_a(cur ^ 1);
            v_wait<0>();
            __syncthreads();
        }
    } else {
        // one stage: each chunk loads after every wave has read the previous one
        RawWeights rw;
        const int rw_co = min(n0 + tid / 4, p.N - 1), rw_cg = tid % 4;
        // grad input: k row tid / 8 of the chunk, input channels 8 (tid % 8) .. + 7 of the tile
        const int rt_kr = tid / 8, rt_cg = tid % 8, rt_c0 = min(n0 + rt_cg * 8, p.N - 8);
        for (int kc = 0; kc < nk; ++kc) {
            if (kc > 0) __syncthreads();
            if constexpr (TB) rw.load_at(p.wraw + ((int64_t)(kc * 32 + rt_kr) * p.N + rt_c0) * 9);
            else if (p.wraw) rw.load(p.wraw, rw_co, p.Cs, kc, rw_cg);
            else issue_b(kc, 0);
            load_a(kc);
            store_a(0);
            if constexpr (TB) rw.store_t(lds + A_BYTES, rt_kr, rt_cg);
            else if (p.wraw) rw.store(lds + A_BYTES, tid / 4, rw_cg);
            v_wait<0>();
            __syncthreads();
            compute(0);
        }
        __syncthreads();
    }

    // [channel][pixel] tile, then 16-byte stores along the output rows
    typedef typename elem<DT>::T T;
    constexpr int LROW = PX + 8;
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ch = j * 16 + lane % 16;
        float bv = 0.0f;
        if (p.has_bias && n0 + ch < p.N) bv = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[n0 + ch]);
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
    uint16_t* out = static_cast<uint16_t*>(p.out);
    for (int idx = tid; idx < HL_BN * (PX / 8); idx += NT) {
        const int ch = idx / (PX / 8), px = (idx % (PX / 8)) * 8;
        const int r = px / W, c = px - r * W;
        if (n0 + ch >= p.N || h0 + r >= p.H) continue;
        st_nt(reinterpret_cast<u32x4*>(out + ((int64_t)img * p.N + n0 + ch) * HWs + (int64_t)(h0 + r) * W + c), *reinterpret_cast<const u32x4*>(tile + ch * LROW + px));
    }
}

// Stride-2 3x3 padding-1 forward from NCHW (W = 2 Wo, H = 2 Ho): the same
// scheme as the stride-1 halo kernel on a 64 * FM output-pixel tile (TR x Wo
// of one image, or ipt whole images of TR = Ho rows where an image has fewer
// pixels) x 64 output channels, 4 waves of 16 * FM pixels. The (2 TR + 1)-row input
// halo is stored with its columns de-interleaved: column hc = iw + 1 goes to
// slot hc / 2 when even and W / 2 + 1 + hc / 2 when odd, so the 16 output
// pixels of a fragment read 16 consecutive slots for every tap (tap column b:
// even slots from c + b / 2, odd slots from W / 2 + 1 + c).
constexpr int H2_A = 41984;      // ipt (2 TR + 1) x (W + 2) slots x 64 bytes <= 656 x 64
constexpr int H2_STAGE = H2_A + HL_B;

// NS: LDS stages, 2 (chunk k + 1 loads while k computes; 157 KB, one
// workgroup a CU) or 1 (78 KB: two workgroups a CU, for grids of more
// workgroups than CUs, which would otherwise run in two rounds).
template <int DT, int FM, int NS>
__global__ __launch_bounds__(256) void conv_halo_s2_kernel(HaloArgs p) {
    constexpr int TPX = 64 * FM;
    __shared__ __attribute__((aligned(1024))) char lds[NS * H2_STAGE];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64), g = lane / 16;
    const int img0 = (blockIdx.x / p.row_tiles) * p.ipt, h0 = (blockIdx.x % p.row_tiles) * p.tr;   // output rows
    const int n0 = blockIdx.y * HL_BN;
    const int W = p.W, RP = W + 2, HWs = p.H * W, Wo = W / 2, Ho = p.H / 2;
    const int HRI = 2 * p.tr + 1, HR = p.ipt * HRI, ODD = W / 2 + 1, ppi = p.tr * Wo;
    const int nk = p.Cs / 32;

    // zero halo column hc = 0 (input column -1: even slot 0) of every stage
    for (int e = tid; e < HR * 4; e += 256) {
        const int hr = e / 4, ch = e % 4, hp = hr * RP;
#pragma unroll
        for (int st = 0; st < NS; ++st)
            *reinterpret_cast<u32x4*>(lds + st * H2_STAGE + hp * 64 + ch * 16) = u32x4{0u, 0u, 0u, 0u};
    }

    // halo gather: block b -> (column group wq, channel group cg, halo row hr
    // = image k of the tile, row 2 h0 - 1 + hr % HRI); up to two a thread
    const int nwq = W / 8, nblk = HR * nwq * 4;
    u32x4 ar[2][8];
    auto load_a = [&](int kc) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int b = tid + u * 256;
            const int wq = b % nwq, cg = (b / nwq) % 4, hr = b / (nwq * 4);
            const int k = hr / HRI, ih = 2 * h0 - 1 + hr % HRI;
            const bool row = b < nblk && ih >= 0 && ih < p.H && img0 + k < p.nimg;
            const uint16_t* src = p.src + ((int64_t)(row ? img0 + k : 0) * p.Cs + kc * 32 + cg * 8) * HWs + (int64_t)(row ? ih : 0) * W + wq * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                ar[u][i] = row ? *reinterpret_cast<const u32x4*>(src + (int64_t)i * HWs) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store_a = [&](int st) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int b = tid + u * 256;
            if (b >= nblk) continue;
            const int wq = b % nwq, cg = (b / nwq) % 4, hr = b / (nwq * 4);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t v[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t lo = ar[u][2 * k][j / 2], hi = ar[u][2 * k + 1][j / 2];
                    v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
                }
                const int hc = wq * 8 + j + 1;
                const int hp = hr * RP + ((hc & 1) ? ODD + hc / 2 : hc / 2);
                *reinterpret_cast<u32x4*>(lds + st * H2_STAGE + hp * 64 + ((cg ^ hl_swz(hp)) * 16)) = u32x4{v[0], v[1], v[2], v[3]};
            }
        }
    };

    // weight rows: 36 DMA instructions of 16 rows a chunk, 9 per wave; row = tap * 64 + channel
    const i32x4 rb = v_rsrc(p.wt, p.wt_bytes);
    int b_off[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) {
        const int row = (wave * 9 + q) * 16 + lane / 4;
        const int t = row / HL_BN, co = min(n0 + row % HL_BN, p.N - 1);
        b_off[q] = ((co * 9 + t) * p.Cs + (((lane % 4) ^ hl_swz(row)) * 8)) * 2;
    }
    auto issue_b = [&](int kc, int st) {
        const uint32_t base = lds0 + (uint32_t)(st * H2_STAGE + H2_A);
#pragma unroll
        for (int q = 0; q < 9; ++q) v_dma16(rb, base + (uint32_t)((wave * 9 + q) * 1024), (uint32_t)(b_off[q] + kc * 64));
    };

    // A fragment rows: this wave's 16 * FM output pixels of the tile
    int hp0[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int q = wave * 16 * FM + i * 16 + lane % 16;
        const int k = q / ppi, rem = q - k * ppi, r = rem / Wo, c = rem - r * Wo;
        hp0[i] = (k * HRI + 2 * r) * RP + c;
    }
    f32x4 acc[FM][4];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // the nine taps of one chunk from stage `cur`
    auto compute = [&](int cur) {
        const char* sa = lds + cur * H2_STAGE;
        const char* sb = sa + H2_A;
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            u32x4 fa[FM], fb[4];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int hp = hp0[i] + p.dtap[t];
                fa[i] = *reinterpret_cast<const u32x4*>(sa + hp * 64 + ((g ^ hl_swz(hp)) * 16));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = t * HL_BN + j * 16 + lane % 16;
                fb[j] = *reinterpret_cast<const u32x4*>(sb + row * 64 + ((g ^ hl_swz(row)) * 16));
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = vmfma<DT>(fa[i], fb[j], acc[i][j]);
        }
    };

    RawWeights rw;
    const int rw_co = min(n0 + tid / 4, p.N - 1), rw_cg = tid % 4;
    if constexpr (NS == 2) {
        if (p.wraw) rw.load(p.wraw, rw_co, p.Cs, 0, rw_cg);
        else issue_b(0, 0);
        load_a(0);
        store_a(0);
        if (p.wraw) rw.store(lds + H2_A, tid / 4, rw_cg);
        v_wait<0>();
        __syncthreads();
        for (int kc = 0; kc < nk; ++kc) {
            const int cur = kc & 1;
            if (kc + 1 < nk) {
                if (p.wraw) rw.load(p.wraw, rw_co, p.Cs, kc + 1, rw_cg);
                else issue_b(kc + 1, cur ^ 1);
                load_a(kc + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(cur);
            __builtin_amdgcn_sched_barrier(0);
            if (kc + 1 < nk) {
                store_a(cur ^ 1);
                if (p.wraw) rw.store(lds + (cur ^ 1) * H2_STAGE + H2_A, tid / 4, rw_cg);
            }
            v_wait<0>();
            __syncthreads();
        }
    } else {
        // one stage: each chunk loads after every wave has read the previous one
        for (int kc = 0; kc < nk; ++kc) {
            if (kc > 0) __syncthreads();
            if (p.wraw) rw.load(p.wraw, rw_co, p.Cs, kc, rw_cg);
            else issue_b(kc, 0);
            load_a(kc);
            store_a(0);
            if (p.wraw) rw.store(lds + H2_A, tid / 4, rw_cg);
            v_wait<0>();
            __syncthreads();
            compute(0);
        }
        __syncthreads();
    }

    // [channel][pixel] tile, then 16-byte stores along the output rows
    typedef typename elem<DT>::T T;
    constexpr int LROW = TPX + 8;
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ch = j * 16 + lane % 16;
        float bv = 0.0f;
        if (p.has_bias && n0 + ch < p.N) bv = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[n0 + ch]);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
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
            const int px = wave * 16 * FM + i * 16 + g * 4;
            *reinterpret_cast<u32x2*>(tile + ch * LROW + px) = u32x2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
        }
    }
    __syncthreads();
    uint16_t* out = static_cast<uint16_t*>(p.out);
    const int HWo = Ho * Wo;
    for (int idx = tid; idx < HL_BN * (TPX / 8); idx += 256) {
        const int ch = idx / (TPX / 8), px = (idx % (TPX / 8)) * 8;
        const int k = px / ppi, rem = px - k * ppi, r = rem / Wo;
        if (n0 + ch >= p.N || h0 + r >= Ho || img0 + k >= p.nimg) continue;
        st_nt(reinterpret_cast<u32x4*>(out + ((int64_t)(img0 + k) * p.N + n0 + ch) * HWo + (int64_t)h0 * Wo + rem), *reinterpret_cast<const u32x4*>(tile + ch * LROW + px));
    }
}

// Stride-2 3x3 padding-1 grad input from NCHW dy (H = 2 Ho, W = 2 Wo). The
// output splits by pixel parity into four phases (ph, pw) = (h % 2, w % 2):
// dx(2i + ph, 2j + pw) sums the taps a with (ph + 1 - a) even, reading dy row
// i + (ph + 1 - a) / 2, and likewise b for the columns, so the phases take 1,
// 2, 2 and 4 of the 9 taps and no product is a zero of the strided grid. A
// workgroup takes TP dy positions (ipt images x tr rows x Wo) x BN input
// channels. Its 8 waves take one phase and half of the positions each: waves
// 0-1 phase (0,0), 2-3 (0,1), 4-5 (1,1), 6-7 (1,0), so waves w and w + 4,
// which share a SIMD, run 5 or 4 taps between them. Per 32-channel chunk the
// dy halo [ipt][tr + 1][Wo + 1] (the last row and column past the image are
// zeros) is staged as in the stride-1 kernel, with the permuted weight rows.
// ---------------------------------------------------------------------------
constexpr int D2_A = 13312;   // ipt (tr + 1) (Wo + 1) pixels x 64 bytes: 3 x 65 at Wo = 64, 18 x 9 at Wo = 8
constexpr int D2_STAGE = D2_A + HL_B;

// TB: weight rows gathered from the weight as given into a k-major tile
// ([tap][32 k rows][BN columns]) read by transposed fragment reads.
template <int DT, int TP, int BN, bool TB = false>
__global__ __launch_bounds__(512) void conv_halo_dgrad_s2_kernel(HaloArgs p) {
    constexpr int FMW = TP / 32;   // A fragments a wave (TP / 2 positions)
    constexpr int FN = BN / 16;    // B fragments (input-channel columns)
    constexpr int NBI = 9 * BN / 16, QB = (NBI + 7) / 8;   // weight DMA instructions a chunk; per wave
    constexpr int LROW = 4 * TP + 8;
    static_assert(BN * LROW * 2 <= 2 * D2_STAGE && 9 * BN * 64 <= HL_B, "tiles fit the stages");
    __shared__ __attribute__((aligned(1024))) char lds[2 * D2_STAGE];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64), g = lane / 16;
    const int Wo = p.W / 2, Ho = p.H / 2, TR = p.tr, RP = Wo + 1, HR = p.ipt * (TR + 1), HWo = Ho * Wo;
    const int img0 = (blockIdx.x / p.row_tiles) * p.ipt, i0 = (blockIdx.x % p.row_tiles) * TR;
    const int n0 = blockIdx.y * BN;
    const int nk = p.Cs / 32;

    // zero halo column Wo of every row of both stages (no load writes it)
    for (int e = tid; e < HR * 4; e += 512) {
        const int hp = (e / 4) * RP + Wo, ch = e % 4;
#pragma unroll
        for (int st = 0; st < 2; ++st)
            *reinterpret_cast<u32x4*>(lds + st * D2_STAGE + hp * 64 + ch * 16) = u32x4{0u, 0u, 0u, 0u};
    }

    // halo gather: thread -> (column group wq, channel group cg, halo row hr
    // = image k of the tile, row r); rows past the image or the batch load zeros
    const int nwq = Wo / 8, nblk = HR * nwq * 4;
    const int wq = tid % nwq, cg = (tid / nwq) % 4, hr = tid / (nwq * 4);
    const int hk = hr / (TR + 1), hi = i0 + hr % (TR + 1);
    const bool a_live = tid < nblk;
    const bool a_row = a_live && hi < Ho && img0 + hk < p.nimg;
    const uint16_t* a_src = p.src + ((int64_t)(a_row ? img0 + hk : 0) * p.Cs + cg * 8) * HWo + (int64_t)(a_row ? hi : 0) * Wo + wq * 8;
    u32x4 ar[8];
    auto load_a = [&](int kc) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ar[i] = a_row ? *reinterpret_cast<const u32x4*>(a_src + (int64_t)(kc * 32 + i) * HWo) : u32x4{0u, 0u, 0u, 0u};
    };
    auto store_a = [&](int st) {
        if (!a_live) return;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = ar[2 * k][j / 2], hi2 = ar[2 * k + 1][j / 2];
                v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi2 << 16)) : ((lo >> 16) | (hi2 & 0xffff0000u));
            }
            const int hp = hr * RP + wq * 8 + j;
            *reinterpret_cast<u32x4*>(lds + st * D2_STAGE + hp * 64 + ((cg ^ hl_swz(hp)) * 16)) = u32x4{v[0], v[1], v[2], v[3]};
        }
    };

    // weight rows: NBI DMA instructions of 16 rows a chunk, instruction q * 8 + wave;
    // row = tap * BN + channel
    const i32x4 rb = v_rsrc(p.wt, p.wt_bytes);
    int b_off[QB];
#pragma unroll
    for (int q = 0; q < QB; ++q) {
        const int row = min(q * 8 + wave, NBI - 1) * 16 + lane / 4;
        const int t = row / BN, co = min(n0 + row % BN, p.N - 1);
        b_off[q] = ((co * 9 + t) * p.Cs + (((lane % 4) ^ hl_swz(row)) * 8)) * 2;
    }
    auto issue_b = [&](int kc, int st) {
        const uint32_t base = lds0 + (uint32_t)(st * D2_STAGE + D2_A);
#pragma unroll
        for (int q = 0; q < QB; ++q)
            if (q * 8 + wave < NBI) v_dma16(rb, base + (uint32_t)((q * 8 + wave) * 1024), (uint32_t)(b_off[q] + kc * 64));
    };

    // this wave's phase and positions: q = half * TP / 2 + i * 16 + lane % 16
    const int ph = wave >= 4 ? 1 : 0, pw = (wave >= 2 && wave <= 5) ? 1 : 0, half = wave & 1;
    const int ppi = TR * Wo;   // positions of one image in the tile
    int hp0[FMW];
#pragma unroll
    for (int i = 0; i < FMW; ++i) {
        const int q = half * (TP / 2) + i * 16 + lane % 16;
        const int k = q / ppi, rem = q - k * ppi, r = rem / Wo, c = rem - r * Wo;
        hp0[i] = (k * (TR + 1) + r) * RP + c;
    }
    f32x4 acc[FMW][FN];
#pragma unroll
    for (int i = 0; i < FMW; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // k-major tile: task tid (< 32 BN / 8) = k row tid / (BN / 8), input channels 8 (tid % (BN / 8)) .. + 7
    constexpr int RTASKS = 32 * BN / 8;
    RawWeights rw;
    const int rt_kr = tid / (BN / 8), rt_cg = tid % (BN / 8), rt_c0 = min(n0 + rt_cg * 8, p.N - 8);
    auto raw_load = [&](int kc) {
        if (tid < RTASKS) rw.load_at(p.wraw + ((int64_t)(kc * 32 + rt_kr) * p.N + rt_c0) * 9);
    };
    auto raw_store = [&](int st) {
        if (tid >= RTASKS) return;
        char* rows = lds + st * D2_STAGE + D2_A;
        if constexpr (BN == 64) rw.store_t(rows, rt_kr, rt_cg);
        else rw.store_t64(rows, rt_kr, rt_cg);
    };
    if constexpr (TB) raw_load(0);
    else issue_b(0, 0);
    load_a(0);
    store_a(0);
    if constexpr (TB) raw_store(0);
    v_wait<0>();
    __syncthreads();
    const int na = ph ? 2 : 1, nb = pw ? 2 : 1;
    for (int kc = 0; kc < nk; ++kc) {
        const int cur = kc & 1;
        if (kc + 1 < nk) {
            if constexpr (TB) raw_load(kc + 1);
            else issue_b(kc + 1, cur ^ 1);
            load_a(kc + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        const char* sa = lds + cur * D2_STAGE;
        const char* sb = sa + D2_A;
        for (int ta = 0; ta < na; ++ta) {
            for (int tb = 0; tb < nb; ++tb) {
                const int a = ph ? 2 * ta : 1, b = pw ? 2 * tb : 1;
                const int off = ((ph + 1 - a) / 2) * RP + (pw + 1 - b) / 2, t = a * 3 + b;
                u32x4 fa[FMW], fb[FN];
#pragma unroll
                for (int i = 0; i < FMW; ++i) {
                    const int hp = hp0[i] + off;
                    fa[i] = *reinterpret_cast<const u32x4*>(sa + hp * 64 + ((g ^ hl_swz(hp)) * 16));
                }
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    if constexpr (TB) {
                        // lane s of group g points at k row 8g + 4rr + s/4, columns 4(s%4)..+3
                        const int sl = lane % 16, col = j * 16 + (sl % 4) * 4;
#pragma unroll
                        for (int rr = 0; rr < 2; ++rr) {
                            const int kr = g * 8 + rr * 4 + sl / 4;
                            const int sw = BN == 64 ? hl_swz_t(kr) : hl_swz_t64(kr);
                            TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(TVK_LDS const char*)(
                                sb + (t * 32 + kr) * (2 * BN) + (((col / 8) ^ sw) * 16) + (col % 8) * 2);
                            const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
                            fb[j][rr * 2] = w.x;
                            fb[j][rr * 2 + 1] = w.y;
                        }
                    } else {
                        const int row = t * BN + j * 16 + lane % 16;
                        fb[j] = *reinterpret_cast<const u32x4*>(sb + row * 64 + ((g ^ hl_swz(row)) * 16));
                    }
                }
#pragma unroll
                for (int i = 0; i < FMW; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = vmfma<DT>(fa[i], fb[j], acc[i][j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kc + 1 < nk) {
            store_a(cur ^ 1);
            if constexpr (TB) raw_store(cur ^ 1);
        }
        v_wait<0>();
        __syncthreads();
    }

    // [channel][dx pixel] tile over ipt x 2 tr x W pixels (the phases
    // interleave along the rows), then 16-byte stores along the dx rows
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int i = 0; i < FMW; ++i) {
        // accumulator rows g * 4 + r: positions q0 .. q0 + 3 of one dy row (Wo % 8 == 0)
        const int q0 = half * (TP / 2) + i * 16 + g * 4;
        const int k = q0 / ppi, rem = q0 - k * ppi, r = rem / Wo, c = rem - r * Wo;
        const int px0 = k * 4 * ppi + (2 * r + ph) * p.W + 2 * c + pw;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int ch = j * 16 + lane % 16;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                tile[ch * LROW + px0 + 2 * rr] = __builtin_bit_cast(uint16_t, elem<DT>::from_f32(acc[i][j][rr]));
        }
    }
    __syncthreads();
    uint16_t* out = static_cast<uint16_t*>(p.out);
    const int HW = p.H * p.W;
    for (int idx = tid; idx < BN * (TP / 2); idx += 512) {
        const int ch = idx / (TP / 2), px = (idx % (TP / 2)) * 8;
        const int k = px / (4 * ppi), rem = px - k * 4 * ppi;
        const int h = 2 * i0 + rem / p.W, w = rem % p.W;
        if (n0 + ch >= p.N || img0 + k >= p.nimg || h >= p.H) continue;
        st_nt(reinterpret_cast<u32x4*>(out + ((int64_t)(img0 + k) * p.N + n0 + ch) * HW + (int64_t)h * p.W + w), *reinterpret_cast<const u32x4*>(tile + ch * LROW + px));
    }
}

// Grad weight of the same convolution (stride 1, 3x3, padding 1) from NCHW:
// a workgroup takes 64 input channels x BN (64 or 32) output channels x all 9 taps and
// sums its share of 256-pixel tiles (TR x W output rows of one image, H % TR
// == 0, W = 16 or 32) into float32 partials [split][(tap, channel)][output
// channel]: C[c][co] += sum_p x(p + tap)[c] * dy[co][p]. The 36 row fragments
// (tap, 16 channels) go to 8 waves as w, w + 8, ... (waves 0-3 take five, 4-7
// four, so the two waves of each SIMD hold nine), each against all 64 columns.
// LDS per stage:
//   x halo [TR + 2][W + 4][64 channels], 128-byte pixel rows, 16-byte chunk c
//     at c ^ (pixel & 3) * 2 (the 16 lanes of a transposed read hit distinct
//     banks); the row pitch W + 4 makes a k step (32 pixels) a multiple of 4
//     pixels, so every fragment address of step s is step 0's plus a constant
//     (an instruction offset: no address arithmetic in the k loop);
//   dy [32 pixel chunks][BN output channels][8 pixels]: a fragment is 16 lanes
//     x 16 contiguous bytes, its offset again linear in the step; one LDS-DMA
//     instruction loads 1 KB, one pixel chunk of 64 channels or two of 32.
// With 32 output channels a workgroup sums twice the tiles of the 64-channel
// form for the same grid, which halves the float32 partials (the 64 -> 64
// layer's are otherwise 256 planes of 147 KB, written and read back once).
// A fragments are transposed reads (ds_read_b64_tr_b16) at the tap's shift.
// Two stages: tile i + 1 loads while i computes.
constexpr int HG_A = 46080;            // (TR + 2) * (W + 4) pixels x 128 bytes: 10 x 36 at W = 32, 18 x 20 at W = 16
constexpr int HG_B = 32 * 1024;
constexpr int HG_STAGE = HG_A + HG_B;

struct HaloWgArgs {
    const uint16_t* x;     // [n][cin][H][W]
    const void* dy;        // [n][cout][H][W]
    float* part;           // [split][9 * cin][cout]
    int cin, cout, H, tiles_per_img, ntiles, split;
    int dy_bytes;
};

__device__ inline int hg_swz(int hp) { return (hp & 3) * 2; }

template <int DT, int W, int BN = 64>
__global__ __launch_bounds__(512) void conv_halo_wgrad_kernel(HaloWgArgs p) {
    constexpr int FNB = BN / 16;   // column fragments; also the dy DMA instructions a wave
    constexpr int TR = 256 / W, WP = W + 4, STEP = (32 / W) * WP;   // halo pixels per k step
    static_assert(STEP % 4 == 0 && (TR + 2) * WP * 128 <= HG_A, "halo layout");
    __shared__ __attribute__((aligned(1024))) char lds[2 * HG_STAGE];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int g = lane / 16, sl = lane % 16;
    const int c0 = blockIdx.y * 64, n0 = blockIdx.z * BN;
    const int HWs = p.H * W;
    // row fragment k of this wave: rf = wave + 8k (k < 4, or 5 for waves 0-3), tap rf / 4, channels (rf % 4) * 16
    const bool five = wave < 4;
    const int cf = wave % 4;

    // zero halo columns 0 and W + 1 of both stages (no load writes them)
    for (int e = tid; e < (TR + 2) * 16; e += 512) {
        const int hr = e / 16, hc = (e / 8) % 2 ? W + 1 : 0, ch = e % 8;
        const int hp = hr * WP + hc;
#pragma unroll
        for (int st = 0; st < 2; ++st)
            *reinterpret_cast<u32x4*>(lds + st * HG_STAGE + hp * 128 + ch * 16) = u32x4{0u, 0u, 0u, 0u};
    }

    // x halo gather: lane -> (column group wq, channel group cg of 8, halo row hr)
    constexpr int NWQ = W / 8;
    const int wq = tid % NWQ, cg = (tid / NWQ) % 8, hr = tid / (NWQ * 8);
    const bool a_live = hr < TR + 2;
    u32x4 ar[8];
    auto load_a = [&](int tile) {
        const int img = tile / p.tiles_per_img, h0 = (tile - img * p.tiles_per_img) * TR;
        const int ih = h0 - 1 + hr;
        const bool row = a_live && ih >= 0 && ih < p.H;
        const uint16_t* src = p.x + ((int64_t)img * p.cin + c0 + cg * 8) * HWs + (int64_t)(row ? ih : 0) * W + wq * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) ar[i] = row ? *reinterpret_cast<const u32x4*>(src + (int64_t)i * HWs) : u32x4{0u, 0u, 0u, 0u};
    };
    auto store_a = [&](int st) {
        if (!a_live) return;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = ar[2 * k][j / 2], hi = ar[2 * k + 1][j / 2];
                v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
            }
            const int hp = hr * WP + wq * 8 + j + 1;
            *reinterpret_cast<u32x4*>(lds + st * HG_STAGE + hp * 128 + ((cg ^ hg_swz(hp)) * 16)) = u32x4{v[0], v[1], v[2], v[3]};
        }
    };

    // dy: DMA instruction u = wave * FNB + q loads 1 KB: pixel chunk u with lane =
    // output channel (BN = 64), or chunks 2u, 2u + 1 with lane = chunk half x 32
    // + output channel (BN = 32)
    const i32x4 rb = v_rsrc(p.dy, p.dy_bytes);
    const uint32_t b_lane = BN == 64 ? (uint32_t)(min(n0 + lane, p.cout - 1) * HWs * 2)
                                     : (uint32_t)(min(n0 + lane % 32, p.cout - 1) * HWs * 2 + (lane / 32) * 16);
    auto issue_b = [&](int tile, int st) {
        const int img = tile / p.tiles_per_img, h0 = (tile - img * p.tiles_per_img) * TR;
        const uint32_t toff = (uint32_t)((((int64_t)img * p.cout) * HWs + (int64_t)h0 * W) * 2);
        const uint32_t base = lds0 + (uint32_t)(st * HG_STAGE + HG_A);
#pragma unroll
        for (int q = 0; q < FNB; ++q) {
            const int u = wave * FNB + q;
            v_dma16(rb, base + (uint32_t)(u * 1024), b_lane + toff + (uint32_t)(u * (1024 / BN)));
        }
    };

    // fragment offsets at k step 0 (step s adds s * STEP pixels)
    int a_off[5][2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const int px = g * 8 + rr * 4 + sl / 4;
        const int hb = (px / W) * WP + px % W;
        const int col = cf * 16 + (sl % 4) * 4;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            const int t = min((wave + 8 * k) / 4, 8);
            const int hp = hb + (t / 3) * WP + t % 3;
            a_off[k][rr] = hp * 128 + (((col / 8) ^ hg_swz(hp)) * 16) + (col % 8) * 2;
        }
    }
    const int b_off = g * (BN * 16) + sl * 16;

    f32x4 acc[5][FNB];
#pragma unroll
    for (int i = 0; i < 5; ++i)
#pragma unroll
        for (int j = 0; j < FNB; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    int tile = blockIdx.x;
    if (tile < p.ntiles) {
        issue_b(tile, 0);
        load_a(tile);
        store_a(0);
    }
    v_wait<0>();
    __syncthreads();
    for (int it = 0; tile < p.ntiles; ++it, tile += p.split) {
        const int cur = it & 1;
        const int next = tile + p.split;
        if (next < p.ntiles) {
            issue_b(next, cur ^ 1);
            load_a(next);
        }
        __builtin_amdgcn_sched_barrier(0);
        const char* sa = lds + cur * HG_STAGE;
        const char* sb = sa + HG_A + b_off;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            // A: rows = 16 input channels of one tap, k = this step's 32 pixels (transposed reads)
            u32x4 fa[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                if (i == 4 && !five) break;
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const char* ptr = sa + a_off[i][rr] + ks * STEP * 128;
                    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((TVK_LDS s16x4*)(uintptr_t)(TVK_LDS const char*)ptr));
                    fa[i][rr * 2] = w.x;
                    fa[i][rr * 2 + 1] = w.y;
                }
            }
            // B: columns = 16 output channels, k = the same 32 pixels
            u32x4 fb[FNB];
#pragma unroll
            for (int j = 0; j < FNB; ++j) fb[j] = *reinterpret_cast<const u32x4*>(sb + ks * (64 * BN) + j * 256);
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                if (i == 4 && !five) break;
#pragma unroll
                for (int j = 0; j < FNB; ++j) acc[i][j] = vmfma<DT>(fa[i], fb[j], acc[i][j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (next < p.ntiles) store_a(cur ^ 1);
        v_wait<0>();
        __syncthreads();
    }

    // partial rows (tap, channel) of this wave's row fragments, columns = output channels
    float* part = p.part + (int64_t)blockIdx.x * 9 * p.cin * p.cout;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        if (i == 4 && !five) break;
        const int t = (wave + 8 * i) / 4;
#pragma unroll
        for (int j = 0; j < FNB; ++j) {
            const int co = n0 + j * 16 + sl;
            if (co >= p.cout) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = c0 + cf * 16 + g * 4 + r;
                part[((int64_t)t * p.cin + c) * p.cout + co] = acc[i][j][r];
            }
        }
    }
}

// Grad weight of the stride-2 3x3 padding-1 convolution from NCHW (W = 2 Wo,
// H = 2 Ho): a workgroup takes 32 input channels x 64 output channels x all 9
// taps and sums its share of TPX-pixel output tiles (TR x Wo rows of one
// image) into float32 partials [split][(tap, channel)][output channel]. LDS
// per stage: the (2 TR + 1)-row x halo with de-interleaved columns (as the
// stride-2 forward: tap column b of output pixel c is slot c + b / 2, or
// W / 2 + 1 + c for b = 1), [slot][32 channels] 64-byte rows, so a transposed
// read's 4 k-rows (output pixels) are 4 consecutive slots; dy as chunk-major
// [TPX / 8][64 output channels][8 pixels]. The 18 row fragments (tap, 16
// channels) go to 8 waves as w, w + 8, w + 16. A k step (32 output pixels)
// moves every fragment address by the same slot count, an instruction offset.
constexpr int HG2_A = 38912;   // (2 TR + 1) x (W + 2) slots x 64 bytes <= 594 x 64, rounded up to 1 KB
constexpr int HG2_B = 16 * 1024;
constexpr int HG2_STAGE = HG2_A + HG2_B;

template <int DT, int WO, int TPX>
__global__ __launch_bounds__(512) void conv_halo_wgrad_s2_kernel(HaloWgArgs p) {
    constexpr int W = 2 * WO, RP = W + 2, ODD = WO + 1, TR = TPX / WO, HR = 2 * TR + 1;
    constexpr int KS = TPX / 32, STEP = 2 * (32 / WO) * RP;   // k steps a tile; slots a k step
    static_assert(TPX % WO == 0 && 32 % WO == 0 && HR * RP * 64 <= HG2_A, "halo layout");
    __shared__ __attribute__((aligned(1024))) char lds[2 * HG2_STAGE];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int g = lane / 16, sl = lane % 16;
    const int c0 = blockIdx.y * 32, n0 = blockIdx.z * 64;
    const int HWs = p.H * W, HWo = (p.H / 2) * WO;
    const int nrf = wave < 2 ? 3 : 2;   // row fragments wave + 8k

    // zero slot 0 (input column -1) of every halo row, both stages
    for (int e = tid; e < HR * 4; e += 512) {
        const int hr = e / 4, ch = e % 4;
#pragma unroll
        for (int st = 0; st < 2; ++st)
            *reinterpret_cast<u32x4*>(lds + st * HG2_STAGE + hr * RP * 64 + ch * 16) = u32x4{0u, 0u, 0u, 0u};
    }

    // x halo gather: lane -> (column group wq, channel group cg of 8, halo row hr)
    constexpr int NWQ = W / 8;
    const int wq = tid % NWQ, cg = (tid / NWQ) % 4, hr = tid / (NWQ * 4);
    const bool a_live = hr < HR;
    u32x4 ar[8];
    auto load_a = [&](int tile) {
        const int img = tile / p.tiles_per_img, h0 = (tile - img * p.tiles_per_img) * TR;
        const int ih = 2 * h0 - 1 + hr;
        const bool row = a_live && ih >= 0 && ih < p.H;
        const uint16_t* src = p.x + ((int64_t)img * p.cin + c0 + cg * 8) * HWs + (int64_t)(row ? ih : 0) * W + wq * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) ar[i] = row ? *reinterpret_cast<const u32x4*>(src + (int64_t)i * HWs) : u32x4{0u, 0u, 0u, 0u};
    };
    auto store_a = [&](int st) {
        if (!a_live) return;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = ar[2 * k][j / 2], hi = ar[2 * k + 1][j / 2];
                v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
            }
            const int hc = wq * 8 + j + 1;
            const int slot = (hc & 1) ? ODD + hc / 2 : hc / 2;
            *reinterpret_cast<u32x4*>(lds + st * HG2_STAGE + (hr * RP + slot) * 64 + cg * 16) = u32x4{v[0], v[1], v[2], v[3]};
        }
    };

    // dy: DMA instruction wave + 8q loads output-pixel chunk wave + 8q: lane = output channel
    const i32x4 rb = v_rsrc(p.dy, p.dy_bytes);
    const uint32_t b_lane = (uint32_t)(min(n0 + lane, p.cout - 1) * HWo * 2);
    auto issue_b = [&](int tile, int st) {
        const int img = tile / p.tiles_per_img, h0 = (tile - img * p.tiles_per_img) * TR;
        const uint32_t toff = (uint32_t)((((int64_t)img * p.cout) * HWo + (int64_t)h0 * WO) * 2);
        const uint32_t base = lds0 + (uint32_t)(st * HG2_STAGE + HG2_A);
#pragma unroll
        for (int q = 0; q < TPX / 64; ++q) {
            const int chunk = wave + 8 * q;
            v_dma16(rb, base + (uint32_t)(chunk * 1024), b_lane + toff + (uint32_t)(chunk * 16));
        }
    };

    // fragment offsets at k step 0: row fragment k = wave + 8k -> tap rf / 2, channels (rf % 2) * 16
    int a_off[3][2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const int px = g * 8 + rr * 4 + sl / 4;
        const int hb = 2 * (px / WO) * RP + px % WO;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int rf = min(wave + 8 * k, 17), t = rf / 2, a = t / 3, b = t % 3;
            const int col = (rf % 2) * 16 + (sl % 4) * 4;
            const int hp = hb + a * RP + (b == 1 ? ODD : b / 2);
            a_off[k][rr] = hp * 64 + col * 2;
        }
    }
    const int b_off = g * 1024 + sl * 16;

    f32x4 acc[3][4];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    int tile = blockIdx.x;
    if (tile < p.ntiles) {
        issue_b(tile, 0);
        load_a(tile);
        store_a(0);
    }
    v_wait<0>();
    __syncthreads();
    for (int it = 0; tile < p.ntiles; ++it, tile += p.split) {
        const int cur = it & 1;
        const int next = tile + p.split;
        if (next < p.ntiles) {
            issue_b(next, cur ^ 1);
            load_a(next);
        }
        __builtin_amdgcn_sched_barrier(0);
        const char* sa = lds + cur * HG2_STAGE;
        const char* sb = sa + HG2_A + b_off;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 fa[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                if (i == 2 && nrf == 2) break;
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const char* ptr = sa + a_off[i][rr] + ks * STEP * 64;
                    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((TVK_LDS s16x4*)(uintptr_t)(TVK_LDS const char*)ptr));
                    fa[i][rr * 2] = w.x;
                    fa[i][rr * 2 + 1] = w.y;
                }
            }
            u32x4 fb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u32x4*>(sb + ks * 4096 + j * 256);
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                if (i == 2 && nrf == 2) break;
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = vmfma<DT>(fa[i], fb[j], acc[i][j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (next < p.ntiles) store_a(cur ^ 1);
        v_wait<0>();
        __syncthreads();
    }

    float* part = p.part + (int64_t)blockIdx.x * 9 * p.cin * p.cout;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (i == 2 && nrf == 2) break;
        const int rf = wave + 8 * i, t = rf / 2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int co = n0 + j * 16 + sl;
            if (co >= p.cout) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = c0 + (rf % 2) * 16 + g * 4 + r;
                part[((int64_t)t * p.cin + c) * p.cout + co] = acc[i][j][r];
            }
        }
    }
}

// Grad weight of a 1x1 convolution with stride 1 or 2 and no padding,
// straight from NCHW without LDS: dW[co][c] = sum_p x[c][s*p] * dy[co][p].
// The output pixels are the reduction, 32 a step (4 groups of 8 in one output
// row: Wo % 8 == 0, Ho * Wo % 32 == 0). A lane's A fragment is 8 consecutive
// pixels of one input channel: one 16-byte load at stride 1, or two and the
// even elements at stride 2; its B fragment is 8 pixels of one output channel,
// one 16-byte load. Workgroup = 64 input x 64 output channels; its 4 waves
// take alternate steps of the workgroup's pixel range and add their sums in
// wave order through LDS into float32 partials [split][c][co].
struct PointWgArgs {
    const uint16_t* x;     // [n][cin][H][W]
    const uint16_t* dy;    // [n][cout][Ho][Wo]
    float* part;
    int cin, cout, H, W, Ho, Wo, stride;
    int steps, steps_per_split, split;   // 32-pixel steps in all; per workgroup
};

template <int DT, int S>
__global__ __launch_bounds__(256) void conv1x1_wgrad_kernel(PointWgArgs p) {
    __shared__ float red[4][64 * 65];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, sl = lane % 16;
    const int c0 = blockIdx.y * 64, n0 = blockIdx.z * 64;
    const int HWo = p.Ho * p.Wo, HW = p.H * p.W;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int s0 = blockIdx.x * p.steps_per_split, s1 = min(s0 + p.steps_per_split, p.steps);
#pragma unroll 2
    for (int st = s0 + wave; st < s1; st += 4) {
        const int px = st * 32 + g * 8;                 // first of this lane's 8 output pixels
        const int img = px / HWo, o = px - img * HWo;
        const int oh = o / p.Wo, ow = o - oh * p.Wo;
        const uint16_t* xr = p.x + ((int64_t)img * p.cin + c0 + sl) * HW + (int64_t)oh * S * p.W + ow * S;
        const uint16_t* dr = p.dy + (int64_t)img * p.cout * HWo + o;
        u32x4 fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t* q = xr + (int64_t)i * 16 * HW;
            if constexpr (S == 1) {
                fa[i] = *reinterpret_cast<const u32x4*>(q);
            } else {
                const u32x4 lo = *reinterpret_cast<const u32x4*>(q), hi = *reinterpret_cast<const u32x4*>(q + 8);
                fa[i] = u32x4{(lo.x & 0xffffu) | (lo.y << 16), (lo.z & 0xffffu) | (lo.w << 16),
                              (hi.x & 0xffffu) | (hi.y << 16), (hi.z & 0xffffu) | (hi.w << 16)};
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u32x4*>(dr + (int64_t)min(n0 + j * 16 + sl, p.cout - 1) * HWo);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = vmfma<DT>(fa[i], fb[j], acc[i][j]);
    }
    // rows = input channels (i * 16 + g * 4 + r), columns = output channels (j * 16 + sl)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(i * 16 + g * 4 + r) * 65 + j * 16 + sl] = acc[i][j][r];
    __syncthreads();
    float* part = p.part + (int64_t)blockIdx.x * p.cin * p.cout;
    for (int e = tid; e < 64 * 64; e += 256) {
        const int cl = e / 64, col = e % 64;
        if (n0 + col >= p.cout) continue;
        const int at = cl * 65 + col;
        part[(int64_t)(c0 + cl) * p.cout + n0 + col] = ((red[0][at] + red[1][at]) + red[2][at]) + red[3][at];
    }
}

// Forward of a 1x1 convolution with stride 1 or 2 and no padding, straight
// from NCHW: a workgroup computes PT consecutive output pixels of one image
// (whole 8-pixel groups of output rows) x 64 output channels. The input
// pixels it reads (every channel) go to LDS once as [channel][PT pixels]
// (one 16-byte load per 8 pixels, or two and their even elements at stride
// 2; 16-byte chunks XOR-swizzled by (channel & 3) * 2) and the A fragments
// (pixels x 32 channels) are transposed reads; the B fragments are 16-byte
// loads of the weight rows. 4 waves of PT / 4 pixels; output through an LDS
// tile into 16-byte NCHW stores.
struct PointFwdArgs {
    const uint16_t* x;     // [n][cin][H][W]
    const uint16_t* w;     // [cout][cin]
    const void* bias;
    void* y;               // [n][cout][Ho][Wo]
    int cin, cout, H, W, Ho, Wo, tiles_per_img, has_bias;
};

template <int DT, int S, int PT>
__global__ __launch_bounds__(256) void conv1x1_fwd_kernel(PointFwdArgs p) {
    typedef typename elem<DT>::T T;
    constexpr int FM = PT / 64, RB = PT * 2, LROW = PT + 8;
    __shared__ __attribute__((aligned(16))) char lds[32768 * 2];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, sl = lane % 16;
    const int img = blockIdx.x / p.tiles_per_img, t0 = (blockIdx.x - img * p.tiles_per_img) * PT;
    const int n0 = blockIdx.y * 64;
    const int HW = p.H * p.W, HWo = p.Ho * p.Wo;
    // input tile: chunk q of channel row c holds output pixels t0 + 8q .. + 8
    const uint16_t* xi = p.x + (int64_t)img * p.cin * HW;
    for (int e = tid; e < p.cin * (PT / 8); e += 256) {
        const int c = e / (PT / 8), q = e - c * (PT / 8);
        const int o = t0 + q * 8, oh = o / p.Wo, ow = o - oh * p.Wo;
        const uint16_t* src = xi + (int64_t)c * HW + (int64_t)oh * S * p.W + ow * S;
        u32x4 v;
        if constexpr (S == 1) {
            v = *reinterpret_cast<const u32x4*>(src);
        } else {
            const u32x4 lo = *reinterpret_cast<const u32x4*>(src), hi = *reinterpret_cast<const u32x4*>(src + 8);
            v = u32x4{(lo.x & 0xffffu) | (lo.y << 16), (lo.z & 0xffffu) | (lo.w << 16), (hi.x & 0xffffu) | (hi.y << 16),
                      (hi.z & 0xffffu) | (hi.w << 16)};
        }
        *reinterpret_cast<u32x4*>(lds + c * RB + ((q ^ swz_mn(c)) * 16)) = v;
    }
    __syncthreads();
    const uint32_t lbase = (uint32_t)(uintptr_t)(TVK_LDS char*)lds;
    f32x4 acc[FM][4];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < p.cin; k0 += 32) {
        u32x4 fb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int co = min(n0 + j * 16 + sl, p.cout - 1);
            fb[j] = *reinterpret_cast<const u32x4*>(p.w + (int64_t)co * p.cin + k0 + g * 8);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            // A: 16 pixels x 32 channels, transposed reads of channel rows k0 + (g * 8 + rr * 4 + sl / 4)
            const int col = wave * (PT / 4) + i * 16 + (sl % 4) * 4;
            u32x4 fa;
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int kr = k0 + g * 8 + rr * 4 + sl / 4;
                TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(lbase + kr * RB + (((col / 8) ^ swz_mn(kr)) * 16) + (col % 8) * 2);
                const u32x2 w2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
                fa[rr * 2] = w2.x;
                fa[rr * 2 + 1] = w2.y;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = vmfma<DT>(fa, fb[j], acc[i][j]);
        }
    }
    __syncthreads();
    // [channel][pixel] tile, then 16-byte stores along the output plane
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ch = j * 16 + sl;
        float bv = 0.0f;
        if (p.has_bias && n0 + ch < p.cout) bv = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[n0 + ch]);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
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
            const int px = wave * (PT / 4) + i * 16 + g * 4;
            *reinterpret_cast<u32x2*>(tile + ch * LROW + px) = u32x2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
        }
    }
    __syncthreads();
    uint16_t* y = static_cast<uint16_t*>(p.y);
    for (int idx = tid; idx < 64 * (PT / 8); idx += 256) {
        const int ch = idx / (PT / 8), pc = idx % (PT / 8);
        if (n0 + ch >= p.cout) continue;
        st_nt(reinterpret_cast<u32x4*>(y + ((int64_t)img * p.cout + n0 + ch) * HWo + t0 + pc * 8), *reinterpret_cast<const u32x4*>(tile + ch * LROW + pc * 8));
    }
}

// Grad input of the same 1x1 convolution: dx[c][s*p] = sum_co W[co][c] *
// dy[co][p], zero at the pixels no output reaches (odd rows and columns at
// stride 2). A workgroup takes PT consecutive dy pixels of one image (whole
// 8-pixel row groups) x 64 input channels: dy[all co][PT] and W[all co][64]
// go to LDS as k-rows (16-byte chunks XOR-swizzled by (row & 3) * 2), and
// both fragments are transposed reads. Each 8-pixel dy group becomes 16
// pixels of dx row s*oh (values and zeros interleaved at stride 2) and, at
// stride 2, 16 zeros of row s*oh + 1: 16-byte stores.
struct PointDgArgs {
    const uint16_t* dy;    // [n][cout][Ho][Wo]
    const uint16_t* w;     // [cout][cin]
    void* dx;              // [n][cin][H][W]
    int cin, cout, H, W, Ho, Wo, tiles_per_img;
};

template <int DT, int S, int PT>
__global__ __launch_bounds__(256) void conv1x1_dgrad_kernel(PointDgArgs p) {
    constexpr int FM = PT / 64, RB = PT * 2, LROW = PT + 8;
    constexpr int DYB = PT == 256 ? 65536 : 32768;   // dy rows: up to 128 (PT 256) or 256 (PT 64) channels
    __shared__ __attribute__((aligned(16))) char lds[DYB + 32768];
    char* wl = lds + DYB;   // W[co][64 channels], 128-byte rows
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, sl = lane % 16;
    const int img = blockIdx.x / p.tiles_per_img, t0 = (blockIdx.x - img * p.tiles_per_img) * PT;
    const int c0 = blockIdx.y * 64;
    const int HWo = p.Ho * p.Wo;
    const uint16_t* dyi = p.dy + (int64_t)img * p.cout * HWo + t0;
    for (int e = tid; e < p.cout * (PT / 8); e += 256) {
        const int co = e / (PT / 8), q = e - co * (PT / 8);
        *reinterpret_cast<u32x4*>(lds + co * RB + ((q ^ swz_mn(co)) * 16)) =
            *reinterpret_cast<const u32x4*>(dyi + (int64_t)co * HWo + q * 8);
    }
    for (int e = tid; e < p.cout * 8; e += 256) {
        const int co = e / 8, q = e % 8;
        const int c = c0 + q * 8;
        *reinterpret_cast<u32x4*>(wl + co * 128 + ((q ^ swz_mn(co)) * 16)) =
            c + 8 <= p.cin ? *reinterpret_cast<const u32x4*>(p.w + (int64_t)co * p.cin + c) : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    const uint32_t lbase = (uint32_t)(uintptr_t)(TVK_LDS char*)lds, wbase = lbase + DYB;
    auto tr = [&](uint32_t base, int rb, int kr, int col) {
        TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(base + kr * rb + (((col / 8) ^ swz_mn(kr)) * 16) + (col % 8) * 2);
        return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
    };
    f32x4 acc[FM][4];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < p.cout; k0 += 32) {
        u32x4 fb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const u32x2 v = tr(wbase, 128, k0 + g * 8 + rr * 4 + sl / 4, j * 16 + (sl % 4) * 4);
                fb[j][rr * 2] = v.x;
                fb[j][rr * 2 + 1] = v.y;
            }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            u32x4 fa;
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const u32x2 v = tr(lbase, RB, k0 + g * 8 + rr * 4 + sl / 4, wave * (PT / 4) + i * 16 + (sl % 4) * 4);
                fa[rr * 2] = v.x;
                fa[rr * 2 + 1] = v.y;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = vmfma<DT>(fa, fb[j], acc[i][j]);
        }
    }
    __syncthreads();
    uint16_t* tile = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ch = j * 16 + sl;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            uint16_t h[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) h[r] = __builtin_bit_cast(uint16_t, elem<DT>::from_f32(acc[i][j][r]));
            const int px = wave * (PT / 4) + i * 16 + g * 4;
            *reinterpret_cast<u32x2*>(tile + ch * LROW + px) = u32x2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
        }
    }
    __syncthreads();
    uint16_t* dx = static_cast<uint16_t*>(p.dx);
    for (int idx = tid; idx < 64 * (PT / 8); idx += 256) {
        const int ch = idx / (PT / 8), pc = idx % (PT / 8);
        if (c0 + ch >= p.cin) continue;
        const u32x4 v = *reinterpret_cast<const u32x4*>(tile + ch * LROW + pc * 8);
        uint16_t* plane = dx + ((int64_t)img * p.cin + c0 + ch) * p.H * p.W;
        const int o = t0 + pc * 8, oh = o / p.Wo, ow = o - oh * p.Wo;
        if constexpr (S == 1) {
            *reinterpret_cast<u32x4*>(plane + (int64_t)oh * p.W + ow) = v;
        } else {
            // values at even columns, zeros at odd ones; the row below is all zeros
            uint16_t* row = plane + (int64_t)(2 * oh) * p.W + 2 * ow;
            *reinterpret_cast<u32x4*>(row) = u32x4{v.x & 0xffffu, v.x >> 16, v.y & 0xffffu, v.y >> 16};
            *reinterpret_cast<u32x4*>(row + 8) = u32x4{v.z & 0xffffu, v.z >> 16, v.w & 0xffffu, v.w >> 16};
            *reinterpret_cast<u32x4*>(row + p.W) = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(row + p.W + 8) = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

}  // namespace

// mode: 0 forward, 1 grad input, 2 grad weight
bool conv_ring_applies(const tvk_conv_desc& d, int mode) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return false;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1) return false;
    // the gathered channels make the k stages (whole 32-channel stages; grad
    // weight gathers 8-channel chunks of the (tap, channel) rows); the other
    // channel count is a GEMM column count and may be anything
    if (mode == 0 && d.c_in % 32 != 0) return false;
    if (mode == 1 && d.c_out % 32 != 0) return false;
    if (mode == 2 && d.c_in % 8 != 0) return false;
    if (d.kh * d.kw > V_MAXTAPS) return false;
    if (d.n <= 0) return false;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.weight) || !al16(d.y)) return false;
    if (mode == 1 && (d.stride[0] > 4 || d.stride[1] > 4)) return false;
    if (mode == 2 && (d.h_out * d.w_out) % 32 != 0) return false;
    // 32-bit element offsets inside the kernels
    const int64_t big = std::max({d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out, d.c_out * d.c_in * d.kh * d.kw});
    return big < (int64_t(1) << 30);
}

tvk_status conv_ring_run(const tvk_conv_desc& d, int mode, const char* who) {
    const int n = (int)d.n, cin = (int)d.c_in, cout = (int)d.c_out, H = (int)d.h, W = (int)d.w;
    const int Ho = (int)d.h_out, Wo = (int)d.w_out, kh = (int)d.kh, kw = (int)d.kw, T = kh * kw;
    const int sh = (int)d.stride[0], sw = (int)d.stride[1], ph = (int)d.padding[0], pw = (int)d.padding[1];
    const int dh = (int)d.dilation[0], dw = (int)d.dilation[1];
    const size_t es = 2;
    hipStream_t s = resolve_stream(d.stream);
    Scratch scratch;

    ConvRing p;
    memset(&p, 0, sizeof(p));
    auto align = [](size_t v) { return (v + 255) / 256 * 256; };
    const bool f16 = d.dtype == TVK_F16;
    if (mode == 0 || mode == 1) {
        // gathered activation: x (forward) or dy (grad input), to bordered NHWC
        const int Cs = mode == 0 ? cin : cout, H0 = mode == 0 ? H : Ho, W0 = mode == 0 ? W : Wo;
        const int Cn = mode == 0 ? cout : cin;   // GEMM columns
        Border bd;
        if (mode == 0) {
            border_for(-ph, sh, Ho, 0, (kh - 1) * dh, H, bd.pt, bd.pb);
            border_for(-pw, sw, Wo, 0, (kw - 1) * dw, W, bd.pl, bd.pr);
        } else {
            // each sub-pixel phase reads dy rows i + nh / sh over its taps (see below)
            for (int r = 0; r < sh; ++r) {
                const int Hp = (H - r + sh - 1) / sh;
                int lo = INT32_MAX, hi = INT32_MIN;
                for (int a = 0; a < kh; ++a) {
                    const int nh = r + ph - a * dh;
                    if (((nh % sh) + sh) % sh != 0) continue;
                    lo = std::min(lo, nh / sh);
                    hi = std::max(hi, nh / sh);
                }
                if (Hp > 0 && lo <= hi) border_for(0, 1, Hp, lo, hi, Ho, bd.pt, bd.pb);
            }
            for (int r = 0; r < sw; ++r) {
                const int Wp = (W - r + sw - 1) / sw;
                int lo = INT32_MAX, hi = INT32_MIN;
                for (int b = 0; b < kw; ++b) {
                    const int nw = r + pw - b * dw;
                    if (((nw % sw) + sw) % sw != 0) continue;
                    lo = std::min(lo, nw / sw);
                    hi = std::max(hi, nw / sw);
                }
                if (Wp > 0 && lo <= hi) border_for(0, 1, Wp, lo, hi, Wo, bd.pl, bd.pr);
            }
        }
        const int Hs = H0 + bd.pt + bd.pb, Ws = W0 + bd.pl + bd.pr;
        const size_t act_b = align((size_t)n * Cs * Hs * Ws * es), wt_b = align((size_t)Cn * T * Cs * es);
        if ((size_t)n * Cs * Hs * Ws * es >= ((size_t)1 << 31))
            return fail(TVK_ERR_UNSUPPORTED, std::string(who) + ": the bordered channels-last copy exceeds 2 GiB");
        char* ws = static_cast<char*>(scratch.get(act_b + wt_b, s));
        if (!ws) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the channels-last copies");
        const void* src = mode == 0 ? d.x : d.y;
        WeightPermute wp;
        wp.w = static_cast<const uint16_t*>(d.weight);
        wp.out = reinterpret_cast<uint16_t*>(ws + act_b);
        wp.cout = cout; wp.cin = cin; wp.taps = T; wp.forward = mode == 0;
        launch_nhwc(src, ws, n, Cs, H0, W0, bd, s, wp);
        p.act = ws;
        p.wt = ws + act_b;
        p.Hs = Hs; p.Ws = Ws; p.Cs = Cs;
        p.N = Cn;
        p.act_bytes = (int)((size_t)n * Cs * Hs * Ws * es);
        p.wt_bytes = (int)((size_t)Cn * T * Cs * es);
        auto set_offsets = [&](ConvRing& q) {
            for (int t = 0; t < q.ntap; ++t) {
                q.tap_off[t] = (q.tap_h[t] * Ws + q.tap_w[t]) * Cs * 2;
                q.wt_off[t] = q.tap_k[t] * Cs * 2;
            }
        };
        p.wt_taps = T;
        p.out = mode == 0 ? d.y : d.x;
        p.Ho = mode == 0 ? Ho : H;
        p.Wo = mode == 0 ? Wo : W;
        if (mode == 0) {
            p.ntap = T;
            for (int t = 0; t < T; ++t) { p.tap_h[t] = (t / kw) * dh; p.tap_w[t] = (t % kw) * dw; p.tap_k[t] = t; }
            p.Hp = Ho; p.Wp = Wo;
            p.pix_sh = sh; p.pix_sw = sw; p.pix_bh = -ph + bd.pt; p.pix_bw = -pw + bd.pl;
            set_offsets(p);
            p.osh = 1; p.osw = 1; p.orh = 0; p.orw = 0;
            p.bias = d.bias;
            p.has_bias = d.bias ? 1 : 0;
            p.M = n * Ho * Wo;
            p.K = T * Cs;
            ConvRingSet set;
            set.ph[0] = p;
            if (f16) launch_ring<TVK_F16, 0>(set, 1, 1, s);
            else launch_ring<TVK_BF16, 0>(set, 1, 1, s);
        } else {
            // sub-pixel phases: input pixels (sh*i + ry, sw*j + rx) only meet taps
            // with (ry + ph - kh*dh) % sh == 0 (and likewise along w); up to 4
            // phases share a launch
            ConvRingSet set;
            int nph = 0;
            auto flush = [&]() {
                if (nph == 0) return;
                if (f16) launch_ring<TVK_F16, 0>(set, nph, 1, s);
                else launch_ring<TVK_BF16, 0>(set, nph, 1, s);
                nph = 0;
            };
            for (int ry = 0; ry < sh; ++ry)
                for (int rx = 0; rx < sw; ++rx) {
                    const int Hp = (H - ry + sh - 1) / sh, Wp = (W - rx + sw - 1) / sw;
                    if (Hp <= 0 || Wp <= 0) continue;
                    ConvRing q = p;
                    q.ntap = 0;
                    for (int a = 0; a < kh; ++a) {
                        const int nh = ry + ph - a * dh;
                        if (((nh % sh) + sh) % sh != 0) continue;
                        for (int b = 0; b < kw; ++b) {
                            const int nw = rx + pw - b * dw;
                            if (((nw % sw) + sw) % sw != 0) continue;
                            q.tap_h[q.ntap] = nh / sh;
                            q.tap_w[q.ntap] = nw / sw;
                            q.tap_k[q.ntap] = a * kw + b;
                            ++q.ntap;
                        }
                    }
                    q.Hp = Hp; q.Wp = Wp;
                    q.pix_sh = 1; q.pix_sw = 1; q.pix_bh = bd.pt; q.pix_bw = bd.pl;
                    set_offsets(q);
                    q.osh = sh; q.osw = sw; q.orh = ry; q.orw = rx;
                    q.M = n * Hp * Wp;
                    q.K = q.ntap * cout;
                    // (a phase no tap reaches has K = 0: the kernel writes its zeros)
                    set.ph[nph++] = q;
                    if (nph == V_MAXPH) flush();
                }
            flush();
        }
    } else {
        // grad weight: x to bordered NHWC; dy read NCHW; K = output pixels split into partials
        Border bd;
        border_for(-ph, sh, Ho, 0, (kh - 1) * dh, H, bd.pt, bd.pb);
        border_for(-pw, sw, Wo, 0, (kw - 1) * dw, W, bd.pl, bd.pr);
        const int Hs = H + bd.pt + bd.pb, Ws = W + bd.pl + bd.pr;
        if ((size_t)n * cin * Hs * Ws * es >= ((size_t)1 << 31))
            return fail(TVK_ERR_UNSUPPORTED, std::string(who) + ": the bordered channels-last copy exceeds 2 GiB");
        const size_t act_b = align((size_t)n * cin * Hs * Ws * es);
        p.M = T * cin;
        p.N = cout;
        p.K = n * Ho * Wo;
        const int bn = cout <= 64 ? 64 : cout <= 128 ? 128 : 256;
        const int64_t tiles = (int64_t)((p.M + 255) / 256) * ((p.N + bn - 1) / bn);
        // split K: more splits fill the device (about 256 workgroups) but each
        // adds M*N float32 partials written and read back. Minimise
        //   split*M*N*8 B / (5 TB/s) + 2*M*N*K / (1 PFLOP/s * min(1, tiles*split/256))
        const double part_us = (double)p.M * p.N * 8 / 5e6;
        const double full_us = 2.0 * p.M * p.N * p.K / 1e9;
        int64_t split = (int64_t)std::sqrt(full_us * 256.0 / (double)tiles / std::max(part_us, 1e-6));
        split = std::min<int64_t>(split, std::max<int64_t>(1, 256 / tiles));
        split = std::max<int64_t>(1, std::min<int64_t>(split, p.K / (8 * V_BK)));
        int64_t chunk = ((p.K + split - 1) / split + V_BK - 1) / V_BK * V_BK;
        split = (p.K + chunk - 1) / chunk;
        const size_t part_b = split > 1 ? (size_t)split * p.M * p.N * 4 : 0;
        char* ws = static_cast<char*>(scratch.get(act_b + part_b, s));
        if (!ws) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the channels-last copy");
        launch_nhwc(d.x, ws, n, cin, H, W, bd, s);
        p.act = ws;
        p.dyc = d.y;
        p.part = split > 1 ? reinterpret_cast<float*>(ws + act_b) : nullptr;
        p.out = d.weight;
        p.Hs = Hs; p.Ws = Ws; p.Cs = cin;
        p.ntap = T;
        p.wt_taps = T;
        for (int t = 0; t < T; ++t) { p.tap_h[t] = (t / kw) * dh - ph + bd.pt; p.tap_w[t] = (t % kw) * dw - pw + bd.pl; p.tap_k[t] = t; }
        p.pix_sh = sh; p.pix_sw = sw;
        p.HWo = Ho * Wo; p.Wd = Wo; p.kh_kw = T;
        p.wdiv = make_div((uint32_t)Wo);
        p.k_chunk = (int)chunk; p.split = (int)split;
        p.act_bytes = (int)((size_t)n * cin * Hs * Ws * es);
        p.dyc_bytes = (int)((size_t)n * cout * Ho * Wo * es);
        ConvRingSet set;
        set.ph[0] = p;
        if (f16) launch_ring<TVK_F16, 1>(set, 1, (int)split, s);
        else launch_ring<TVK_BF16, 1>(set, 1, (int)split, s);
        if (split > 1) {
            // group count: enough workgroups to fill the device, at most the splits
            const int total = p.M * p.N;
            int sg = 1;
            while (sg < 16 && sg * 2 <= split && (int64_t)total * sg / 1024 < 1024) sg *= 2;
            const dim3 grid((unsigned)((total + 1024 / sg - 1) / (1024 / sg)));
            if (f16) hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_F16>, grid, dim3(256), 0, s, p.part, d.weight, p.M, p.N, cin, T, (int)split, sg);
            else hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_BF16>, grid, dim3(256), 0, s, p.part, d.weight, p.M, p.N, cin, T, (int)split, sg);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}


// stride 1, 3x3, padding 1, dilation 1. Forward / grad input: the gathered
// side in whole 32-channel chunks, widths 8, 16, 32 or 64. Grad weight: input
// channels in 64-channel blocks, widths 16 or 32 with whole 256-pixel tiles.
bool conv1x1_wgrad_applies(const tvk_conv_desc& d);
tvk_status conv1x1_wgrad_run(const tvk_conv_desc& d, const char* who);

// 1x1 forward from NCHW: stride 1 or 2, no padding, input channels in 32s, the
// pixel tile (256 or 64 output pixels, whole 8-pixel row groups) and all its
// input channels within 64 KB of LDS
int conv1x1_fwd_tile(const tvk_conv_desc& d) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return 0;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return 0;
    if (d.kh != 1 || d.kw != 1 || d.padding[0] != 0 || d.padding[1] != 0) return 0;
    if (d.stride[0] != d.stride[1] || (d.stride[0] != 1 && d.stride[0] != 2)) return 0;
    if (d.c_in % 32 != 0 || d.w_out % 8 != 0 || d.w % 8 != 0) return 0;
    if (d.stride[1] == 2 && 2 * d.w_out > d.w) return 0;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y) || !al16(d.weight)) return 0;
    if (std::max(d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out) >= (int64_t(1) << 30)) return 0;
    const int64_t hwo = d.h_out * d.w_out;
    const int pt = hwo % 256 == 0 ? 256 : hwo % 64 == 0 ? 64 : 0;
    if (pt == 0 || d.c_in * pt > 32768) return 0;
    return pt;
}

// 1x1 grad input from NCHW: stride 1 or 2 with dx exactly covered (W = s*Wo,
// H = s*Ho), output channels in 32s, dy tile and the weight rows in LDS
int conv1x1_dgrad_tile(const tvk_conv_desc& d) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return 0;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return 0;
    if (d.kh != 1 || d.kw != 1 || d.padding[0] != 0 || d.padding[1] != 0) return 0;
    if (d.stride[0] != d.stride[1] || (d.stride[0] != 1 && d.stride[0] != 2)) return 0;
    if (d.w != d.stride[1] * d.w_out || d.h != d.stride[0] * d.h_out) return 0;
    if (d.c_out % 32 != 0 || d.c_in % 8 != 0 || d.w_out % 8 != 0) return 0;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y) || !al16(d.weight)) return 0;
    if (std::max(d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out) >= (int64_t(1) << 30)) return 0;
    const int64_t hwo = d.h_out * d.w_out;
    // 256-pixel tiles only where they still give a workgroup per CU
    int pt = hwo % 64 == 0 ? 64 : 0;
    if (hwo % 256 == 0 && d.n * (hwo / 256) * ((d.c_in + 63) / 64) >= 256) pt = 256;
    if (pt == 0 || d.c_out * pt * 2 > (pt == 256 ? 65536 : 32768) || d.c_out * 128 > 32768) return 0;
    return pt;
}

tvk_status conv1x1_dgrad_run(const tvk_conv_desc& d, const char* who) {
    const int pt = conv1x1_dgrad_tile(d);
    hipStream_t s = resolve_stream(d.stream);
    PointDgArgs p;
    memset(&p, 0, sizeof(p));
    p.dy = static_cast<const uint16_t*>(d.y);
    p.w = static_cast<const uint16_t*>(d.weight);
    p.dx = d.x;
    p.cin = (int)d.c_in; p.cout = (int)d.c_out; p.H = (int)d.h; p.W = (int)d.w;
    p.Ho = (int)d.h_out; p.Wo = (int)d.w_out;
    p.tiles_per_img = (int)(d.h_out * d.w_out / pt);
    const dim3 grid((unsigned)(d.n * p.tiles_per_img), (unsigned)((p.cin + 63) / 64));
    const bool f16 = d.dtype == TVK_F16, s2 = d.stride[0] == 2;
#define TVK_PD(DT_, S_, PT_) hipLaunchKernelGGL((conv1x1_dgrad_kernel<DT_, S_, PT_>), grid, dim3(256), 0, s, p)
    if (pt == 256) {
        if (f16) { if (s2) TVK_PD(TVK_F16, 2, 256); else TVK_PD(TVK_F16, 1, 256); }
        else { if (s2) TVK_PD(TVK_BF16, 2, 256); else TVK_PD(TVK_BF16, 1, 256); }
    } else {
        if (f16) { if (s2) TVK_PD(TVK_F16, 2, 64); else TVK_PD(TVK_F16, 1, 64); }
        else { if (s2) TVK_PD(TVK_BF16, 2, 64); else TVK_PD(TVK_BF16, 1, 64); }
    }
#undef TVK_PD
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status conv1x1_fwd_run(const tvk_conv_desc& d, const char* who) {
    const int pt = conv1x1_fwd_tile(d);
    hipStream_t s = resolve_stream(d.stream);
    PointFwdArgs p;
    memset(&p, 0, sizeof(p));
    p.x = static_cast<const uint16_t*>(d.x);
    p.w = static_cast<const uint16_t*>(d.weight);
    p.bias = d.bias;
    p.has_bias = d.bias ? 1 : 0;
    p.y = d.y;
    p.cin = (int)d.c_in; p.cout = (int)d.c_out; p.H = (int)d.h; p.W = (int)d.w;
    p.Ho = (int)d.h_out; p.Wo = (int)d.w_out;
    p.tiles_per_img = (int)(d.h_out * d.w_out / pt);
    const dim3 grid((unsigned)(d.n * p.tiles_per_img), (unsigned)((p.cout + 63) / 64));
    const bool f16 = d.dtype == TVK_F16, s2 = d.stride[0] == 2;
#define TVK_PF(DT_, S_, PT_) hipLaunchKernelGGL((conv1x1_fwd_kernel<DT_, S_, PT_>), grid, dim3(256), 0, s, p)
    if (pt == 256) {
        if (f16) { if (s2) TVK_PF(TVK_F16, 2, 256); else TVK_PF(TVK_F16, 1, 256); }
        else { if (s2) TVK_PF(TVK_BF16, 2, 256); else TVK_PF(TVK_BF16, 1, 256); }
    } else {
        if (f16) { if (s2) TVK_PF(TVK_F16, 2, 64); else TVK_PF(TVK_F16, 1, 64); }
        else { if (s2) TVK_PF(TVK_BF16, 2, 64); else TVK_PF(TVK_BF16, 1, 64); }
    }
#undef TVK_PF
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

// stride-2 3x3 padding-1 forward: W = 2 Wo in 16..64, H = 2 Ho, input channels in 32s
int conv_halo_s2_fm(const tvk_conv_desc& d, int* ipt = nullptr) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return 0;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return 0;
    if (d.kh != 3 || d.kw != 3 || d.stride[0] != 2 || d.stride[1] != 2 || d.dilation[0] != 1 || d.dilation[1] != 1) return 0;
    if (d.padding[0] != 1 || d.padding[1] != 1 || d.c_in % 32 != 0) return 0;
    if ((d.w != 16 && d.w != 32 && d.w != 64) || d.w != 2 * d.w_out || d.h != 2 * d.h_out) return 0;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y) || !al16(d.weight)) return 0;
    if (std::max({d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out, d.c_out * d.c_in * 9}) >= (int64_t(1) << 30)) return 0;
    // 128-pixel tiles: rows of one image, or whole images where an image has
    // fewer pixels (64-pixel tiles of one small image measured no faster than
    // the ring kernel and its channels-last copy: their weight rows serve too
    // few pixels)
    const int64_t hw = d.h_out * d.w_out;
    if (hw >= 128) {
        if (ipt) *ipt = 1;
        return 2;
    }
    if (128 % hw != 0) return 0;
    const int64_t k = 128 / hw;
    if (k * (2 * d.h_out + 1) * (d.w + 2) * 64 > H2_A || k * (2 * d.h_out + 1) * (d.w / 8) * 4 > 512) return 0;
    if (ipt) *ipt = (int)k;
    return 2;
}

// Stride-2 3x3 grad input by phases: TP dy positions a tile (128, or 64 where
// 128-position tiles would leave the device short of workgroups) x BN input
// channels (64, or 32 where that keeps 128-position tiles); tr rows of one
// image, or ipt whole images where an image has fewer than TP positions.
// 0 when the kernel does not apply.
int conv_halo_dgrad_s2_tp(const tvk_conv_desc& d, int* tr = nullptr, int* ipt = nullptr, int* bn_out = nullptr) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return 0;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return 0;
    if (d.kh != 3 || d.kw != 3 || d.stride[0] != 2 || d.stride[1] != 2 || d.dilation[0] != 1 || d.dilation[1] != 1) return 0;
    if (d.padding[0] != 1 || d.padding[1] != 1 || d.c_out % 32 != 0) return 0;
    const int64_t Ho = d.h_out, Wo = d.w_out;
    if ((Wo != 8 && Wo != 16 && Wo != 32 && Wo != 64) || d.w != 2 * Wo || d.h != 2 * Ho) return 0;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y) || !al16(d.weight)) return 0;
    if (std::max({d.n * d.c_in * d.h * d.w, d.n * d.c_out * Ho * Wo, d.c_out * d.c_in * 9}) >= (int64_t(1) << 30)) return 0;
    // (TP, BN) in order: (128, 64), (128, 32), (64, 64); the first two only
    // where they give at least 256 workgroups
    for (int c = 0; c < 3; ++c) {
        const int tp = c < 2 ? 128 : 64, bn = c == 1 ? 32 : 64;
        const int64_t r = std::min<int64_t>(Ho, tp / Wo);
        if (r < 1 || tp % (r * Wo) != 0) continue;
        const int64_t k = tp / (r * Wo);
        if (k == 1 ? Ho % r != 0 : r != Ho) continue;
        if (k * (r + 1) * (Wo + 1) * 64 > D2_A) continue;   // the halo fits its LDS stage
        const int64_t tiles = (d.n + k - 1) / k * (Ho / r) * ((d.c_in + bn - 1) / bn);
        if (tp == 128 && tiles < 256) continue;
        if (tr) *tr = (int)r;
        if (ipt) *ipt = (int)k;
        if (bn_out) *bn_out = bn;
        return tp;
    }
    return 0;
}

int conv_halo_wgrad_s2_tpx(const tvk_conv_desc& d);
tvk_status conv_halo_wgrad_s2_run(const tvk_conv_desc& d, const char* who);

bool conv_halo_applies(const tvk_conv_desc& d, int mode) {
    if (mode == 0 && conv_halo_s2_fm(d) != 0) return true;
    if (mode == 1 && conv_halo_dgrad_s2_tp(d) != 0) return true;
    if (mode == 2 && conv_halo_wgrad_s2_tpx(d) != 0) return true;
    if (mode == 2 && conv1x1_wgrad_applies(d)) return true;
    if (mode == 0 && conv1x1_fwd_tile(d) != 0) return true;
    if (mode == 1 && conv1x1_dgrad_tile(d) != 0) return true;
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return false;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return false;
    if (d.kh != 3 || d.kw != 3 || d.stride[0] != 1 || d.stride[1] != 1 || d.dilation[0] != 1 || d.dilation[1] != 1) return false;
    if (d.padding[0] != 1 || d.padding[1] != 1) return false;
    if (d.w != 8 && d.w != 16 && d.w != 32 && d.w != 64) return false;
    if (mode == 2) {
        if ((d.w != 16 && d.w != 32) || d.c_in % 64 != 0 || d.h % (256 / d.w) != 0) return false;
    } else if ((mode == 0 ? d.c_in : d.c_out) % 32 != 0) {
        return false;
    }
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y) || !al16(d.weight)) return false;
    const int64_t big = std::max({d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h * d.w, d.c_out * d.c_in * 9});
    return big < (int64_t(1) << 30);
}

// 1x1 grad weight from NCHW: stride 1 or 2 on both axes, no padding, input
// channels in 64-channel blocks, output rows in 8-pixel groups of 32-pixel steps
bool conv1x1_wgrad_applies(const tvk_conv_desc& d) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return false;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return false;
    if (d.kh != 1 || d.kw != 1 || d.padding[0] != 0 || d.padding[1] != 0) return false;
    if (d.stride[0] != d.stride[1] || (d.stride[0] != 1 && d.stride[0] != 2)) return false;
    if (d.c_in % 64 != 0 || d.w_out % 8 != 0 || (d.h_out * d.w_out) % 32 != 0) return false;
    // 16-byte loads: rows and planes of x and dy start 16-byte aligned
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y) || d.w % 8 != 0) return false;
    // the stride-2 pair of loads reads 16 input pixels from column 2 * ow: inside the row
    if (d.stride[1] == 2 && 2 * d.w_out > d.w) return false;
    return std::max(d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out) < (int64_t(1) << 30);
}

tvk_status conv1x1_wgrad_run(const tvk_conv_desc& d, const char* who) {
    hipStream_t s = resolve_stream(d.stream);
    Scratch scratch;
    PointWgArgs p;
    memset(&p, 0, sizeof(p));
    p.x = static_cast<const uint16_t*>(d.x);
    p.dy = static_cast<const uint16_t*>(d.y);
    p.cin = (int)d.c_in; p.cout = (int)d.c_out; p.H = (int)d.h; p.W = (int)d.w;
    p.Ho = (int)d.h_out; p.Wo = (int)d.w_out; p.stride = (int)d.stride[0];
    p.steps = (int)(d.n * p.Ho * p.Wo / 32);
    const int cb = p.cin / 64, nb = (p.cout + 63) / 64;
    // about 256 workgroups, at least 8 steps (two a wave) each
    p.split = std::max(1, std::min(p.steps / 8, 256 / (cb * nb)));
    p.steps_per_split = (p.steps + p.split - 1) / p.split;
    p.split = (p.steps + p.steps_per_split - 1) / p.steps_per_split;
    const size_t part_b = (size_t)p.split * p.cin * p.cout * sizeof(float);
    p.part = static_cast<float*>(scratch.get(part_b, s));
    if (!p.part) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the grad-weight partials");
    const dim3 grid((unsigned)p.split, (unsigned)cb, (unsigned)nb);
    const bool f16 = d.dtype == TVK_F16;
    if (p.stride == 1) {
        if (f16) hipLaunchKernelGGL((conv1x1_wgrad_kernel<TVK_F16, 1>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((conv1x1_wgrad_kernel<TVK_BF16, 1>), grid, dim3(256), 0, s, p);
    } else {
        if (f16) hipLaunchKernelGGL((conv1x1_wgrad_kernel<TVK_F16, 2>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((conv1x1_wgrad_kernel<TVK_BF16, 2>), grid, dim3(256), 0, s, p);
    }
    const int total = p.cin * p.cout;
    int sg = 1;
    while (sg < 16 && sg * 2 <= p.split && (int64_t)total * sg / 1024 < 1024) sg *= 2;
    const dim3 rgrid((unsigned)((total + 1024 / sg - 1) / (1024 / sg)));
    if (f16) hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_F16>, rgrid, dim3(256), 0, s, p.part, d.weight, p.cin, p.cout, p.cin, 1, p.split, sg);
    else hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_BF16>, rgrid, dim3(256), 0, s, p.part, d.weight, p.cin, p.cout, p.cin, 1, p.split, sg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

// stride-2 grad weight: W = 2 Wo with Wo in 8..32, H = 2 Ho, output tiles of
// 128 pixels (64 when Wo = 8), whole tiles per image, input channels in 32s
int conv_halo_wgrad_s2_tpx(const tvk_conv_desc& d) {
    if (d.dtype != TVK_F16 && d.dtype != TVK_BF16) return 0;
    if ((d.flags & TVK_GEMM_EXACT) || d.groups != 1 || d.n <= 0) return 0;
    if (d.kh != 3 || d.kw != 3 || d.stride[0] != 2 || d.stride[1] != 2 || d.dilation[0] != 1 || d.dilation[1] != 1) return 0;
    if (d.padding[0] != 1 || d.padding[1] != 1 || d.c_in % 32 != 0) return 0;
    if ((d.w_out != 8 && d.w_out != 16 && d.w_out != 32) || d.w != 2 * d.w_out || d.h != 2 * d.h_out) return 0;
    const int tpx = d.w_out == 8 ? 64 : 128;
    if ((d.h_out * d.w_out) % tpx != 0) return 0;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(d.x) || !al16(d.y)) return 0;
    if (std::max(d.n * d.c_in * d.h * d.w, d.n * d.c_out * d.h_out * d.w_out) >= (int64_t(1) << 30)) return 0;
    return tpx;
}

tvk_status conv_halo_wgrad_s2_run(const tvk_conv_desc& d, const char* who) {
    const int cin = (int)d.c_in, cout = (int)d.c_out, Wo = (int)d.w_out;
    const int tpx = conv_halo_wgrad_s2_tpx(d);
    hipStream_t s = resolve_stream(d.stream);
    Scratch scratch;
    HaloWgArgs p;
    memset(&p, 0, sizeof(p));
    p.x = static_cast<const uint16_t*>(d.x);
    p.dy = d.y;
    p.cin = cin; p.cout = cout; p.H = (int)d.h;
    p.tiles_per_img = (int)(d.h_out * d.w_out / tpx);
    p.ntiles = (int)d.n * p.tiles_per_img;
    p.dy_bytes = (int)(d.n * cout * d.h_out * d.w_out * 2);
    const int cb = cin / 32, nb = (cout + 63) / 64;
    // about 256 workgroups, each summing at least 2 tiles
    p.split = std::max(1, std::min(p.ntiles / 2, 256 / (cb * nb)));
    const size_t part_b = (size_t)p.split * 9 * cin * cout * sizeof(float);
    char* ws = static_cast<char*>(scratch.get(part_b, s));
    if (!ws) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the grad-weight partials");
    p.part = reinterpret_cast<float*>(ws);
    const dim3 grid((unsigned)p.split, (unsigned)cb, (unsigned)nb);
    const bool f16 = d.dtype == TVK_F16;
#define TVK_HW2(WO_, TPX_)                                                                                           \
    do {                                                                                                             \
        if (f16) hipLaunchKernelGGL((conv_halo_wgrad_s2_kernel<TVK_F16, WO_, TPX_>), grid, dim3(512), 0, s, p);     \
        else hipLaunchKernelGGL((conv_halo_wgrad_s2_kernel<TVK_BF16, WO_, TPX_>), grid, dim3(512), 0, s, p);        \
    } while (0)
    if (Wo == 8) TVK_HW2(8, 64);
    else if (Wo == 16) TVK_HW2(16, 128);
    else TVK_HW2(32, 128);
#undef TVK_HW2
    const int M = 9 * cin, total = M * cout;
    int sg = 1;
    while (sg < 16 && sg * 2 <= p.split && (int64_t)total * sg / 1024 < 1024) sg *= 2;
    const dim3 rgrid((unsigned)((total + 1024 / sg - 1) / (1024 / sg)));
    if (f16) hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_F16>, rgrid, dim3(256), 0, s, p.part, d.weight, M, cout, cin, 9, p.split, sg);
    else hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_BF16>, rgrid, dim3(256), 0, s, p.part, d.weight, M, cout, cin, 9, p.split, sg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status conv_halo_wgrad_run(const tvk_conv_desc& d, const char* who) {
    const int cin = (int)d.c_in, cout = (int)d.c_out, H = (int)d.h, W = (int)d.w;
    hipStream_t s = resolve_stream(d.stream);
    Scratch scratch;
    HaloWgArgs p;
    memset(&p, 0, sizeof(p));
    p.x = static_cast<const uint16_t*>(d.x);
    p.dy = d.y;
    p.cin = cin; p.cout = cout; p.H = H;
    p.tiles_per_img = H / (256 / W);
    p.ntiles = (int)d.n * p.tiles_per_img;
    p.dy_bytes = (int)(d.n * cout * H * W * 2);
    const int cb = cin / 64;
    // 32 output channels a workgroup where one 64 x 64 block covers the weight
    // (half the partials for the same grid); 64 otherwise
    const int bn = (cb * ((cout + 63) / 64) == 1 && cout > 32) ? 32 : 64;
    const int nb = (cout + bn - 1) / bn;
    // about 256 workgroups (one a CU), each summing at least 2 tiles
    p.split = std::max(1, std::min(p.ntiles / 2, 256 / (cb * nb)));
    const size_t part_b = (size_t)p.split * 9 * cin * cout * sizeof(float);
    char* ws = static_cast<char*>(scratch.get(part_b, s));
    if (!ws) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the grad-weight partials");
    p.part = reinterpret_cast<float*>(ws);
    const dim3 grid((unsigned)p.split, (unsigned)cb, (unsigned)nb);
    const bool f16 = d.dtype == TVK_F16;
#define TVK_HW1(W_, BN_)                                                                                          \
    do {                                                                                                          \
        if (f16) hipLaunchKernelGGL((conv_halo_wgrad_kernel<TVK_F16, W_, BN_>), grid, dim3(512), 0, s, p);       \
        else hipLaunchKernelGGL((conv_halo_wgrad_kernel<TVK_BF16, W_, BN_>), grid, dim3(512), 0, s, p);          \
    } while (0)
    if (W == 32 && bn == 32) TVK_HW1(32, 32);
    else if (W == 32) TVK_HW1(32, 64);
    else if (bn == 32) TVK_HW1(16, 32);
    else TVK_HW1(16, 64);
#undef TVK_HW1
    // partials [split][(tap, channel)][output channel] -> dW[co][c][tap]
    const int M = 9 * cin, total = M * cout;
    int sg = 1;
    while (sg < 16 && sg * 2 <= p.split && (int64_t)total * sg / 1024 < 1024) sg *= 2;
    const dim3 rgrid((unsigned)((total + 1024 / sg - 1) / (1024 / sg)));
    if (f16) hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_F16>, rgrid, dim3(256), 0, s, p.part, d.weight, M, cout, cin, 9, p.split, sg);
    else hipLaunchKernelGGL(wgrad_ring_reduce_kernel<TVK_BF16>, rgrid, dim3(256), 0, s, p.part, d.weight, M, cout, cin, 9, p.split, sg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

// Stride-1 halo tile: 256 pixels (two workgroups a CU) where 512-pixel tiles
// would give the 256 CUs fewer than two workgroups each. N: the output's
// channels (forward c_out, grad input c_in).
int halo_s1_px(const tvk_conv_desc& d, int N) {
    const int H = (int)d.h, W = (int)d.w;
    const int64_t wg512 = d.n * ((H + HL_PX / W - 1) / (HL_PX / W)) * ((N + HL_BN - 1) / HL_BN);
    return wg512 < 512 ? 256 : HL_PX;
}

tvk_status conv_halo_run(const tvk_conv_desc& d, int mode, const char* who) {
    if (mode == 2) {
        if (conv1x1_wgrad_applies(d)) return conv1x1_wgrad_run(d, who);
        if (conv_halo_wgrad_s2_tpx(d) != 0) return conv_halo_wgrad_s2_run(d, who);
        return conv_halo_wgrad_run(d, who);
    }
    if (mode == 0 && conv1x1_fwd_tile(d) != 0) return conv1x1_fwd_run(d, who);
    if (mode == 1 && conv1x1_dgrad_tile(d) != 0) return conv1x1_dgrad_run(d, who);
    const int cin = (int)d.c_in, cout = (int)d.c_out, H = (int)d.h, W = (int)d.w;
    const int Cs = mode == 0 ? cin : cout, N = mode == 0 ? cout : cin;
    hipStream_t s = resolve_stream(d.stream);
    Scratch scratch;
    const size_t wt_b = (size_t)N * 9 * Cs * 2;
    const uint16_t* w16 = static_cast<const uint16_t*>(d.weight);
    // the forward kernels on 256 threads (the stride-2 one, and the stride-1 one
    // on 256-pixel tiles) gather their weight rows from the weight as given
    // and so do the grad inputs (stride 2, and stride 1 on 256-pixel tiles)
    // into a k-major tile
    const bool tb = mode == 1 && N % 8 == 0 && (reinterpret_cast<uintptr_t>(w16) & 15) == 0 &&
                    (conv_halo_dgrad_s2_tp(d, nullptr, nullptr, nullptr) != 0 || halo_s1_px(d, N) == 256);
    const bool raw = tb || (mode == 0 && (reinterpret_cast<uintptr_t>(w16) & 15) == 0 &&
                            (conv_halo_s2_fm(d, nullptr) != 0 || halo_s1_px(d, N) == 256));
    char* ws = nullptr;
    if (!raw) {
        ws = static_cast<char*>(scratch.get(wt_b, s));
        if (!ws) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the permuted weight");
        const int pgroups = N * 9 * (Cs / 8);
        const dim3 pgrid((unsigned)std::min((pgroups + 255) / 256, 1024));
        if (mode == 0) hipLaunchKernelGGL(weight_permute9_kernel<true>, pgrid, dim3(256), 0, s, w16, reinterpret_cast<uint16_t*>(ws), cout, cin);
        else hipLaunchKernelGGL(weight_permute9_kernel<false>, pgrid, dim3(256), 0, s, w16, reinterpret_cast<uint16_t*>(ws), cout, cin);
    }
    HaloArgs p;
    memset(&p, 0, sizeof(p));
    p.wraw = raw ? w16 : nullptr;
    p.src = static_cast<const uint16_t*>(mode == 0 ? d.x : d.y);
    p.wt = ws;
    p.bias = mode == 0 ? d.bias : nullptr;
    p.has_bias = (mode == 0 && d.bias) ? 1 : 0;
    p.out = mode == 0 ? d.y : d.x;
    p.Cs = Cs; p.N = N; p.H = H; p.W = W;
    p.ipt = 1;
    p.nimg = (int)d.n;
    int tr2 = 0, ipt2 = 0, bn2 = 64;
    const int tp2 = mode == 1 ? conv_halo_dgrad_s2_tp(d, &tr2, &ipt2, &bn2) : 0;
    if (tp2) {
        p.tr = tr2;
        p.ipt = ipt2;
        p.nimg = (int)d.n;
        p.row_tiles = (H / 2) / tr2;
        p.wt_bytes = (int)wt_b;
        const dim3 grid((unsigned)((d.n + ipt2 - 1) / ipt2 * p.row_tiles), (unsigned)((N + bn2 - 1) / bn2));
        const bool f16 = d.dtype == TVK_F16;
#define TVK_D2(TP_, BN_)                                                                                        \
    do {                                                                                                        \
        if (tb) {                                                                                               \
            if (f16) hipLaunchKernelGGL((conv_halo_dgrad_s2_kernel<TVK_F16, TP_, BN_, true>), grid, dim3(512), 0, s, p);   \
            else hipLaunchKernelGGL((conv_halo_dgrad_s2_kernel<TVK_BF16, TP_, BN_, true>), grid, dim3(512), 0, s, p);      \
        } else {                                                                                                \
            if (f16) hipLaunchKernelGGL((conv_halo_dgrad_s2_kernel<TVK_F16, TP_, BN_>), grid, dim3(512), 0, s, p);         \
            else hipLaunchKernelGGL((conv_halo_dgrad_s2_kernel<TVK_BF16, TP_, BN_>), grid, dim3(512), 0, s, p);            \
        }                                                                                                       \
    } while (0)
        if (tp2 == 128 && bn2 == 64) TVK_D2(128, 64);
        else if (tp2 == 128) TVK_D2(128, 32);
        else TVK_D2(64, 64);
#undef TVK_D2
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
        return TVK_OK;
    }
    int ipt_f = 1;
    const int fm2 = mode == 0 ? conv_halo_s2_fm(d, &ipt_f) : 0;
    p.ipt = ipt_f;
    const int px = fm2 ? HL_PX : halo_s1_px(d, N);
    p.tr = fm2 ? (ipt_f > 1 ? H / 2 : 64 * fm2 / (W / 2)) : px / W;
    p.row_tiles = fm2 ? ((H / 2) + p.tr - 1) / p.tr : (H + p.tr - 1) / p.tr;
    p.wt_bytes = (int)wt_b;
    // forward: tap (a, b) reads source (h + a - 1, w + b - 1); grad input: (h + 1 - a, w + 1 - b);
    // stride 2: halo row 2r + a, de-interleaved column slot (b == 1 ? W / 2 + 1 + c : c + b / 2)
    for (int t = 0; t < 9; ++t) {
        const int a = t / 3, b = t % 3;
        if (fm2) {
            p.dtap[t] = a * (W + 2) + (b == 1 ? W / 2 + 1 : b / 2);
        } else {
            const int ho = mode == 0 ? a - 1 : 1 - a, wo = mode == 0 ? b - 1 : 1 - b;
            p.dtap[t] = ho * (W + 2) + wo;
        }
    }
    const dim3 grid((unsigned)((d.n + p.ipt - 1) / p.ipt * p.row_tiles), (unsigned)((N + HL_BN - 1) / HL_BN));
    if (fm2) {
        // one LDS stage (two workgroups a CU) where the grid has more workgroups than CUs
        const bool one = (int64_t)grid.x * grid.y > 256;
        if (one) {
            if (d.dtype == TVK_F16) hipLaunchKernelGGL((conv_halo_s2_kernel<TVK_F16, 2, 1>), grid, dim3(256), 0, s, p);
            else hipLaunchKernelGGL((conv_halo_s2_kernel<TVK_BF16, 2, 1>), grid, dim3(256), 0, s, p);
        } else {
            if (d.dtype == TVK_F16) hipLaunchKernelGGL((conv_halo_s2_kernel<TVK_F16, 2, 2>), grid, dim3(256), 0, s, p);
            else hipLaunchKernelGGL((conv_halo_s2_kernel<TVK_BF16, 2, 2>), grid, dim3(256), 0, s, p);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
        return TVK_OK;
    }
    if (px == 256 && tb) {
        if (d.dtype == TVK_F16) hipLaunchKernelGGL((conv_halo_kernel<TVK_F16, 256, true>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((conv_halo_kernel<TVK_BF16, 256, true>), grid, dim3(256), 0, s, p);
    } else if (px == 256) {
        if (d.dtype == TVK_F16) hipLaunchKernelGGL((conv_halo_kernel<TVK_F16, 256>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((conv_halo_kernel<TVK_BF16, 256>), grid, dim3(256), 0, s, p);
    } else {
        if (d.dtype == TVK_F16) hipLaunchKernelGGL((conv_halo_kernel<TVK_F16, 512>), grid, dim3(512), 0, s, p);
        else hipLaunchKernelGGL((conv_halo_kernel<TVK_BF16, 512>), grid, dim3(512), 0, s, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

}  // namespace tvk
