// Dense GEMM kernels for gfx950 (MI355X) and the tvk_gemm dispatcher.
//
// Reference semantics followed (file:line under the reference tree):
//   - operand model: base + batch*s0 + row*s1 + col*s2, TensorStrides
//     (src/shaders/helpers/gemm.slang:3-9, src/api/ops/matmul.cpp:156-160)
//   - epilogue: v = acc*alpha; if has_bias: v += bias*beta; v = act(v); one
//     rounding to the storage type (src/shaders/helpers/gemm_simd.slang:67-99,
//     src/shaders/ops/matmul_coop.slang:383-408, src/shaders/core/dtype.slang:255-282)
//   - has_bias = bias defined && beta != 0 (src/api/ops/matmul.cpp:259,394)
//   - K == 0: act(beta*bias) or zeros (src/api/ops/matmul.cpp:284-288,402-406)
//
// Kernels:
//   gemm16_mfma  float16/bfloat16, 256x256 or 128x128 block tiles, 4 waves,
//                v_mfma_f32_32x32x16_{f16,bf16}, both operands staged through
//                LDS in a k-contiguous padded layout, double buffered. An operand
//                whose contiguous dimension is M or N (a transposed view) is
//                transposed in registers on its way into LDS, so no copy is made.
//   gemm_seq_mfma  float32 (and every dtype under TVK_GEMM_EXACT) in the
//                reference SIMD tile's summation order: every output
//                accumulates fmaf(a_k, b_k, acc) for k = 0..K-1 in sequence
//                (src/shaders/helpers/gemm_simd.slang:219-239), issued as
//                v_mfma_f32_32x32x1f32 rank-1 updates (one rounding each).
//   gemm_generic any strides / dtype, one thread per output, same order.
#include "gemm_common.h"

#include <mutex>
#include "tune_table.h"

#include <algorithm>
#include <cmath>
#include <vector>
#include <string>
#include <cstring>
#include <cstdio>
#include <cstdlib>

namespace tvk {
namespace {

// ----------------------------------------------------------------------------
// K == 0 and generic kernels
// ----------------------------------------------------------------------------

template <int DT>
__global__ void gemm_k0_kernel(GemmArgs p) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t total = (int64_t)p.batch * p.M * p.N;
    if (idx >= total) return;
    int col = (int)(idx % p.N);
    int row = (int)((idx / p.N) % p.M);
    int b = (int)(idx / ((int64_t)p.N * p.M));
    store_out<DT, true>(p, b, row, col, 0.0f);
}

// One output per thread, sequential k, fmaf accumulate: the reference SIMD
// tile's per-output order, for operands no tiled kernel accepts.
// Outputs of one batch matrix (blockIdx.y) are dealt out along x in a
// grid-stride loop, so any M x N fits the grid.
template <int DT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmArgs p) {
    typedef typename elem<DT>::T T;
    const int b = blockIdx.y;
    const int64_t total = (int64_t)p.M * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
        const int row = (int)(idx / p.N), col = (int)(idx % p.N);
        const T* a = reinterpret_cast<const T*>(p.a) + a_boff(p, b) + (int64_t)row * p.sa[1];
        const T* bm = reinterpret_cast<const T*>(p.b) + b_boff(p, b) + (int64_t)col * p.sb[2];
        float acc = 0.0f;
        for (int k = 0; k < p.K; ++k)
            acc = fmaf(elem<DT>::to_f32(a[(int64_t)k * p.sa[2]]), elem<DT>::to_f32(bm[(int64_t)k * p.sb[1]]), acc);
        store_out<DT, true>(p, b, row, col, acc);
    }
}

// ----------------------------------------------------------------------------
// float16 / bfloat16 MFMA kernel
// ----------------------------------------------------------------------------

constexpr int H_BK = 64;          // k per LDS stage
constexpr int H_LDK = H_BK + 8;   // padded LDS row (halfs): 144 B, conflict-free b128 reads

template <int DT>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Loader of one operand tile of R rows (rows = M for A, N for B) x 64 k into
// LDS laid out [R][H_LDK] with k contiguous.
//   KMAJ: the operand's k stride is 1: thread t loads 16 B chunks (8 k) of rows
//         t/8 + 32*i, chunk t%8.
//   else: the operand's row stride is 1 (M or N contiguous): thread t loads,
//         for k = 4*(t%16) + 0..3, eight consecutive rows starting at
//         8*(t/16 + 16*u), and transposes the 4x8 block into 8 rows of 4 k.
template <int R, bool KMAJ, bool VEC, int NT>
struct TileLoader {
    static constexpr int NREG = R * 8 / NT;   // 16-byte registers per thread per stage
    static_assert(KMAJ || NREG % 4 == 0, "transposing loader works on 4 k rows");
    u32x4 reg[NREG];

    __device__ inline void load(__amdgpu_buffer_rsrc_t rsrc, int64_t s_row, int64_t s_k, int row0, int rows, int k0, int K, int tid) {
        if constexpr (KMAJ) {
            const int kc = (tid % 8) * 8;
#pragma unroll
            for (int i = 0; i < NREG; ++i) {
                int r = tid / 8 + (NT / 8) * i;
                int gr = row0 + r, gk = k0 + kc;
                int valid = K - gk;
                reg[i] = load_chunk<VEC>(rsrc, gr < rows, (int64_t)gr * s_row + (int64_t)gk * s_k, s_k, valid);
            }
        } else {
            const int kq = (tid % 16) * 4;
#pragma unroll
            for (int u = 0; u < NREG / 4; ++u) {
                int rc = 8 * (tid / 16 + (NT / 16) * u);
                int gr = row0 + rc;
                int valid = rows - gr;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    int gk = k0 + kq + q;
                    reg[u * 4 + q] = load_chunk<VEC>(rsrc, gk < K, (int64_t)gk * s_k + (int64_t)gr * s_row, s_row, valid);
                }
            }
        }
    }

    __device__ inline void store(uint16_t* lds, int tid) {
        if constexpr (KMAJ) {
            const int kc = (tid % 8) * 8;
#pragma unroll
            for (int i = 0; i < NREG; ++i) {
                int r = tid / 8 + (NT / 8) * i;
                *reinterpret_cast<u32x4*>(lds + r * H_LDK + kc) = reg[i];
            }
        } else {
            const int kq = (tid % 16) * 4;
#pragma unroll
            for (int u = 0; u < NREG / 4; ++u) {
                int rc = 8 * (tid / 16 + (NT / 16) * u);
                const u32x4 r0 = reg[u * 4 + 0], r1 = reg[u * 4 + 1], r2 = reg[u * 4 + 2], r3 = reg[u * 4 + 3];
                const uint32_t w0[4] = {r0.x, r0.y, r0.z, r0.w};
                const uint32_t w1[4] = {r1.x, r1.y, r1.z, r1.w};
                const uint32_t w2[4] = {r2.x, r2.y, r2.z, r2.w};
                const uint32_t w3[4] = {r3.x, r3.y, r3.z, r3.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    // element 2d (low halves) and 2d+1 (high halves) of each k row
                    u32x2 lo, hi;
                    lo.x = __builtin_amdgcn_perm(w1[d], w0[d], 0x05040100u);
                    lo.y = __builtin_amdgcn_perm(w3[d], w2[d], 0x05040100u);
                    hi.x = __builtin_amdgcn_perm(w1[d], w0[d], 0x07060302u);
                    hi.y = __builtin_amdgcn_perm(w3[d], w2[d], 0x07060302u);
                    *reinterpret_cast<u32x2*>(lds + (rc + 2 * d) * H_LDK + kq) = lo;
                    *reinterpret_cast<u32x2*>(lds + (rc + 2 * d + 1) * H_LDK + kq) = hi;
                }
            }
        }
    }
};

// WGN: waves along N (1, 2 or 4); 2 waves along M. NT = 128 * WGN threads.
template <int DT, bool AK, bool BK, int BM, int BN, bool VEC, int WGN>
__global__ __launch_bounds__(128 * WGN) void gemm16_mfma_kernel(GemmArgs p) {
    constexpr int NT = 128 * WGN;
    constexpr int WM = BM / 2, WN = BN / WGN;  // wave tile
    constexpr int FM = WM / 32, FN = WN / 32;  // 32x32 fragments per wave
    __shared__ uint16_t lds[2][(BM + BN) * H_LDK];

    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int wm = wave / WGN, wn = wave % WGN;
    const int b = blockIdx.y;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // operand buffers of this batch (and of this k split): A rows are M, B rows are N
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a) + a_boff(p, b);
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.b) + b_boff(p, b);
    int K = p.K;
    if (p.split > 1) {
        const int kb = blockIdx.z * p.k_chunk;
        A += (int64_t)kb * p.sa[2];
        B += (int64_t)kb * p.sb[1];
        K = min(p.k_chunk, p.K - kb);
    }
    // With 16-byte loads the contiguous dimension is padded to 8 elements in
    // memory (it is a multiple of 8, or the operand was repacked with zero
    // padding): the range covers the padding so that the last chunk of the
    // last row loads whole
    auto pad8 = [](int v) { return (v + 7) / 8 * 8; };
    const int ea_m = VEC && !AK ? pad8(p.M) : p.M, ea_k = VEC && AK ? pad8(K) : K;
    const int eb_n = VEC && !BK ? pad8(p.N) : p.N, eb_k = VEC && BK ? pad8(K) : K;
    const int64_t a_bytes = 2 * ((int64_t)(ea_m - 1) * p.sa[1] + (int64_t)(ea_k - 1) * p.sa[2] + 1);
    const int64_t b_bytes = 2 * ((int64_t)(eb_n - 1) * p.sb[2] + (int64_t)(eb_k - 1) * p.sb[1] + 1);
    __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)min(a_bytes, (int64_t)0x7fffffff), 0x00020000);
    __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)B, 0, (int)min(b_bytes, (int64_t)0x7fffffff), 0x00020000);

    TileLoader<BM, AK, VEC, NT> la;
    TileLoader<BN, BK, VEC, NT> lb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // A: row stride sa[1] (over M), k stride sa[2]; B: "row" = N with stride sb[2], k stride sb[1]
    const int nk = (K + H_BK - 1) / H_BK;
    la.load(ra, p.sa[1], p.sa[2], m0, p.M, 0, K, tid);
    lb.load(rb, p.sb[2], p.sb[1], n0, p.N, 0, K, tid);
    la.store(lds[0], tid);
    lb.store(lds[0] + BM * H_LDK, tid);
    __syncthreads();

    const int frag_row = lane % 32;
    const int frag_k = (lane / 32) * 8;
    const int a_off = (wm * WM + frag_row) * H_LDK + frag_k;
    const int b_off = BM * H_LDK + (wn * WN + frag_row) * H_LDK + frag_k;
    u32x4 af[2][FM], bf[2][FN];
    auto read_frags = [&](const uint16_t* base, int kk, int slot) {
#pragma unroll
        for (int i = 0; i < FM; ++i) af[slot][i] = *reinterpret_cast<const u32x4*>(base + a_off + i * 32 * H_LDK + kk);
#pragma unroll
        for (int j = 0; j < FN; ++j) bf[slot][j] = *reinterpret_cast<const u32x4*>(base + b_off + j * 32 * H_LDK + kk);
    };
    // One LDS stage per iteration, four MFMA steps of 16 k each. The global
    // loads of the next stage are interleaved with the MFMAs of step 0 and
    // their LDS stores (into the other buffer) with the MFMAs of step 3, so
    // the matrix pipe stays busy while the memory instructions issue. On the
    // last iteration the loads fall outside K and read zeros (buffer range
    // check), which keeps the loop body free of branches.
    constexpr int NMF = FM * FN;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        const uint16_t* base = lds[buf];
        read_frags(base, 0, 0);
#pragma unroll
        for (int kk = 0; kk < H_BK / 16; ++kk) {
            const int cur = kk & 1;
            if (kk + 1 < H_BK / 16) read_frags(base, (kk + 1) * 16, cur ^ 1);
            if (kk == 0) {
                la.load(ra, p.sa[1], p.sa[2], m0, p.M, (kt + 1) * H_BK, K, tid);
                lb.load(rb, p.sb[2], p.sb[1], n0, p.N, (kt + 1) * H_BK, K, tid);
            }
            if (kk == H_BK / 16 - 1) {
                la.store(lds[buf ^ 1], tid);
                lb.store(lds[buf ^ 1] + BM * H_LDK, tid);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma32<DT>(af[cur][i], bf[cur][j], acc[i][j]);
            if (kk + 1 < H_BK / 16) {
                // next step's fragment reads first, then the MFMAs
                __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
            }
            if (kk == 0) {
                // one global load between consecutive MFMAs
#pragma unroll
                for (int q = 0; q < NMF; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            } else if (kk == H_BK / 16 - 1) {
                // LDS stores of the next stage between the MFMAs
#pragma unroll
                for (int q = 0; q < NMF; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
                }
            } else {
                __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    }

    // accumulator layout of v_mfma_f32_32x32x16: lane holds column lane%32,
    // register r holds row (r/4)*8 + (lane/32)*4 + r%4
    if (p.split > 1) {
        float* part = p.part + ((int64_t)blockIdx.z * p.batch + b) * p.M * p.N;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int row0 = m0 + wm * WM + i * 32 + (lane / 32) * 4, col = n0 + wn * WN + j * 32 + lane % 32;
                if (col >= p.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = row0 + (r / 4) * 8 + (r % 4);
                    if (row < p.M) part[(int64_t)row * p.N + col] = acc[i][j][r];
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
            store_frag16<DT, BM <= 128>(p, b, m0 + wm * WM + i * 32 + (lane / 32) * 4, n0 + wn * WN + j * 32 + lane % 32, acc[i][j]);
}

// ----------------------------------------------------------------------------
// sequential-k kernel on v_mfma_f32_32x32x1f32 (all dtypes; exact mode)
// ----------------------------------------------------------------------------
//
// v_mfma_f32_32x32x1f32 is two 32x32 outer products with k = 1: lane l gives
// A[row l%32] and B[col l%32] of block l/32, and every output gets one fused
// multiply-add with a single rounding. Feeding the same A to both blocks makes
// one instruction a 32x64 rank-1 update, and issuing them for k = 0, 1, 2, ...
// reproduces acc = fmaf(a_k, b_k, acc) in sequence for every output: the
// reference SIMD tile's order, at the float32 matrix-core rate. Operands of
// any input dtype are widened to float32 (exactly) on their way into LDS.

constexpr int Q_BK = 16;   // k per LDS stage

__device__ inline f32x32 mfma_x1(float a, float b, f32x32 c) {
    return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}

// Widens the elements of a 16-byte chunk to float32.
template <int DT>
__device__ inline void widen_chunk(u32x4 v, float* out) {
    if constexpr (DT == TVK_F32) {
        // bit-cast the whole vector: clang 22 miscompiles a bit-cast of one
        // ext_vector element (it reads element 0 for every element)
        const f32x4 fv = __builtin_bit_cast(f32x4, v);
        out[0] = fv.x; out[1] = fv.y; out[2] = fv.z; out[3] = fv.w;
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (DT == TVK_F16) {
                out[2 * i] = (float)__builtin_bit_cast(half_t, (uint16_t)(w[i] & 0xffffu));
                out[2 * i + 1] = (float)__builtin_bit_cast(half_t, (uint16_t)(w[i] >> 16));
            } else {
                out[2 * i] = __builtin_bit_cast(float, w[i] << 16);
                out[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
            }
        }
    }
}

// One operand tile in its own global layout: OUTER rows x INNER contiguous
// elements, staged as float32 in LDS with the same layout ([OUTER][INNER+4]).
template <int DT, int OUTER, int INNER, bool VEC>
struct SeqLoader {
    static constexpr int ES = DT == TVK_F32 ? 4 : 2;
    static constexpr int CE = 16 / ES;                    // elements per chunk
    static constexpr int CPR = INNER / CE;                // chunks per row
    static constexpr int NCH = OUTER * CPR;               // chunks per tile
    static constexpr int PER = (NCH + 255) / 256;
    static constexpr int LD = INNER + 4;
    u32x4 reg[PER];

    __device__ inline void load(__amdgpu_buffer_rsrc_t r, int64_t s_outer, int64_t s_inner, int outer0, int outer_n,
                                int inner0, int inner_n, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int id = tid + 256 * i;
            const int ro = id / CPR, ci = (id % CPR) * CE;
            const int go = outer0 + ro, gi = inner0 + ci;
            const bool ok = (id < NCH) && go < outer_n;
            const int valid = inner_n - gi;
            const int64_t off = (int64_t)go * s_outer + (int64_t)gi * s_inner;
            if constexpr (VEC) {
                reg[i] = buf_load16(r, (ok && valid > 0) ? (uint32_t)(off * ES) : kOOB);
            } else {
                uint32_t e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < CE; ++j) {
                    const uint32_t o = (ok && j < valid) ? (uint32_t)((off + j * s_inner) * ES) : kOOB;
                    if constexpr (ES == 4) e[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)o, 0, 0);
                    else e[j] = buf_load2(r, o);
                }
                if constexpr (ES == 4) reg[i] = u32x4{e[0], e[1], e[2], e[3]};
                else reg[i] = u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
            }
        }
    }

    __device__ inline void store(float* lds, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int id = tid + 256 * i;
            if (id >= NCH) break;
            const int ro = id / CPR, ci = (id % CPR) * CE;
            float f[8];
            widen_chunk<DT>(reg[i], f);
#pragma unroll
            for (int j = 0; j < CE; j += 4)
                *reinterpret_cast<f32x4*>(lds + ro * LD + ci + j) = f32x4{f[j], f[j + 1], f[j + 2], f[j + 3]};
        }
    }
};

template <int DT, bool AK, bool BK, int BM, int BN, bool VEC>
__global__ __launch_bounds__(256) void gemm_seq_mfma_kernel(GemmArgs p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 64;
    // A k-major: [BM][Q_BK]; A m-major: [Q_BK][BM]. Same for B with N.
    typedef SeqLoader<DT, AK ? BM : Q_BK, AK ? Q_BK : BM, VEC> LA;
    typedef SeqLoader<DT, BK ? BN : Q_BK, BK ? Q_BK : BN, VEC> LB;
    constexpr int A_FL = (AK ? BM : Q_BK) * LA::LD;
    constexpr int B_FL = (BK ? BN : Q_BK) * LB::LD;
    __shared__ float lds[2][A_FL + B_FL];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / 2, wn = wave % 2;
    const int b = blockIdx.y;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    constexpr int ES = DT == TVK_F32 ? 4 : 2;
    const char* A = reinterpret_cast<const char*>(p.a) + a_boff(p, b) * ES;
    const char* B = reinterpret_cast<const char*>(p.b) + b_boff(p, b) * ES;
    const int64_t a_bytes = ES * ((int64_t)(p.M - 1) * p.sa[1] + (int64_t)(p.K - 1) * p.sa[2] + 1);
    const int64_t b_bytes = ES * ((int64_t)(p.N - 1) * p.sb[2] + (int64_t)(p.K - 1) * p.sb[1] + 1);
    __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)min(a_bytes, (int64_t)0x7fffffff), 0x00020000);
    __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)B, 0, (int)min(b_bytes, (int64_t)0x7fffffff), 0x00020000);

    LA la;
    LB lb;
    auto load = [&](int k0) {
        if constexpr (AK) la.load(ra, p.sa[1], p.sa[2], m0, p.M, k0, p.K, tid);
        else la.load(ra, p.sa[2], p.sa[1], k0, p.K, m0, p.M, tid);
        if constexpr (BK) lb.load(rb, p.sb[2], p.sb[1], n0, p.N, k0, p.K, tid);
        else lb.load(rb, p.sb[1], p.sb[2], k0, p.K, n0, p.N, tid);
    };

    f32x32 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 32; ++r) acc[i][j][r] = 0.0f;

    const int nk = (p.K + Q_BK - 1) / Q_BK;
    load(0);
    la.store(lds[0], tid);
    lb.store(lds[0] + A_FL, tid);
    __syncthreads();
    const int arow = wm * WM + lane % 32;   // + 32*i
    const int bcol = wn * WN + lane;        // + 64*j
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * Q_BK);
        const float* As = lds[buf];
        const float* Bs = lds[buf] + A_FL;
#pragma unroll
        for (int k4 = 0; k4 < Q_BK; k4 += 4) {
            float av[FM][4], bv[FN][4];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                if constexpr (AK) {
                    f32x4 v = *reinterpret_cast<const f32x4*>(As + (arow + 32 * i) * LA::LD + k4);
                    av[i][0] = v.x; av[i][1] = v.y; av[i][2] = v.z; av[i][3] = v.w;
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) av[i][q] = As[(k4 + q) * LA::LD + arow + 32 * i];
                }
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (BK) {
                    f32x4 v = *reinterpret_cast<const f32x4*>(Bs + (bcol + 64 * j) * LB::LD + k4);
                    bv[j][0] = v.x; bv[j][1] = v.y; bv[j][2] = v.z; bv[j][3] = v.w;
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) bv[j][q] = Bs[(k4 + q) * LB::LD + bcol + 64 * j];
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = mfma_x1(av[i][q], bv[j][q], acc[i][j]);
        }
        if (kt + 1 < nk) {
            la.store(lds[buf ^ 1], tid);
            lb.store(lds[buf ^ 1] + A_FL, tid);
        }
        __syncthreads();
    }

    // output of block r/16: row (rr/4)*8 + (lane/32)*4 + rr%4, column (r/16)*32 + lane%32
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int row0 = m0 + wm * WM + 32 * i + (lane / 32) * 4;
            const int col0 = n0 + wn * WN + 64 * j + lane % 32;
            store_frag16<DT, BM <= 128>(p, b, row0, col0, acc[i][j].lo);
            store_frag16<DT, BM <= 128>(p, b, row0, col0 + 32, acc[i][j].hi);
        }
}

// The same order on 64x64 tiles for products with few tiles (1024^2 float32:
// 256 tiles against 128 of 64x128): each of the four waves owns 16 rows x 64
// columns and issues v_mfma_f32_16x16x1_4b_f32 with its row's A value in all
// four blocks, so one instruction is a 16x64 rank-1 update (block q: columns
// 16q .. 16q+15), at the matrix core's float32 rate like the 32x32x1 form.
// Every output again accumulates fmaf(a_k, b_k, acc) for k = 0, 1, 2, ...
template <int DT, bool AK, bool BK, int BM, int BN, bool VEC>
__global__ __launch_bounds__(256) void gemm_seq16_kernel(GemmArgs p) {
    static_assert(BM == 64 && BN == 64, "64x64 tiles of four 16x64 waves");
    typedef SeqLoader<DT, AK ? BM : Q_BK, AK ? Q_BK : BM, VEC> LA;
    typedef SeqLoader<DT, BK ? BN : Q_BK, BK ? Q_BK : BN, VEC> LB;
    constexpr int A_FL = (AK ? BM : Q_BK) * LA::LD;
    constexpr int B_FL = (BK ? BN : Q_BK) * LB::LD;
    __shared__ float lds[2][A_FL + B_FL];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int b = blockIdx.y;
    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    constexpr int ES = DT == TVK_F32 ? 4 : 2;
    const char* A = reinterpret_cast<const char*>(p.a) + a_boff(p, b) * ES;
    const char* B = reinterpret_cast<const char*>(p.b) + b_boff(p, b) * ES;
    const int64_t a_bytes = ES * ((int64_t)(p.M - 1) * p.sa[1] + (int64_t)(p.K - 1) * p.sa[2] + 1);
    const int64_t b_bytes = ES * ((int64_t)(p.N - 1) * p.sb[2] + (int64_t)(p.K - 1) * p.sb[1] + 1);
    __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)min(a_bytes, (int64_t)0x7fffffff), 0x00020000);
    __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)B, 0, (int)min(b_bytes, (int64_t)0x7fffffff), 0x00020000);

    LA la;
    LB lb;
    auto load = [&](int k0) {
        if constexpr (AK) la.load(ra, p.sa[1], p.sa[2], m0, p.M, k0, p.K, tid);
        else la.load(ra, p.sa[2], p.sa[1], k0, p.K, m0, p.M, tid);
        if constexpr (BK) lb.load(rb, p.sb[2], p.sb[1], n0, p.N, k0, p.K, tid);
        else lb.load(rb, p.sb[1], p.sb[2], k0, p.K, n0, p.N, tid);
    };

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    const int nk = (p.K + Q_BK - 1) / Q_BK;
    load(0);
    la.store(lds[0], tid);
    lb.store(lds[0] + A_FL, tid);
    __syncthreads();
    const int arow = wave * 16 + lane % 16;   // the same row in all four blocks
    const int bcol = lane;                    // block lane / 16, column lane % 16
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * Q_BK);
        const float* As = lds[buf];
        const float* Bs = lds[buf] + A_FL;
#pragma unroll
        for (int k4 = 0; k4 < Q_BK; k4 += 4) {
            float av[4], bv[4];
            if constexpr (AK) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(As + arow * LA::LD + k4);
                av[0] = v.x; av[1] = v.y; av[2] = v.z; av[3] = v.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) av[q] = As[(k4 + q) * LA::LD + arow];
            }
            if constexpr (BK) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(Bs + bcol * LB::LD + k4);
                bv[0] = v.x; bv[1] = v.y; bv[2] = v.z; bv[3] = v.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) bv[q] = Bs[(k4 + q) * LB::LD + bcol];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x1f32(av[q], bv[q], acc, 0, 0, 0);
        }
        if (kt + 1 < nk) {
            la.store(lds[buf ^ 1], tid);
            lb.store(lds[buf ^ 1] + A_FL, tid);
        }
        __syncthreads();
    }

    // register r: block r / 4 (columns 16 (r / 4) ..), row (lane / 16) * 4 + r % 4, column lane % 16
    if (!p.has_bias && p.act == TVK_ACT_NONE) {
        // no bias, no activation: alpha times the sum, as store_out computes it,
        // with the batch offset once for the lane's 16 outputs
        typedef typename elem<DT>::T T;
        T* c = reinterpret_cast<T*>(p.c) + c_boff(p, b);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wave * 16 + (lane / 16) * 4 + r % 4;
            const int col = n0 + (r / 4) * 16 + lane % 16;
            if (row < p.M && col < p.N) {
#pragma clang fp contract(off)
                const float o = acc[r] * p.alpha;
                c[(int64_t)row * p.sc[1] + (int64_t)col * p.sc[2]] = elem<DT>::from_f32(o);
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = m0 + wave * 16 + (lane / 16) * 4 + r % 4;
        const int col = n0 + (r / 4) * 16 + lane % 16;
        if (row < p.M && col < p.N) store_out<DT, true>(p, b, row, col, acc[r]);
    }
}

// ----------------------------------------------------------------------------
// operand repack: dst[b][r][c] = src(b, r, c) for c < C, 0 for C <= c < Cp
// (c is the operand's contiguous dimension; rows are Cp elements apart)
// ----------------------------------------------------------------------------

__global__ __launch_bounds__(256) void repack16_kernel(const uint16_t* src, uint16_t* dst, int64_t s0, int64_t sr, int64_t sc,
                                                        int batch, int R, int C, int Cp) {
    const int64_t chunks = (int64_t)batch * R * (Cp / 8);
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < chunks; q += (int64_t)gridDim.x * 256) {
        const int c0 = (int)(q % (Cp / 8)) * 8;
        const int64_t br = q / (Cp / 8);
        const int r = (int)(br % R), b = (int)(br / R);
        const uint16_t* sp = src + (int64_t)b * s0 + (int64_t)r * sr;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c0 + 2 * e;
            const uint32_t lo = c < C ? sp[(int64_t)c * sc] : 0u;
            const uint32_t hi = c + 1 < C ? sp[(int64_t)(c + 1) * sc] : 0u;
            w[e] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x4*>(dst + ((int64_t)b * R + r) * Cp + c0) = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// ----------------------------------------------------------------------------
// host dispatch
// ----------------------------------------------------------------------------

enum class Kern { K0, GENERIC, SEQ128, SEQ64, SEQ16, MFMA256, MFMA256W8, MFMA128, MFMA64, SKINNY, DMA256, DMA128, DMA128R8, DMA128X256, DMA256X128 };

struct Plan {
    Kern kern;
    bool ak = true, bk = true, vec = true;
    const char* name;
    int split = 1, k_chunk = 0;   // MFMA128 split-K
    // operands copied to an aligned workspace layout first (contiguous
    // dimension padded with zeros to a multiple of 8 elements)
    bool repack_a = false, repack_b = false;
};

bool fits_i32(int64_t v) { return v >= 0 && v <= 0x7fffffff; }

int64_t operand_extent_bytes(int64_t rows, int64_t s_row, int64_t cols, int64_t s_col, size_t es) {
    return (int64_t)es * ((rows - 1) * s_row + (cols - 1) * s_col + 1);
}

// Row (mc) and column (nc) block sizes that bring A's and B's per-matrix
// extents below 2 GiB, the tiled kernels' buffer range. Unchanged sizes when
// they already fit; false when no block of whole rows and columns fits (a
// single row or column spans 2 GiB), which leaves the product to the generic
// kernel.
bool extent_chunks(const tvk_gemm_desc& d, int64_t& mc, int64_t& nc) {
    const int64_t es = (int64_t)dtype_size(d.dtype), lim = (int64_t(0x7fffffff) - 256) / es;
    auto rows_fitting = [&](int64_t rows, int64_t s_row, int64_t cols, int64_t s_col) -> int64_t {
        const int64_t fixed = (cols - 1) * s_col + 1;
        if (fixed >= lim) return 0;
        if (s_row == 0 || (rows - 1) * s_row + fixed < lim) return rows;
        int64_t r = (lim - fixed) / s_row + 1;
        if (r >= 256) r = r / 256 * 256;   // whole 256-row tiles
        return std::min(r, rows);
    };
    mc = rows_fitting(d.M, d.a_stride[1], d.K, d.a_stride[2]);
    nc = rows_fitting(d.N, d.b_stride[2], d.K, d.b_stride[1]);
    return mc > 0 && nc > 0;
}

GemmArgs make_args(const tvk_gemm_desc& d) {
    GemmArgs p;
    memset(&p, 0, sizeof(p));
    p.a = d.a; p.b = d.b; p.bias = d.bias; p.c = d.c;
    for (int i = 0; i < 3; ++i) {
        p.sa[i] = d.a_stride[i]; p.sb[i] = d.b_stride[i]; p.sbias[i] = d.bias_stride[i]; p.sc[i] = d.c_stride[i];
    }
    p.M = (int)d.M; p.N = (int)d.N; p.K = (int)d.K;
    p.batch = (int)d.batch;
    p.alpha = (float)d.alpha;
    p.beta = (float)d.beta;
    p.has_bias = (d.bias != nullptr && d.beta != 0.0) ? 1 : 0;
    p.act = d.activation;
    p.bh = d.batch_inner > 1 ? (int)d.batch_inner : 1;
    if (p.bh > 1) {
        p.sa_h = d.a_stride_inner; p.sb_h = d.b_stride_inner; p.sbias_h = d.bias_stride_inner; p.sc_h = d.c_stride_inner;
    }
    return p;
}

// Leading dimension of a repacked operand: its contiguous dimension padded to
// 8, or to 32 when that dimension is K (the padding is zeros, so the
// LDS-ring kernels can run a last k step of 32 past K).
int64_t pad8(int64_t v) { return (v + 7) / 8 * 8; }
int64_t repack_ld(int64_t v, bool kdim) { return kdim ? (v + 31) / 32 * 32 : pad8(v); }

// Whether every load of k in [K, K rounded up to 32) returns zero under plan
// pl: each k-contiguous operand is repacked (zero-padded rows), and each
// m/n-contiguous one has rows at least as long as its extent, so row K and
// beyond lie past its buffer range.
bool k_tail_zero(const tvk_gemm_desc& d, const struct Plan& pl);

// Arguments as the kernels see them once the planned repacks are done (the
// pointers of repacked operands only matter for alignment: workspace offsets
// are 256-byte aligned).
GemmArgs repacked_args(const tvk_gemm_desc& d, const struct Plan& pl);

// Operand layout facts every tiled kernel shares: which dimension of each
// operand is contiguous, whether 16-byte loads are legal (vec) and which
// operands are worth one copy into an aligned layout. False: no tiled kernel
// applies and the generic kernel runs.
bool plan_layout(const tvk_gemm_desc& d, Plan& pl) {
    const size_t es = dtype_size(d.dtype);
    // which dimension of each operand is contiguous (size-1 dims have any stride)
    const bool a_k = d.a_stride[2] == 1 || d.K == 1;
    const bool a_m = d.a_stride[1] == 1 || d.M == 1;
    const bool b_k = d.b_stride[1] == 1 || d.K == 1;
    const bool b_n = d.b_stride[2] == 1 || d.N == 1;
    if (!(a_k || a_m) || !(b_k || b_n)) return false;
    if (operand_extent_bytes(d.M, d.a_stride[1], d.K, d.a_stride[2], es) >= 0x7fffffff ||
        operand_extent_bytes(d.N, d.b_stride[2], d.K, d.b_stride[1], es) >= 0x7fffffff)
        return false;
    pl.ak = a_k;
    pl.bk = b_k;
    // 16-byte chunks need 16-byte aligned rows and whole chunks along the contiguous dimension
    const int64_t ce = 16 / (int64_t)es;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    bool vec = al16(d.a) && al16(d.b);
    if (d.batch > 1) vec = vec && d.a_stride[0] % ce == 0 && d.b_stride[0] % ce == 0;
    if (d.batch_inner > 1) vec = vec && d.a_stride_inner % ce == 0 && d.b_stride_inner % ce == 0;
    if (pl.ak) vec = vec && d.K % ce == 0 && (d.M == 1 || d.a_stride[1] % ce == 0);
    else vec = vec && d.M % ce == 0 && (d.K == 1 || d.a_stride[2] % ce == 0);
    if (pl.bk) vec = vec && d.K % ce == 0 && (d.N == 1 || d.b_stride[2] % ce == 0);
    else vec = vec && d.N % ce == 0 && (d.K == 1 || d.b_stride[1] % ce == 0);
    pl.vec = vec;
    // A sizeable fp16/bf16 product whose operands miss the 16-byte layout
    // (rows not 8-element multiples, as [1000,777] or a sliced view) is worth
    // one copy of the offending operands into an aligned layout
    // (the repack copies address one batch dimension: a two-level batch is not repacked)
    if (!vec && d.dtype != TVK_F32 && !(d.flags & TVK_GEMM_EXACT) && !skinny_applies(d.M, d.N, d.K, d.batch) &&
        d.batch_inner <= 1 && (double)d.M * d.N * d.K * d.batch >= double(1 << 28)) {
        auto ok_a = [&]() {
            bool v = al16(d.a) && (d.batch == 1 || d.a_stride[0] % ce == 0);
            if (pl.ak) return v && d.K % ce == 0 && (d.M == 1 || d.a_stride[1] % ce == 0);
            return v && d.M % ce == 0 && (d.K == 1 || d.a_stride[2] % ce == 0);
        };
        auto ok_b = [&]() {
            bool v = al16(d.b) && (d.batch == 1 || d.b_stride[0] % ce == 0);
            if (pl.bk) return v && d.K % ce == 0 && (d.N == 1 || d.b_stride[2] % ce == 0);
            return v && d.N % ce == 0 && (d.K == 1 || d.b_stride[1] % ce == 0);
        };
        pl.repack_a = !ok_a();
        pl.repack_b = !ok_b();
        pl.vec = true;
    }
    return true;
}

Plan with_kern(Plan pl, Kern k, const char* name) {
    pl.kern = k;
    pl.name = name;
    pl.split = 1;
    pl.k_chunk = 0;
    return pl;
}

// The M <= 16 streaming kernel on a laid-out plan (no repacks: the layout
// never repacks such a product); it loads A by rows of k, so 16-byte loads
// need A k-contiguous too.
Plan skinny_plan(const tvk_gemm_desc& d, Plan pl) {
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    bool v = al16(d.a) && al16(d.b) && pl.ak && d.K % 8 == 0 && (d.M == 1 || d.a_stride[1] % 8 == 0);
    if (d.batch > 1) v = v && d.a_stride[0] % 8 == 0 && d.b_stride[0] % 8 == 0;
    if (d.batch_inner > 1) v = v && d.a_stride_inner % 8 == 0 && d.b_stride_inner % 8 == 0;
    if (pl.bk) v = v && (d.N == 1 || d.b_stride[2] % 8 == 0);
    else v = v && d.N % 8 == 0 && (d.K == 1 || d.b_stride[1] % 8 == 0);
    pl = with_kern(pl, Kern::SKINNY, nullptr);
    pl.vec = v;
    pl.name = skinny_name(make_args(d), pl.bk, v);
    return pl;
}

// MFMA128 with K split about `want` ways into chunks of whole 64-k steps,
// float32 partials; false when that would not split or the partials would
// exceed 512 MB.
bool split_plan(const tvk_gemm_desc& d, int64_t want, Plan& pl, Kern kern = Kern::MFMA128) {
    if (want < 2) return false;
    const int64_t chunk = ((d.K + want - 1) / want + 63) / 64 * 64;
    const int64_t split = (d.K + chunk - 1) / chunk;
    if (split < 2 || split * d.batch * d.M * d.N * 4 > (int64_t(512) << 20)) return false;
    const char* name = "gemm16_mfma_128x128_splitk";
    switch (kern) {
    case Kern::DMA128: name = "gemm16_dma_128x128_splitk"; break;
    case Kern::DMA128R8: name = "gemm16_dma_128x128_ring8_splitk"; break;
    case Kern::DMA256X128: name = "gemm16_dma_256x128_splitk"; break;
    case Kern::DMA128X256: name = "gemm16_dma_128x256_splitk"; break;
    case Kern::DMA256: name = "gemm16_dma_256x256_splitk"; break;
    default: break;
    }
    pl = with_kern(pl, kern, name);
    pl.split = (int)split;
    pl.k_chunk = (int)chunk;
    return true;
}

// The kernel chosen from the shape alone (used unless the kernel-choice table
// holds another candidate for the product's shape class).
Plan make_plan(const tvk_gemm_desc& d) {
    Plan pl{Kern::GENERIC, true, true, true, "gemm_generic"};
    if (d.K == 0) return Plan{Kern::K0, true, true, true, "gemm_k0_fill"};
    if (!plan_layout(d, pl)) return pl;
    if (d.dtype != TVK_F32 && !(d.flags & TVK_GEMM_EXACT) && skinny_applies(d.M, d.N, d.K, d.batch))
        return skinny_plan(d, pl);
    const int64_t t256 = ((d.M + 255) / 256) * ((d.N + 255) / 256) * d.batch;
    const bool big = d.M >= 256 && d.N >= 256 && t256 >= 192;
    if (d.dtype == TVK_F32 || (d.flags & TVK_GEMM_EXACT)) {
        // 128x128 tiles at every size (a 256x256 variant, four waves of 128x128
        // float32 accumulators, ran 2.3-8x slower from 2048^3 to 8192^3)
        pl.kern = Kern::SEQ128;
        pl.name = "gemm_seq_mfma_128x128";
        // at most one round of 128x128 tiles: 64x64 tiles of four 16x64 waves,
        // four times the workgroups (same k order; 1024^3 53.7 -> 40.0 us,
        // 512^3 x 16 53.3 -> 48.2, 4096x1024x1024 91.1 -> 87.4; 2048^3 within 1 %;
        // the 64x128 tiles of 2x2 waves of 32x64 stay a kernel-choice candidate)
        if (((d.M + 127) / 128) * ((d.N + 127) / 128) * d.batch <= 256) {
            pl.kern = Kern::SEQ16;
            pl.name = "gemm_seq_mfma_64x64";
        }
        return pl;
    }
    const bool dma_ok = pl.vec && dma_applies(repacked_args(d, pl), pl.ak, pl.bk);
    // 256x256 tiles whose last round on the 256 CUs is at most half full, with
    // few rounds (the transformer's gate_up, 8192x3072x512: 384 tiles, one and
    // a half rounds; 6144^3: 576 tiles): 128x256 tiles, twice as many, whole
    // rounds (gate_up 38.2-40.7 us against 41.9-45.8 for 256x256; 6144^3 409
    // against 449 for 256x128 tiles)
    const bool half_round = t256 < 1024 && t256 % 256 != 0 && t256 % 256 <= 128;
    if (big && dma_ok) {
        pl.kern = half_round ? Kern::DMA128X256 : Kern::DMA256;
        pl.name = half_round ? "gemm16_dma_128x256" : "gemm16_dma_256x256";
    } else if (big) {
        // 8 waves; the 4-wave form stays a kernel-choice candidate
        pl.kern = Kern::MFMA256W8;
        pl.name = "gemm16_mfma_256x256_w8";
    } else {
        pl.kern = Kern::MFMA128;
        pl.name = "gemm16_mfma_128x128";
        const int64_t t128 = ((d.M + 127) / 128) * ((d.N + 127) / 128) * d.batch;
        // Few output tiles and a long K (weight gradients, batch-256 layers):
        // split K into a power of two of chunks so at least one workgroup per
        // CU runs, chunks of at least 256 k, partials in float32. Below
        // K = 2048 the partials' round trip costs more than the idle CUs.
        // The LDS-ring kernel takes the split where it applies (measured
        // 1.2-1.7x on the C2/C3 batch-256 and weight-gradient products, 1.08-1.2x
        // on 10-column, 32-row and 64-row outputs).
        if (t128 < 192 && d.K >= 2048) {
            auto pow2_ceil = [](int64_t v) { int64_t r = 1; while (r < v) r *= 2; return r; };
            auto pow2_floor = [](int64_t v) { int64_t r = 1; while (r * 2 <= v) r *= 2; return r; };
            const bool dma = pl.vec && dma_applies(repacked_args(d, pl), pl.ak, pl.bk);
            if (split_plan(d, std::min<int64_t>({pow2_ceil((256 + t128 - 1) / t128), pow2_floor(d.K / 256), 32}), pl,
                           dma ? Kern::DMA128 : Kern::MFMA128))
                return pl;
        }
        if (t128 <= 128 && !(dma_ok && d.K >= 1024)) {
            // at most half as many 128x128 tiles as CUs: 64x64 tiles on two
            // waves, four times the workgroups (measured ahead of both 128x128
            // kernels: 1.27-1.49x on 256x4096x784 and 8192x96x512, 64 tiles;
            // 1.05-1.08x on 8192x256x512, 128 tiles, on three boxes; 1.3x on
            // the per-head attention products, 16 and 32 tiles). From K = 1024
            // the ring's 128x128 tiles lead again (1024^3: 14.4 against 16.0 us)
            pl.kern = Kern::MFMA64;
            pl.name = "gemm16_mfma_64x64";
        } else if (dma_ok) {
            // the LDS-ring kernel on 128x128 tiles (13-18 % ahead of the
            // register-staged one on 8192 x {512, 256} x 512)
            pl.kern = Kern::DMA128;
            pl.name = "gemm16_dma_128x128";
            // More than one round of 128x128 tiles at K >= 1024: the tile whose
            // rounds of 256 workgroups cost least, a 128x128 / 128x256 / 256x256
            // tile costing 1 : 1.6 : 2.4 (measured at 2560^3, 3072^3, 4096x2048x4096
            // and 2048x4096x2048: 1.10-1.24x over 128x128 tiles)
            if (t128 > 256 && d.K >= 1024) {
                const int64_t t12 = ((d.M + 127) / 128) * ((d.N + 255) / 256) * d.batch;
                auto rounds = [](int64_t t) { return (double)((t + 255) / 256); };
                const double c128 = rounds(t128), c12 = 1.6 * rounds(t12), c256 = 2.4 * rounds(t256);
                if (c256 < c128 && c256 < c12 && d.M >= 256 && d.N >= 256) {
                    pl.kern = Kern::DMA256;
                    pl.name = "gemm16_dma_256x256";
                } else if (c12 < c128 && d.N >= 256) {
                    pl.kern = Kern::DMA128X256;
                    pl.name = "gemm16_dma_128x256";
                }
            }
        }
    }
    return pl;
}

// A candidate's name in the kernel-choice table: the kernel name, and the
// number of K chunks for a split-K plan.
std::string plan_id(const Plan& pl) {
    std::string id = pl.name;
    if (pl.split > 1) id += ":" + std::to_string(pl.split);
    return id;
}

// Every plan that computes this product, make_plan's choice first. float32
// (and TVK_GEMM_EXACT) offers only the sequential-order kernels, which give
// identical bits; float16/bfloat16 offer every tiled kernel whose layout
// conditions hold.
std::vector<Plan> candidate_plans(const tvk_gemm_desc& d) {
    std::vector<Plan> out{make_plan(d)};
    if (out[0].kern == Kern::K0 || out[0].kern == Kern::GENERIC) return out;
    Plan lay{Kern::GENERIC, true, true, true, "gemm_generic"};
    plan_layout(d, lay);
    auto add = [&](const Plan& p) {
        for (const Plan& q : out)
            if (q.kern == p.kern && q.split == p.split) return;
        out.push_back(p);
    };
    if (d.dtype == TVK_F32 || (d.flags & TVK_GEMM_EXACT)) {
        add(with_kern(lay, Kern::SEQ128, "gemm_seq_mfma_128x128"));
        add(with_kern(lay, Kern::SEQ64, "gemm_seq_mfma_64x128"));
        add(with_kern(lay, Kern::SEQ16, "gemm_seq_mfma_64x64"));
        return out;
    }
    if (skinny_applies(d.M, d.N, d.K, d.batch)) add(skinny_plan(d, lay));
    add(with_kern(lay, Kern::MFMA128, "gemm16_mfma_128x128"));
    add(with_kern(lay, Kern::MFMA64, "gemm16_mfma_64x64"));
    for (int64_t want : {2, 4, 8, 16}) {
        Plan p = lay;
        if (split_plan(d, want, p)) add(p);
    }
    const bool dma = lay.vec && dma_applies(repacked_args(d, lay), lay.ak, lay.bk);
    if (dma) {
        add(with_kern(lay, Kern::DMA128, "gemm16_dma_128x128"));
        add(with_kern(lay, Kern::DMA128R8, "gemm16_dma_128x128_ring8"));
        for (int64_t want : {2, 4, 8, 16}) {
            Plan p = lay;
            if (split_plan(d, want, p, Kern::DMA128)) add(p);
            p = lay;
            if (split_plan(d, want, p, Kern::DMA128R8)) add(p);
        }
    }
    if (d.M >= 128 && d.N >= 128) {
        add(with_kern(lay, Kern::MFMA256W8, "gemm16_mfma_256x256_w8"));
        add(with_kern(lay, Kern::MFMA256, "gemm16_mfma_256x256"));
        if (dma) {
            add(with_kern(lay, Kern::DMA256, "gemm16_dma_256x256"));
            add(with_kern(lay, Kern::DMA128X256, "gemm16_dma_128x256"));
            add(with_kern(lay, Kern::DMA256X128, "gemm16_dma_256x128"));
            // the larger ring tiles split along K too (fewer workgroups fetch each
            // operand block; more float32 partials)
            for (Kern k : {Kern::DMA256X128, Kern::DMA128X256, Kern::DMA256})
                for (int64_t want : {2, 4, 8, 16}) {
                    Plan p = lay;
                    if (split_plan(d, want, p, k)) add(p);
                }
        }
    }
    return out;
}

// Shape class of a product in the kernel-choice table, after the reference's
// matmul tune key (src/api/ops/matmul.cpp:166-171,541): dtype, flags,
// epilogue, the operand layout facts that decide which kernels apply, and
// ceil(log2) of M, N, K and the batch.
uint64_t tune_key(const tvk_gemm_desc& d) {
    Plan lay{Kern::GENERIC, true, true, true, "gemm_generic"};
    const bool tiled = d.K > 0 && plan_layout(d, lay);
    const bool dma = tiled && lay.vec && dma_applies(repacked_args(d, lay), lay.ak, lay.bk);
    auto lg = [](int64_t v) {
        uint64_t r = 0;
        while (r < 63 && (int64_t(1) << r) < v) ++r;
        return r;
    };
    const bool bias = d.bias != nullptr && d.beta != 0.0;
    return (uint64_t)(d.dtype & 15) | (uint64_t)(d.flags & 1) << 4 | (uint64_t)(d.activation & 3) << 5 |
           (uint64_t)bias << 7 | (uint64_t)tiled << 8 | (uint64_t)lay.ak << 9 | (uint64_t)lay.bk << 10 |
           (uint64_t)lay.vec << 11 | (uint64_t)dma << 12 | (uint64_t)lay.repack_a << 13 | (uint64_t)lay.repack_b << 14 |
           lg(d.M) << 16 | lg(d.N) << 24 | lg(d.K) << 32 | lg(d.batch) << 40;
}

GemmArgs repacked_args(const tvk_gemm_desc& d, const Plan& pl) {
    GemmArgs p = make_args(d);
    static const char aligned_dummy[16] __attribute__((aligned(256))) = {0};
    if (pl.repack_a) {
        p.a = aligned_dummy;
        if (pl.ak) { const int64_t ld = repack_ld(d.K, true); p.sa[0] = d.M * ld; p.sa[1] = ld; p.sa[2] = 1; }
        else { const int64_t ld = pad8(d.M); p.sa[0] = d.K * ld; p.sa[1] = 1; p.sa[2] = ld; }
        p.a_ext = 2 * p.sa[0];
    }
    if (pl.repack_b) {
        p.b = aligned_dummy;
        if (pl.bk) { const int64_t ld = repack_ld(d.K, true); p.sb[0] = d.N * ld; p.sb[1] = 1; p.sb[2] = ld; }
        else { const int64_t ld = pad8(d.N); p.sb[0] = d.K * ld; p.sb[1] = ld; p.sb[2] = 1; }
        p.b_ext = 2 * p.sb[0];
    }
    p.kzero = k_tail_zero(d, pl) ? 1 : 0;
    return p;
}

bool k_tail_zero(const tvk_gemm_desc& d, const Plan& pl) {
    if (d.K % 32 == 0) return true;
    const bool a_ok = pl.ak ? pl.repack_a : (pl.repack_a || d.a_stride[2] >= d.M);
    const bool b_ok = pl.bk ? pl.repack_b : (pl.repack_b || d.b_stride[1] >= d.N);
    return a_ok && b_ok;
}

#define TVK_LAYOUT_SWITCH(PL, NTHR, KERNEL, ...)                                            \
    do {                                                                                    \
        if ((PL).vec) {                                                                     \
            if ((PL).ak && (PL).bk) hipLaunchKernelGGL((KERNEL<DT, true, true, BM, BN, true __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);   \
            else if ((PL).ak) hipLaunchKernelGGL((KERNEL<DT, true, false, BM, BN, true __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);        \
            else if ((PL).bk) hipLaunchKernelGGL((KERNEL<DT, false, true, BM, BN, true __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);        \
            else hipLaunchKernelGGL((KERNEL<DT, false, false, BM, BN, true __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);                    \
        } else {                                                                            \
            if ((PL).ak && (PL).bk) hipLaunchKernelGGL((KERNEL<DT, true, true, BM, BN, false __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);  \
            else if ((PL).ak) hipLaunchKernelGGL((KERNEL<DT, true, false, BM, BN, false __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);       \
            else if ((PL).bk) hipLaunchKernelGGL((KERNEL<DT, false, true, BM, BN, false __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);       \
            else hipLaunchKernelGGL((KERNEL<DT, false, false, BM, BN, false __VA_ARGS__>), grid, dim3(NTHR), 0, s, p);                   \
        }                                                                                   \
    } while (0)

template <int DT, int BM, int BN, int WGN>
void launch_mfma(const Plan& pl, GemmArgs& p, dim3 grid, hipStream_t s) {
    TVK_LAYOUT_SWITCH(pl, 128 * WGN, gemm16_mfma_kernel, , WGN);
}

template <int DT, int BM, int BN>
void launch_seq(const Plan& pl, GemmArgs& p, dim3 grid, hipStream_t s) {
    TVK_LAYOUT_SWITCH(pl, 256, gemm_seq_mfma_kernel);
}

template <int DT>
void launch_seq16(const Plan& pl, GemmArgs& p, dim3 grid, hipStream_t s) {
    constexpr int BM = 64, BN = 64;
    TVK_LAYOUT_SWITCH(pl, 256, gemm_seq16_kernel);
}

// Scratch bytes one batch chunk of `nb` matrices needs under plan pl:
// repacked operands (256-byte aligned each), then split-K partials, or the
// streaming kernel's partials. rep_a / rep_b / part_b return the pieces.
size_t plan_scratch_bytes(const tvk_gemm_desc& d, const Plan& pl, int nb, size_t* rep_a_out = nullptr,
                          size_t* rep_b_out = nullptr) {
    auto al256 = [](size_t v) { return (v + 255) / 256 * 256; };
    const int64_t a_rows = pl.ak ? d.M : d.K, a_ld = repack_ld(pl.ak ? d.K : d.M, pl.ak);
    const int64_t b_rows = pl.bk ? d.N : d.K, b_ld = repack_ld(pl.bk ? d.K : d.N, pl.bk);
    const size_t rep_a = pl.repack_a ? al256((size_t)nb * a_rows * a_ld * 2) : 0;
    const size_t rep_b = pl.repack_b ? al256((size_t)nb * b_rows * b_ld * 2) : 0;
    size_t part_b = pl.split > 1 ? (size_t)pl.split * nb * d.M * d.N * 4 : 0;
    if (pl.kern == Kern::SKINNY) {
        GemmArgs q = make_args(d);
        q.batch = nb;
        part_b = skinny_scratch_bytes(q, pl.bk, pl.vec);
    }
    if (rep_a_out) *rep_a_out = rep_a;
    if (rep_b_out) *rep_b_out = rep_b;
    return rep_a + rep_b + part_b;
}

// Runs one planned product. `fixed` (capacity fixed_cap bytes) replaces the
// pool lease when the caller brings its own scratch.
template <int DT>
tvk_status run(const tvk_gemm_desc& d, const Plan& pl, hipStream_t s, char* fixed = nullptr, size_t fixed_cap = 0) {
    const GemmArgs p = make_args(d);

    // batch chunks within the grid's y limit, of whole inner batches when there
    // are two batch dimensions (each chunk then starts at an outer index bo)
    const int64_t max_y = 65535 / p.bh * p.bh;
    for (int64_t b0 = 0; b0 < d.batch; b0 += max_y) {
        const int nb = (int)std::min<int64_t>(max_y, d.batch - b0);
        const int64_t bo = b0 / p.bh;
        GemmArgs q = p;
        q.batch = nb;
        const size_t es = dtype_size(d.dtype);
        q.a = (const char*)d.a + (size_t)(bo * d.a_stride[0]) * es;
        q.b = (const char*)d.b + (size_t)(bo * d.b_stride[0]) * es;
        if (q.has_bias) q.bias = (const char*)d.bias + (size_t)(bo * d.bias_stride[0]) * es;
        q.c = (char*)d.c + (size_t)(bo * d.c_stride[0]) * es;
        // scratch: repacked operands, then split-K partials
        const int64_t a_rows = pl.ak ? d.M : d.K, a_ld = repack_ld(pl.ak ? d.K : d.M, pl.ak);
        const int64_t b_rows = pl.bk ? d.N : d.K, b_ld = repack_ld(pl.bk ? d.K : d.N, pl.bk);
        size_t rep_a = 0, rep_b = 0;
        const size_t need = plan_scratch_bytes(d, pl, nb, &rep_a, &rep_b);
        char* ws = nullptr;
        Scratch scratch;
        if (fixed) {
            if (need > fixed_cap) return fail(TVK_ERR_INVALID, "tvk_gemm: scratch of " + std::to_string(need) + " bytes exceeds the " +
                                                                   std::to_string(fixed_cap) + " provided");
            ws = fixed;
        } else if (need > 0) {
            ws = static_cast<char*>(scratch.get(need, s));
            if (!ws) return fail(TVK_ERR_OOM, "tvk_gemm: no workspace for repacked operands or split-K partials");
        }
        if constexpr (DT != TVK_F32) {
            auto repack = [&](const void* src, int64_t s0, int64_t sr, int64_t sc, int64_t rows, int64_t cols, int64_t ld, char* dst) {
                const int64_t chunks = (int64_t)nb * rows * (ld / 8);
                const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 16384);
                hipLaunchKernelGGL(repack16_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(src),
                                   reinterpret_cast<uint16_t*>(dst), s0, sr, sc, nb, (int)rows, (int)cols, (int)ld);
            };
            if (pl.repack_a) {
                if (pl.ak) repack(q.a, d.a_stride[0], d.a_stride[1], d.a_stride[2], d.M, d.K, a_ld, ws);
                else repack(q.a, d.a_stride[0], d.a_stride[2], d.a_stride[1], d.K, d.M, a_ld, ws);
                q.a = ws;
                q.sa[0] = a_rows * a_ld;
                q.sa[1] = pl.ak ? a_ld : 1;
                q.sa[2] = pl.ak ? 1 : a_ld;
                q.a_ext = 2 * q.sa[0];
            }
            if (pl.repack_b) {
                if (pl.bk) repack(q.b, d.b_stride[0], d.b_stride[2], d.b_stride[1], d.N, d.K, b_ld, ws + rep_a);
                else repack(q.b, d.b_stride[0], d.b_stride[1], d.b_stride[2], d.K, d.N, b_ld, ws + rep_a);
                q.b = ws + rep_a;
                q.sb[0] = b_rows * b_ld;
                q.sb[1] = pl.bk ? 1 : b_ld;
                q.sb[2] = pl.bk ? b_ld : 1;
                q.b_ext = 2 * q.sb[0];
            }
        }
        switch (pl.kern) {
        case Kern::K0: {
            int64_t total = (int64_t)nb * d.M * d.N;
            hipLaunchKernelGGL(gemm_k0_kernel<DT>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, q);
            break;
        }
        case Kern::GENERIC:
            hipLaunchKernelGGL(gemm_generic_kernel<DT>, dim3((unsigned)std::min<int64_t>(((int64_t)d.M * d.N + 255) / 256, 65536), nb),
                               dim3(256), 0, s, q);
            break;
        case Kern::SEQ16: {
            q.tiles_m = (int)((d.M + 63) / 64);
            q.tiles_n = (int)((d.N + 63) / 64);
            dim3 grid(q.tiles_m * q.tiles_n, nb);
            launch_seq16<DT>(pl, q, grid, s);
            break;
        }
        case Kern::SEQ128:
        case Kern::SEQ64: {
            const int TM = pl.kern == Kern::SEQ128 ? 128 : 64;
            const int TN = 128;
            q.tiles_m = (int)((d.M + TM - 1) / TM);
            q.tiles_n = (int)((d.N + TN - 1) / TN);
            dim3 grid(q.tiles_m * q.tiles_n, nb);
            if (TM == 128) launch_seq<DT, 128, 128>(pl, q, grid, s);
            else launch_seq<DT, 64, 128>(pl, q, grid, s);
            break;
        }
        case Kern::SKINNY:
            if constexpr (DT != TVK_F32) {
                hipError_t e = launch_skinny(DT, q, pl.bk, pl.vec, s, fixed ? reinterpret_cast<float*>(ws) : nullptr);
                if (e != hipSuccess) return fail(e == hipErrorOutOfMemory ? TVK_ERR_OOM : TVK_ERR_DEVICE,
                                                  std::string("tvk_gemm: skinny launch failed: ") + hipGetErrorString(e));
            }
            break;
        case Kern::DMA256:
        case Kern::DMA128:
        case Kern::DMA128R8:
        case Kern::DMA128X256:
        case Kern::DMA256X128:
            if constexpr (DT != TVK_F32) {
                if (pl.split > 1) {
                    q.part = reinterpret_cast<float*>(ws + rep_a + rep_b);
                    q.split = pl.split;
                    q.k_chunk = pl.k_chunk;
                }
                const int tile = pl.kern == Kern::DMA256 ? 256 : pl.kern == Kern::DMA128X256 ? DMA_TILE_128X256
                                 : pl.kern == Kern::DMA256X128 ? DMA_TILE_256X128 : 128;
                hipError_t e = launch_dma(DT, q, pl.ak, pl.bk, tile, s, pl.kern == Kern::DMA128R8 ? 8 : 4);
                if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_gemm: launch failed: ") + hipGetErrorString(e));
                if (pl.split > 1) {
                    launch_split_reduce<DT>(q, s);
                }
            }
            break;
        case Kern::MFMA256:
        case Kern::MFMA256W8:
        case Kern::MFMA128:
        case Kern::MFMA64:
            if constexpr (DT != TVK_F32) {
                const int T = pl.kern == Kern::MFMA64 ? 64 : pl.kern == Kern::MFMA128 ? 128 : 256;
                q.tiles_m = (int)((d.M + T - 1) / T);
                q.tiles_n = (int)((d.N + T - 1) / T);
                dim3 grid(q.tiles_m * q.tiles_n, nb);
                if (pl.kern == Kern::MFMA256W8) launch_mfma<DT, 256, 256, 4>(pl, q, grid, s);
                else if (pl.kern == Kern::MFMA256) launch_mfma<DT, 256, 256, 2>(pl, q, grid, s);
                else if (pl.kern == Kern::MFMA64) launch_mfma<DT, 64, 64, 1>(pl, q, grid, s);
                else if (pl.split > 1) {
                    q.part = reinterpret_cast<float*>(ws + rep_a + rep_b);
                    q.split = pl.split;
                    q.k_chunk = pl.k_chunk;
                    grid.z = pl.split;
                    launch_mfma<DT, 128, 128, 2>(pl, q, grid, s);
                    launch_split_reduce<DT>(q, s);
                } else launch_mfma<DT, 128, 128, 2>(pl, q, grid, s);
            }
            break;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_gemm: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status validate(const tvk_gemm_desc* d) {
    if (!d) return fail(TVK_ERR_INVALID, "tvk_gemm: desc is NULL");
    if (d->dtype != TVK_F32 && d->dtype != TVK_F16 && d->dtype != TVK_BF16 && !gemm_wide_dtype(d->dtype))
        return fail(TVK_ERR_UNSUPPORTED, "tvk_gemm: unsupported dtype " + std::to_string(d->dtype));
    if ((d->flags & ~TVK_GEMM_EXACT) != 0 || d->reserved != 0)
        return fail(TVK_ERR_INVALID, "tvk_gemm: unknown flags or nonzero reserved field");
    if (d->activation < TVK_ACT_NONE || d->activation > TVK_ACT_GELU)
        return fail(TVK_ERR_INVALID, "tvk_gemm: invalid activation " + std::to_string(d->activation));
    if (d->batch < 0 || d->M < 0 || d->N < 0 || d->K < 0) return fail(TVK_ERR_INVALID, "tvk_gemm: negative size");
    if (!fits_i32(d->M) || !fits_i32(d->N) || !fits_i32(d->K) || !fits_i32(d->batch))
        return fail(TVK_ERR_UNSUPPORTED, "tvk_gemm: a dimension exceeds 2^31-1");
    for (int i = 0; i < 3; ++i)
        if (d->a_stride[i] < 0 || d->b_stride[i] < 0 || d->c_stride[i] < 0 || d->bias_stride[i] < 0)
            return fail(TVK_ERR_UNSUPPORTED, "tvk_gemm: negative strides are not supported");
    if (d->batch_inner < 0 || (d->batch_inner > 1 && d->batch % d->batch_inner != 0))
        return fail(TVK_ERR_INVALID, "tvk_gemm: batch_inner must divide batch");
    if (d->batch_inner > 1 &&
        (d->a_stride_inner < 0 || d->b_stride_inner < 0 || d->c_stride_inner < 0 || d->bias_stride_inner < 0))
        return fail(TVK_ERR_UNSUPPORTED, "tvk_gemm: negative strides are not supported");
    if (d->batch == 0 || d->M == 0 || d->N == 0) return TVK_OK;
    if (!d->c) return fail(TVK_ERR_INVALID, "tvk_gemm: c is NULL");
    if (d->K > 0 && (!d->a || !d->b)) return fail(TVK_ERR_INVALID, "tvk_gemm: a or b is NULL");
    return TVK_OK;
}

// make_plan's choice unless the kernel-choice table holds another candidate
// for the product's shape class (Autotuner::select's lookup,
// src/vulkan/autotuner.cpp:56-84); a recorded kernel that does not apply to
// this product is ignored, as the reference ignores a stored config outside
// the current space (in_space, :20-29).
Plan choose_plan(const tvk_gemm_desc& d) {
    std::string id;
    if (d.K > 0 && tune_lookup("gemm", tune_key(d), id))
        for (const Plan& p : candidate_plans(d))
            if (plan_id(p) == id) return p;
    return make_plan(d);
}

tvk_status run_plan(const tvk_gemm_desc& d, const Plan& pl, char* fixed = nullptr, size_t fixed_cap = 0) {
    const hipStream_t s = resolve_stream(d.stream);
    switch (d.dtype) {
    case TVK_F32: return run<TVK_F32>(d, pl, s, fixed, fixed_cap);
    case TVK_F16: return run<TVK_F16>(d, pl, s, fixed, fixed_cap);
    default: return run<TVK_BF16>(d, pl, s, fixed, fixed_cap);
    }
}

// Times every candidate on the product and picks the fastest: one warm-up
// launch, then the median of five timed launches each (the reference takes
// the median of five spans per config, src/vulkan/autotuner.cpp:16-18,137-152,
// and times every config of a space this small, :11-12,194-198). A candidate
// that fails to launch is skipped. When c shares memory with an operand the
// timed launches write a scratch output instead, so no input changes.
tvk_status time_candidates(const tvk_gemm_desc& d, const std::vector<Plan>& cands, Plan& best) {
    const size_t es = dtype_size(d.dtype);
    const int64_t bh = d.batch_inner > 1 ? d.batch_inner : 1;
    auto extent = [&](const void* base, const int64_t* st, int64_t sh, int64_t rows, int64_t cols) {
        const char* lo = static_cast<const char*>(base);
        return std::make_pair(lo, lo + es * ((d.batch / bh - 1) * st[0] + (bh - 1) * sh + (rows - 1) * st[1] +
                                             (cols - 1) * st[2] + 1));
    };
    const auto c = extent(d.c, d.c_stride, d.c_stride_inner, d.M, d.N);
    auto overlaps = [&](std::pair<const char*, const char*> r) { return r.first < c.second && c.first < r.second; };
    bool alias = overlaps(extent(d.a, d.a_stride, d.a_stride_inner, d.M, d.K)) ||
                 overlaps(extent(d.b, d.b_stride, d.b_stride_inner, d.K, d.N));
    if (d.bias && d.beta != 0.0) alias = alias || overlaps(extent(d.bias, d.bias_stride, d.bias_stride_inner, d.M, d.N));
    tvk_gemm_desc t = d;
    void* scratch = nullptr;
    if (alias) {
        if (hipMalloc(&scratch, (size_t)(c.second - c.first)) != hipSuccess) {
            (void)hipGetLastError();
            return fail(TVK_ERR_OOM, "tvk_gemm_tune: no memory for a scratch output");
        }
        t.c = scratch;
    }
    const hipStream_t s = resolve_stream(d.stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        (void)hipGetLastError();
        if (e0) (void)hipEventDestroy(e0);
        if (scratch) (void)hipFree(scratch);
        return fail(TVK_ERR_DEVICE, "tvk_gemm_tune: hipEventCreate failed");
    }
    // The shader clock ramps up over the first milliseconds of work after an
    // idle spell, which would count against whichever candidate is timed
    // first: run the first one for about 2 ms (at most 200 launches) first.
    if (!cands.empty() && hipEventRecord(e0, s) == hipSuccess) {
        for (int i = 0; i < 200; ++i) {
            if (run_plan(t, cands[0]) != TVK_OK) break;
            float ms = 0.0f;
            if (i % 8 == 7 && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                               hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms > 2.0f))
                break;
        }
        (void)hipGetLastError();
    }
    float best_ms = INFINITY;
    for (const Plan& pl : cands) {
        float spans[5];
        bool ok = run_plan(t, pl) == TVK_OK;
        for (int i = 0; ok && i < 5; ++i)
            ok = hipEventRecord(e0, s) == hipSuccess && run_plan(t, pl) == TVK_OK && hipEventRecord(e1, s) == hipSuccess &&
                 hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&spans[i], e0, e1) == hipSuccess;
        if (!ok) {
            (void)hipGetLastError();
            continue;
        }
        std::nth_element(spans, spans + 2, spans + 5);
        if (spans[2] < best_ms) {
            best_ms = spans[2];
            best = pl;
        }
    }
    (void)hipStreamSynchronize(s);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (scratch) (void)hipFree(scratch);
    if (best_ms == INFINITY) return fail(TVK_ERR_DEVICE, "tvk_gemm_tune: no candidate kernel ran");
    return TVK_OK;
}

void put_name(char* name, size_t name_len, const std::string& n) {
    if (name && name_len) snprintf(name, name_len, "%s", n.c_str());
}

}  // namespace
}  // namespace tvk

using namespace tvk;

extern "C" tvk_status tvk_gemm_plan(const tvk_gemm_desc* desc, char* name, size_t name_len) {
    tvk_status st = validate(desc);
    if (st != TVK_OK) return st;
    if (!name || name_len == 0) return fail(TVK_ERR_INVALID, "tvk_gemm_plan: name buffer is empty");
    if (desc->batch == 0 || desc->M == 0 || desc->N == 0) {
        snprintf(name, name_len, "none");
        return TVK_OK;
    }
    if (gemm_wide_dtype(desc->dtype)) {
        snprintf(name, name_len, "%s", gemm_wide_name(desc->dtype));
        return TVK_OK;
    }
    // a product tvk_gemm runs in row/column blocks is named by its first block's kernel
    tvk_gemm_desc first = *desc;
    int64_t mc = first.M, nc = first.N;
    if (first.K > 0 && extent_chunks(first, mc, nc)) {
        first.M = mc;
        first.N = nc;
    }
    snprintf(name, name_len, "%s", choose_plan(first).name);
    return TVK_OK;
}

namespace tvk {
namespace {

// tvk_gemm's body: the product, in row/column blocks when an operand spans
// 2 GiB. `plan_of` picks each block's kernel; `fixed` as for run().
template <class PlanOf>
tvk_status gemm_blocks(const tvk_gemm_desc& d, PlanOf plan_of, char* fixed, size_t fixed_cap) {
    tvk_status st = TVK_OK;
    int64_t mc = d.M, nc = d.N;
    if (d.K > 0 && extent_chunks(d, mc, nc) && (mc < d.M || nc < d.N)) {
        // row and column blocks whose operand extents fit the tiled kernels'
        // 32-bit buffer offsets, each its own product
        const size_t es = dtype_size(d.dtype);
        for (int64_t m0 = 0; m0 < d.M; m0 += mc)
            for (int64_t n0 = 0; n0 < d.N; n0 += nc) {
                tvk_gemm_desc sub = d;
                sub.M = std::min(mc, d.M - m0);
                sub.N = std::min(nc, d.N - n0);
                sub.a = static_cast<const char*>(d.a) + (size_t)(m0 * d.a_stride[1]) * es;
                sub.b = static_cast<const char*>(d.b) + (size_t)(n0 * d.b_stride[2]) * es;
                sub.c = static_cast<char*>(d.c) + (size_t)(m0 * d.c_stride[1] + n0 * d.c_stride[2]) * es;
                if (d.bias) sub.bias = static_cast<const char*>(d.bias) + (size_t)(m0 * d.bias_stride[1] + n0 * d.bias_stride[2]) * es;
                st = run_plan(sub, plan_of(sub), fixed, fixed_cap);
                if (st != TVK_OK) return st;
            }
        return TVK_OK;
    }
    return run_plan(d, plan_of(d), fixed, fixed_cap);
}

// Scratch of the allocation-free entry point: one array per device, in the
// code object (the runtime places it when the library's module loads on a
// device and keeps it until the process ends). Host code must not pass the
// array's name to a kernel: that is a host-side stand-in, not the device
// address. Each device's address comes from hipGetSymbolAddress, once per
// device, with that device current.
constexpr size_t kNoAllocScratch = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

constexpr int kMaxScratchDevices = 64;
std::once_flag g_scratch_once[kMaxScratchDevices];
char* g_scratch_ptr[kMaxScratchDevices] = {};
hipError_t g_scratch_err[kMaxScratchDevices] = {};

// The current device's address of `scratch` (NULL with *err set on failure).
char* noalloc_scratch(int dev, hipError_t* err) {
    std::call_once(g_scratch_once[dev], [dev]() {
        void* ptr = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (g_scratch_err[dev] == hipSuccess) g_scratch_ptr[dev] = static_cast<char*>(ptr);
        else (void)hipGetLastError();
    });
    *err = g_scratch_err[dev];
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace tvk

extern "C" tvk_status tvk_gemm(const tvk_gemm_desc* desc) {
    tvk_status st = validate(desc);
    if (st != TVK_OK) return st;
    const tvk_gemm_desc& d = *desc;
    if (d.batch == 0 || d.M == 0 || d.N == 0) return TVK_OK;
    if (gemm_wide_dtype(d.dtype)) return gemm_wide_run(d);
    return gemm_blocks(d, [](const tvk_gemm_desc& x) { return choose_plan(x); }, nullptr, 0);
}

extern "C" tvk_status tvk_gemm_noalloc(const tvk_gemm_desc* desc) {
    tvk_status st = validate(desc);
    if (st != TVK_OK) return st;
    const tvk_gemm_desc& d = *desc;
    if (d.batch == 0 || d.M == 0 || d.N == 0) return TVK_OK;
    if (gemm_wide_dtype(d.dtype)) return gemm_wide_run(d);   // no scratch
    // every block's scratch must fit the array before anything is queued
    int64_t mc = d.M, nc = d.N;
    tvk_gemm_desc first = d;
    if (d.K > 0 && extent_chunks(d, mc, nc)) {
        first.M = mc;
        first.N = nc;
    }
    const int nb = (int)std::min<int64_t>(65535, d.batch);
    const size_t need = plan_scratch_bytes(first, make_plan(first), nb);
    if (need > kNoAllocScratch)
        return fail(TVK_ERR_INVALID, "tvk_gemm_noalloc: this product needs " + std::to_string(need) +
                                         " bytes of scratch (split-K partials or repacked operands), more than the " +
                                         std::to_string(kNoAllocScratch) + " the entry point holds; use tvk_gemm");
    int dev = 0;
    TVK_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDevices) return fail(TVK_ERR_INVALID, "tvk_gemm_noalloc: device index out of range");
    hipError_t err = hipSuccess;
    char* ws = noalloc_scratch(dev, &err);
    if (!ws) return fail(TVK_ERR_DEVICE, std::string("tvk_gemm_noalloc: hipGetSymbolAddress failed: ") + hipGetErrorString(err));
    return gemm_blocks(d, [](const tvk_gemm_desc& x) { return make_plan(x); }, ws, kNoAllocScratch);
}

extern "C" tvk_status tvk_gemm_candidates(const tvk_gemm_desc* desc, char* names, size_t names_len) {
    tvk_status st = validate(desc);
    if (st != TVK_OK) return st;
    if (!names || names_len == 0) return fail(TVK_ERR_INVALID, "tvk_gemm_candidates: name buffer is empty");
    std::string all;
    if (desc->batch == 0 || desc->M == 0 || desc->N == 0) all = "none";
    else if (gemm_wide_dtype(desc->dtype)) all = gemm_wide_name(desc->dtype);
    else
        for (const Plan& p : candidate_plans(*desc)) all += (all.empty() ? "" : "\n") + plan_id(p);
    if (all.size() + 1 > names_len)
        return fail(TVK_ERR_INVALID, "tvk_gemm_candidates: the names need " + std::to_string(all.size() + 1) + " bytes");
    snprintf(names, names_len, "%s", all.c_str());
    return TVK_OK;
}

extern "C" tvk_status tvk_gemm_choose(const tvk_gemm_desc* desc, const char* kernel, int persist) {
    tvk_status st = validate(desc);
    if (st != TVK_OK) return st;
    if (!kernel) return fail(TVK_ERR_INVALID, "tvk_gemm_choose: kernel is NULL");
    if (desc->batch == 0 || desc->M == 0 || desc->N == 0 || desc->K == 0)
        return fail(TVK_ERR_INVALID, "tvk_gemm_choose: an empty product has no kernel choice");
    if (gemm_wide_dtype(desc->dtype)) {
        // one kernel: nothing to record
        if (std::string(kernel) == gemm_wide_name(desc->dtype)) return TVK_OK;
        return fail(TVK_ERR_INVALID, std::string("tvk_gemm_choose: ") + kernel + " does not compute this product");
    }
    for (const Plan& p : candidate_plans(*desc))
        if (plan_id(p) == kernel) {
            tune_record("gemm", tune_key(*desc), plan_id(p), persist != 0);
            return TVK_OK;
        }
    return fail(TVK_ERR_INVALID, std::string("tvk_gemm_choose: ") + kernel + " does not compute this product");
}

extern "C" tvk_status tvk_gemm_tune(const tvk_gemm_desc* desc, char* name, size_t name_len) {
    tvk_status st = validate(desc);
    if (st != TVK_OK) return st;
    const tvk_gemm_desc& d = *desc;
    if (d.batch == 0 || d.M == 0 || d.N == 0) {
        put_name(name, name_len, "none");
        return TVK_OK;
    }
    if (gemm_wide_dtype(d.dtype)) {
        put_name(name, name_len, gemm_wide_name(d.dtype));
        return gemm_wide_run(d);
    }
    const std::vector<Plan> cands = candidate_plans(d);
    Plan best = cands[0];
    if (d.K > 0) {
        const uint64_t key = tune_key(d);
        std::string id;
        bool known = false;
        if (tune_lookup("gemm", key, id))
            for (const Plan& p : cands)
                if (plan_id(p) == id) {
                    best = p;
                    known = true;
                    break;
                }
        if (!known) {
            if (cands.size() > 1) {
                st = time_candidates(d, cands, best);
                if (st != TVK_OK) return st;
            }
            tune_record("gemm", key, plan_id(best), true);
        }
    }
    put_name(name, name_len, plan_id(best));
    return run_plan(d, best);
}

extern "C" tvk_status tvk_tune_reset(void) {
    tune_reset();
    return TVK_OK;
}

extern "C" tvk_status tvk_tune_path(char* path, size_t path_len) {
    if (!path || path_len == 0) return fail(TVK_ERR_INVALID, "tvk_tune_path: buffer is empty");
    const std::string p = tune_path();
    if (p.size() + 1 > path_len) return fail(TVK_ERR_INVALID, "tvk_tune_path: the path needs " + std::to_string(p.size() + 1) + " bytes");
    snprintf(path, path_len, "%s", p.c_str());
    return TVK_OK;
}
