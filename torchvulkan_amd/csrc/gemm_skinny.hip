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
// B n-contiguous with 16-byte aligned rows ([K][N], the C5 layout) takes a
// second kernel, gemm16_skinny_ring: workgroups of 8 waves own 128 columns
// (256 bytes of each row of B) and a K range; B and A arrive by buffer loads
// straight into a 4-stage LDS ring (no register staging), each wave reads its
// 16 columns back along k with ds_read_b64_tr_b16 and issues one
// v_mfma_f32_16x16x32 per 32 k. The K range is split between workgroups
// until about one workgroup per CU runs; float32 partials are then summed in
// split order by a second kernel that applies the epilogue.
//
// Epilogue semantics are the reference's (src/shaders/helpers/gemm_simd.slang:67-99).
#include "gemm_common.h"

#include <algorithm>

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

    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a) + a_boff(p, b);
    const uint16_t* B = reinterpret_cast<const uint16_t*>(p.b) + b_boff(p, b);
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
        if (m < p.M && n < p.N) store_out<DT, true>(p, b, m, n, v);
    }
}


// ---------------------------------------------------------------------------
// gemm16_skinny_ring
// ---------------------------------------------------------------------------

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
#define TVK_LDS __attribute__((address_space(3)))

constexpr int SR_NB = 128;                 // columns per workgroup
constexpr int SR_NW = 8;                   // waves, 16 columns each
constexpr int SR_NS = 4;                   // ring stages of 32 k
constexpr int SR_ROW = SR_NB * 2;          // bytes of one k-row of the B tile
constexpr int SR_BST = 32 * SR_ROW;        // B bytes per stage: 8 loads of 1 KB, one per wave
constexpr int SR_STB = SR_BST + 1024;      // + A: 16 rows x 32 k, one load (wave 0)

__device__ inline i32x4 sr_rsrc(const void* ptr, int64_t bytes) {
    const uint64_t a = (uint64_t)ptr;
    return i32x4{(int)(uint32_t)a, (int)((a >> 32) & 0xffff), (int)min(bytes, (int64_t)0x7fffffff), 0x00020000};
}

// 16 bytes per lane into LDS at lds_addr + 16 * lane (lds_addr wave-uniform,
// carried in M0). Issued from asm so the compiler does not order every later
// LDS read behind it; the waits are explicit.
__device__ inline void sr_dma16(i32x4 r, uint32_t lds_addr, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voff), "s"(r) : "memory");
}
template <int N>
__device__ inline void sr_wait() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }

__device__ inline int sr_swz(int kr) { return (kr & 3) * 2; }

// grid (strips, splits, batch); requires A k-contiguous, B n-contiguous, rows
// of both 16-byte aligned, N % 8 == 0 and k_chunk % 32 == 0.
template <int DT>
__global__ __launch_bounds__(64 * SR_NW) void gemm_skinny_ring_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(1024))) char lds_raw[SR_NS * SR_STB];
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(TVK_LDS char*)lds_raw);
    const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int n0 = blockIdx.x * SR_NB, z = blockIdx.y, b = blockIdx.z;
    const int kb = p.split > 1 ? z * p.k_chunk : 0;
    const int klen = p.split > 1 ? p.k_chunk : p.K;
    const int nk = klen / 32;

    const char* A = reinterpret_cast<const char*>(p.a) + a_boff(p, b) * 2;
    const char* B = reinterpret_cast<const char*>(p.b) + b_boff(p, b) * 2;
    const i32x4 ra = sr_rsrc(A, 2 * ((int64_t)(p.M - 1) * p.sa[1] + p.K));
    const i32x4 rb = sr_rsrc(B, 2 * ((int64_t)(p.K - 1) * p.sb[1] + p.N));
    // wave w loads B block w (k-rows 4w..4w+3 of the stage); wave 0 also loads A
    const int kr = wave * 4 + lane / 16;
    const int bc = (lane % 16) ^ sr_swz(kr);
    const int gc = n0 + bc * 8;
    const uint32_t b_off = gc < p.N ? (uint32_t)(((int64_t)(kb + kr) * p.sb[1] + gc) * 2) : kOOB;
    const uint32_t b_step = (uint32_t)(32 * p.sb[1] * 2);
    const int ar = lane / 4;
    const uint32_t a_off = ar < p.M ? (uint32_t)(((int64_t)ar * p.sa[1] + kb + (lane % 4) * 8) * 2) : kOOB;
    auto issue = [&](int s) {
        if (s >= nk) return;
        const uint32_t slot = lds0 + (uint32_t)((s % SR_NS) * SR_STB);
        sr_dma16(rb, slot + (uint32_t)(wave * 1024), b_off + (uint32_t)s * b_step);
        if (wave == 0) sr_dma16(ra, slot + SR_BST, a_off + (uint32_t)s * 64);
    };

    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < SR_NS - 1; ++s) issue(s);
    // this wave's B fragment: 16 columns, lane s of group g gets k 8g..8g+7 of column s
    const int g = lane / 16, sl = lane % 16;
    const int col = wave * 16 + (sl % 4) * 4;
    const int chunk = col / 8, within = (col % 8) * 2;
    for (int kt = 0; kt < nk; ++kt) {
        // stage kt landed; the two stages issued after it may be in flight
        if (nk - 1 - kt >= SR_NS - 2) {
            if (wave == 0) sr_wait<2 * (SR_NS - 2)>();
            else sr_wait<SR_NS - 2>();
        } else {
            sr_wait<0>();
        }
        __syncthreads();
        issue(kt + SR_NS - 1);
        const uint32_t st = lds0 + (uint32_t)((kt % SR_NS) * SR_STB);
        const u32x4 af = *(const TVK_LDS u32x4*)(uintptr_t)(st + SR_BST + (lane % 16) * 64 + (lane / 16) * 16);
        u32x4 bf;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int r = g * 8 + rr * 4 + sl / 4;
            TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(st + r * SR_ROW + ((chunk ^ sr_swz(r)) * 16) + within);
            const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
            bf[rr * 2] = w.x;
            bf[rr * 2 + 1] = w.y;
        }
        acc = mfma16<DT>(af, bf, acc);
    }
    sr_wait<0>();

    // lane l holds column l % 16 of the wave's 16, rows (l / 16) * 4 + r
    const int n = n0 + wave * 16 + lane % 16;
    if (n < p.N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = (lane / 16) * 4 + r;
            if (m >= p.M) continue;
            const int64_t pi = (((int64_t)z * p.batch + b) * p.M + m) * p.N + n;
            if (p.split > 1 && p.tile_count) part_store(part_rsrc(p), pi, acc[r]);   // written through (split_fixup)
            else if (p.split > 1) p.part[pi] = acc[r];
            else store_out<DT, true>(p, b, m, n, acc[r]);
        }
    }
    // every wave has drained its loads into the ring: its first word serves
    // as the fixup's flag (the fixup's first barrier orders that)
    if (p.split > 1 && p.tile_count)
        split_fixup<DT, 64 * SR_NW, 16, SR_NB>(p, b, 0, n0, p.tile_count + (int64_t)b * gridDim.x + blockIdx.x,
                                               reinterpret_cast<int*>(lds_raw));
}

// Splits of K for the ring kernel: powers of two while the grid stays within
// about one workgroup per CU and every split keeps at least 4 stages.
int ring_splits(const GemmArgs& p) {
    const int64_t wgs = (int64_t)((p.N + SR_NB - 1) / SR_NB) * p.batch;
    int split = 1;
    while (wgs * split * 2 <= 256 && p.K % (64 * split) == 0 && p.K / (2 * split) >= 128) split *= 2;
    return split;
}

bool ring_applies(const GemmArgs& p, bool b_kmajor, bool vec) {
    if (b_kmajor || !vec) return false;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(p.a) || !al16(p.b) || p.sa[2] != 1 || p.sb[2] != 1) return false;
    if (p.K % 32 != 0 || p.N % 8 != 0 || (p.M > 1 && p.sa[1] % 8 != 0) || (p.K > 1 && p.sb[1] % 8 != 0)) return false;
    if (p.batch > 1 && (p.sa[0] % 8 != 0 || p.sb[0] % 8 != 0)) return false;
    if (p.bh > 1 && (p.sa_h % 8 != 0 || p.sb_h % 8 != 0)) return false;
    return true;
}
}  // namespace

bool skinny_applies(int64_t M, int64_t N, int64_t K, int64_t batch) {
    return M >= 1 && M <= 16 && N >= 64 && K >= 64 && batch <= 65535;
}

const char* skinny_name(const GemmArgs& p, bool b_kmajor, bool vec) {
    if (ring_applies(p, b_kmajor, vec)) return ring_splits(p) > 1 ? "gemm16_skinny_ring_splitk" : "gemm16_skinny_ring";
    return b_kmajor ? "gemm16_skinny_bk" : "gemm16_skinny_bn";
}

size_t skinny_scratch_bytes(const GemmArgs& p, bool b_kmajor, bool vec) {
    if (!ring_applies(p, b_kmajor, vec)) return 0;
    const int split = ring_splits(p);
    return split > 1 ? (size_t)split * p.batch * p.M * p.N * 4 : 0;
}

hipError_t launch_skinny(int dtype, const GemmArgs& p, bool b_kmajor, bool vec, hipStream_t s, float* part) {
    if (ring_applies(p, b_kmajor, vec)) {
        GemmArgs q = p;
        q.split = ring_splits(p);
        q.k_chunk = p.K / q.split;
        Scratch scratch;
        if (q.split > 1) {
            q.part = part ? part : static_cast<float*>(scratch.get((size_t)q.split * p.batch * p.M * p.N * 4, s));
            if (!q.part) return hipErrorOutOfMemory;
        }
        const dim3 grid((p.N + SR_NB - 1) / SR_NB, q.split, p.batch);
        // the reduction in the same launch, except on caller-provided scratch
        // (the allocation-free entry point keeps its second launch)
        if (q.split > 1 && !part && (int64_t)q.split * p.batch * p.M * p.N * 4 < (int64_t(1) << 31))
            q.tile_count = split_counters(s, (int64_t)grid.x * p.batch);
        if (dtype == TVK_F16) hipLaunchKernelGGL(gemm_skinny_ring_kernel<TVK_F16>, grid, dim3(64 * SR_NW), 0, s, q);
        else hipLaunchKernelGGL(gemm_skinny_ring_kernel<TVK_BF16>, grid, dim3(64 * SR_NW), 0, s, q);
        if (q.split > 1 && !q.tile_count) {
            if (dtype == TVK_F16) launch_split_reduce<TVK_F16>(q, s);
            else launch_split_reduce<TVK_BF16>(q, s);
        }
        return hipGetLastError();
    }
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
