// Pieces shared by the GEMM translation units: kernel arguments, the fused
// epilogue and buffer-resource loads with hardware range checking.
#pragma once

#include "tvk_common.h"

namespace tvk {

struct GemmArgs {
    const void* a;
    const void* b;
    const void* bias;
    void* c;
    int64_t sa[3], sb[3], sbias[3], sc[3];
    int M, N, K;
    int batch;
    float alpha, beta;
    int has_bias;
    int act;
    int tiles_m, tiles_n;
    // split-K (split > 1): blockIdx.z takes k in [z*k_chunk, (z+1)*k_chunk) and
    // writes float32 partials to part[z][batch][M][N]; a second kernel sums
    // them in z order and applies the epilogue
    float* part;
    int k_chunk;
    int split;
    // 1: loads of k in [K, K rounded up to 32) return zeros for both operands
    // (a k-contiguous operand was copied with zero-padded rows; rows past K of
    // an m/n-contiguous one lie outside its buffer range), so the LDS-ring
    // kernels may run the last k step whole
    int kzero;
    // bytes of one matrix of a repacked operand (the whole zero-padded
    // [rows][ld] copy, which the LDS-ring kernels' buffer ranges then cover);
    // 0: the range ends at the operand's last element
    int64_t a_ext, b_ext;
    // split-K with the reduction in the same launch (split_fixup, the M <= 16
    // streaming kernel): one counter per output tile, zero before the launch
    // and left zero after it; NULL: the partials are summed by a second kernel
    unsigned* tile_count;
    // a second batch dimension (bh > 1): batch index b is (b / bh, b % bh),
    // addressed with stride [0] and the *_h stride (batch_off)
    int bh;
    int64_t sa_h, sb_h, sbias_h, sc_h;
};

// Element offset of batch b of an operand with outer stride s0 and inner
// stride sh (tvk_gemm_desc.batch_inner).
__host__ __device__ __forceinline__ int64_t batch_off(const GemmArgs& p, int b, int64_t s0, int64_t sh) {
    if (p.bh <= 1) return (int64_t)b * s0;
    const int bo = b / p.bh;
    return (int64_t)bo * s0 + (int64_t)(b - bo * p.bh) * sh;
}
__host__ __device__ __forceinline__ int64_t a_boff(const GemmArgs& p, int b) { return batch_off(p, b, p.sa[0], p.sa_h); }
__host__ __device__ __forceinline__ int64_t b_boff(const GemmArgs& p, int b) { return batch_off(p, b, p.sb[0], p.sb_h); }
__host__ __device__ __forceinline__ int64_t c_boff(const GemmArgs& p, int b) { return batch_off(p, b, p.sc[0], p.sc_h); }
__host__ __device__ __forceinline__ int64_t bias_boff(const GemmArgs& p, int b) { return batch_off(p, b, p.sbias[0], p.sbias_h); }

// ----------------------------------------------------------------------------
// epilogue (shared by all kernels)
// ----------------------------------------------------------------------------

__device__ inline float gelu_erf(float v) {
#pragma clang fp contract(off)
    return 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
}

// v = acc*alpha; v = v + bias*beta; act(v). Contraction is off so the two
// products round separately, as the reference's ext_mul/ext_add chain does.
// Out of line, with scalar arguments only: the tiled kernels call it from an
// unrolled epilogue and must keep their accumulators in registers.
static __device__ __noinline__ float epilogue_math(float acc, float alpha, int has_bias, float bv, float beta, int act) {
#pragma clang fp contract(off)
    float v = acc * alpha;
    if (has_bias) {
        float t = bv * beta;
        v = v + t;
    }
    if (act == TVK_ACT_RELU) v = v > 0.0f ? v : (v != v ? v : 0.0f);
    else if (act == TVK_ACT_GELU) v = gelu_erf(v);
    return v;
}

// The same arithmetic inline for every activation but GELU (a few VALU
// instructions, no call).
__device__ __forceinline__ float epilogue_linear(float acc, float alpha, int has_bias, float bv, float beta, int act) {
#pragma clang fp contract(off)
    float v = acc * alpha;
    if (has_bias) {
        float t = bv * beta;
        v = v + t;
    }
    if (act == TVK_ACT_RELU) v = v > 0.0f ? v : (v != v ? v : 0.0f);
    return v;
}

__device__ __forceinline__ float epilogue(float acc, float alpha, int has_bias, float bv, float beta, int act) {
    return act == TVK_ACT_GELU ? epilogue_math(acc, alpha, has_bias, bv, beta, act)
                               : epilogue_linear(acc, alpha, has_bias, bv, beta, act);
}

// INL: the arithmetic inline except for GELU, and a row-broadcast bias loaded
// once per fragment (store_frag16); the 256-wide tiles take neither, their
// accumulators fill the register file.
template <int DT, bool INL = false>
__device__ inline void store_out(const GemmArgs& p, int b, int row, int col, float acc) {
    typedef typename elem<DT>::T T;
    T* c = reinterpret_cast<T*>(p.c);
    float v;
    if (!p.has_bias && p.act == TVK_ACT_NONE) {
#pragma clang fp contract(off)
        v = acc * p.alpha;
    } else {
        float bv = 0.0f;
        if (p.has_bias) {
            const T* bias = reinterpret_cast<const T*>(p.bias);
            bv = elem<DT>::to_f32(bias[bias_boff(p, b) + (int64_t)row * p.sbias[1] + (int64_t)col * p.sbias[2]]);
        }
        v = INL ? epilogue(acc, p.alpha, p.has_bias, bv, p.beta, p.act) : epilogue_math(acc, p.alpha, p.has_bias, bv, p.beta, p.act);
    }
    c[c_boff(p, b) + (int64_t)row * p.sc[1] + (int64_t)col * p.sc[2]] = elem<DT>::from_f32(v);
}

// Epilogue of 16 accumulators of one lane that share a column and sit at
// rows row0 + (r/4)*8 + r%4 (the 32x32 MFMA accumulator layout). A bias that
// is constant along the rows (a Linear layer's, broadcast with row stride 0)
// is loaded once: loaded per element, each load would sit after a store to c
// (which may be the bias itself) and be waited for on its own.
template <int DT, bool INL = false>
__device__ inline void store_frag16(const GemmArgs& p, int b, int row0, int col, const f32x16& v) {
    if (col >= p.N) return;
    if (!p.has_bias && p.act == TVK_ACT_NONE) {
        // no bias, no activation: each element is its sum times alpha, as in
        // store_out, with the batch offset computed once for the 16 elements
        // (per element it cost a scalar division sequence where bh > 1)
        typedef typename elem<DT>::T T;
        T* c = reinterpret_cast<T*>(p.c) + c_boff(p, b) + (int64_t)col * p.sc[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + (r / 4) * 8 + (r % 4);
            if (row < p.M) {
#pragma clang fp contract(off)
                const float o = v[r] * p.alpha;
                c[(int64_t)row * p.sc[1]] = elem<DT>::from_f32(o);
            }
        }
        return;
    }
    if (INL && p.has_bias && p.sbias[1] == 0) {
        typedef typename elem<DT>::T T;
        const float bv = elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[bias_boff(p, b) + (int64_t)col * p.sbias[2]]);
        T* c = reinterpret_cast<T*>(p.c) + c_boff(p, b) + (int64_t)col * p.sc[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + (r / 4) * 8 + (r % 4);
            if (row < p.M)
                c[(int64_t)row * p.sc[1]] = elem<DT>::from_f32(INL ? epilogue(v[r], p.alpha, 1, bv, p.beta, p.act)
                                                                   : epilogue_math(v[r], p.alpha, 1, bv, p.beta, p.act));
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = row0 + (r / 4) * 8 + (r % 4);
        if (row < p.M) store_out<DT, INL>(p, b, row, col, v[r]);
    }
}


// Maps a block index to its (tile_m, tile_n) so that the blocks one XCD runs
// at a time cover a compact patch of C: blocks are dealt to the 8 XCDs round
// robin, so consecutive ids on one XCD are made consecutive in a grouped
// (GROUP_M rows at a time) column-major walk over the tiles.
__device__ inline void tile_of(int bid, int nblocks, int tiles_m, int tiles_n, int& tm, int& tn) {
    int lid = bid;
    if (nblocks % 8 == 0) lid = (bid % 8) * (nblocks / 8) + bid / 8;
    const int GM = 8;
    int per_group = GM * tiles_n;
    int g = lid / per_group;
    int first_m = g * GM;
    int gm = min(tiles_m - first_m, GM);
    int in = lid % per_group;
    tm = first_m + in % gm;
    tn = in / gm;
}

// Finishes four consecutive outputs (row, col .. col + 3) of matrix b from
// their float32 sums: the epilogue, one rounding to the output type, and one
// 8-byte store where the output rows are contiguous and 8-byte aligned (vec).
template <int DT>
__device__ __forceinline__ void finish4(const GemmArgs& p, int b, int row, int col, f32x4 v, bool vec) {
    typedef typename elem<DT>::T T;
    T* c = reinterpret_cast<T*>(p.c);
    // the bias row's address once for the four outputs
    const T* bp = p.has_bias ? reinterpret_cast<const T*>(p.bias) + bias_boff(p, b) + (int64_t)row * p.sbias[1] + (int64_t)col * p.sbias[2]
                             : nullptr;
    uint16_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float bv = 0.0f;
        if (p.has_bias) bv = elem<DT>::to_f32(bp[(int64_t)r * p.sbias[2]]);
        h[r] = __builtin_bit_cast(uint16_t, elem<DT>::from_f32(epilogue(v[r], p.alpha, p.has_bias, bv, p.beta, p.act)));
    }
    T* cp = c + c_boff(p, b) + (int64_t)row * p.sc[1] + (int64_t)col * p.sc[2];
    if (vec) {
        st_nt(reinterpret_cast<u32x2*>(cp), u32x2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)});
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) cp[(int64_t)r * p.sc[2]] = __builtin_bit_cast(T, h[r]);
    }
}

// Whether finish4 may store four outputs as one 8-byte write.
__device__ __forceinline__ bool finish4_vec(const GemmArgs& p) {
    return p.sc[2] == 1 && p.sc[1] % 4 == 0 && (p.batch == 1 || (p.sc[0] % 4 == 0 && (p.bh <= 1 || p.sc_h % 4 == 0))) &&
           (reinterpret_cast<uintptr_t>(p.c) & 7) == 0;
}

// Split-K without a second launch. The float32 partial planes of such a
// launch are written through to memory and read back coherently, without a
// fence: the L2 of each XCD is private, and a device-scope fence would write
// back and invalidate whole L2s under every other workgroup's loads.
// The cache-policy operand's SC1:SC0 bits select the scope of a vector memory
// instruction on gfx942/gfx950 (AMD CDNA3 ISA reference, "Memory Scope and
// Temporal Controls": 0 wave, 1 workgroup, 2 device, 3 system). At system
// scope a store writes through the L2 to memory and a load is coherent at
// that scope, so it cannot return a line another XCD's L2 held from before
// the write; the LLVM AMDGPU memory model for GFX942 (AMDGPUUsage, "Memory
// Model GFX942") emits the same sc0=1 sc1=1 bits for system-scope atomic
// loads and stores. tests/test_split_fixup_gpu.py alternates these launches
// with a two-launch split-K whose reduction reads the same pool buffer with
// ordinary cached loads. Buffer offsets are 32-bit: the host keeps the
// partials under 2 GiB.
constexpr int kCoherent = 1 | 16;   // sc0 | sc1: system scope

__device__ inline __amdgpu_buffer_rsrc_t part_rsrc(const GemmArgs& p) {
    const int64_t bytes = (int64_t)p.split * p.batch * p.M * p.N * 4;
    return __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, (int)bytes, 0x00020000);
}

__device__ inline void part_store(__amdgpu_buffer_rsrc_t r, int64_t idx, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)(idx * 4), 0, kCoherent);
}

// Each workgroup of an output tile has stored its plane with part_store; it
// waits for its stores and counts itself in on the tile's counter `cnt`
// (a system-scope atomic, performed in memory). The workgroup that brings
// the count to `split` resets the counter for the next launch and sums the
// tile's planes in split order with the additions and rounding of
// gemm_split_reduce4_kernel, so both paths give the same bits. No workgroup
// waits on another. Tile: rows m0 .. m0 + BM - 1, columns n0 .. n0 + BN - 1
// of matrix b (N % 4 == 0: 16-byte partial rows). `flag`: one word of LDS
// that no wave reads, nor loads into, any more.
template <int DT, int NT, int BM, int BN>
__device__ void split_fixup(const GemmArgs& p, int b, int m0, int n0, unsigned* cnt, int* flag) {
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's plane stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned old = atomicAdd_system(cnt, 1u);
        const int last = old + 1 == (unsigned)p.split;
        if (last) atomicExch_system(cnt, 0u);
        *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    const __amdgpu_buffer_rsrc_t r = part_rsrc(p);
    const int64_t mn = (int64_t)p.M * p.N, total = (int64_t)p.batch * mn;
    auto ld = [&](int64_t idx) {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(idx * 4), 0, kCoherent));
    };
    const bool vec = finish4_vec(p);
    constexpr int G4 = BN / 4;
    for (int g = threadIdx.x; g < BM * G4; g += NT) {
        const int row = m0 + g / G4, col = n0 + (g % G4) * 4;
        if (row >= p.M || col >= p.N) continue;
        const int64_t e = (int64_t)b * mn + (int64_t)row * p.N + col;
        f32x4 v = ld(e);
        // four planes' loads in flight before their adds (still in split order)
        int z = 1;
        for (; z + 3 < p.split; z += 4) {
#pragma clang fp contract(off)
            f32x4 w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) w[u] = ld((int64_t)(z + u) * total + e);
#pragma unroll
            for (int u = 0; u < 4; ++u) v = f32x4{v[0] + w[u][0], v[1] + w[u][1], v[2] + w[u][2], v[3] + w[u][3]};
        }
        {
#pragma clang fp contract(off)
            f32x4 w[3];
            const int rem = p.split - z;
#pragma unroll
            for (int u = 0; u < 3; ++u)
                if (u < rem) w[u] = ld((int64_t)(z + u) * total + e);
#pragma unroll
            for (int u = 0; u < 3; ++u)
                if (u < rem) v = f32x4{v[0] + w[u][0], v[1] + w[u][1], v[2] + w[u][2], v[3] + w[u][3]};
        }
        finish4<DT>(p, b, row, col, v, vec);
    }
}

namespace {
// Sums the split-K partials of one output in split order, then applies the
// epilogue and rounds once to the output type.
template <int DT>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(GemmArgs p) {
    const int64_t mn = (int64_t)p.M * p.N;
    const int64_t total = (int64_t)p.batch * mn;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
        const int b = (int)(idx / mn);
        const int64_t e = idx - (int64_t)b * mn;
        float v = p.part[idx];
        // eight planes' loads in flight before their adds (still in split order)
        int z = 1;
        for (; z + 7 < p.split; z += 8) {
            float w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = p.part[(int64_t)(z + u) * total + idx];
#pragma unroll
            for (int u = 0; u < 8; ++u) v += w[u];
        }
        {
            // the last planes (fewer than eight): every load issued before the first add
            float w[7];
            const int rem = p.split - z;
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (u < rem) w[u] = p.part[(int64_t)(z + u) * total + idx];
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (u < rem) v += w[u];
        }
        store_out<DT>(p, b, (int)(e / p.N), (int)(e % p.N), v);
    }
}

// The same sum, four consecutive outputs of one row a thread (N % 4 == 0, so
// a group never straddles two rows): 16-byte loads from each partial plane,
// added in split order, the epilogue inline, and one 8-byte store where the
// output rows are contiguous and 8-byte aligned (VEC).
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void gemm_split_reduce4_kernel(GemmArgs p) {
    const int64_t mn = (int64_t)p.M * p.N;
    const int64_t total = (int64_t)p.batch * mn;
    const int64_t groups = total / 4;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < groups; q += (int64_t)gridDim.x * 256) {
        const int64_t idx = q * 4;
        f32x4 v = *reinterpret_cast<const f32x4*>(p.part + idx);
        // eight planes' loads in flight before their adds (still in split order)
        int z = 1;
        for (; z + 7 < p.split; z += 8) {
#pragma clang fp contract(off)
            f32x4 w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const f32x4*>(p.part + (int64_t)(z + u) * total + idx);
#pragma unroll
            for (int u = 0; u < 8; ++u) v = f32x4{v[0] + w[u][0], v[1] + w[u][1], v[2] + w[u][2], v[3] + w[u][3]};
        }
        {
            // the last planes (fewer than eight): every load issued before the first add
#pragma clang fp contract(off)
            f32x4 w[7];
            const int rem = p.split - z;
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (u < rem) w[u] = *reinterpret_cast<const f32x4*>(p.part + (int64_t)(z + u) * total + idx);
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (u < rem) v = f32x4{v[0] + w[u][0], v[1] + w[u][1], v[2] + w[u][2], v[3] + w[u][3]};
        }
        const int b = (int)(idx / mn);
        const int64_t e = idx - (int64_t)b * mn;
        const int row = (int)(e / p.N), col = (int)(e - (int64_t)row * p.N);
        finish4<DT>(p, b, row, col, v, VEC);
    }
}

}  // namespace

// The split-K reduction for a float16/bfloat16 output: the four-wide kernel
// where N is a multiple of 4 and the output fills at least 256 of its
// workgroups or there are 8 or more partial planes (smaller outputs of few
// planes, such as the M <= 16 products', keep more workgroups with one output
// a thread: measured 0.2 us faster there).
template <int DT>
inline void launch_split_reduce(const GemmArgs& q, hipStream_t s) {
    const int64_t total = (int64_t)q.batch * q.M * q.N;
    if (q.N % 4 == 0 && (total >= 4 * 256 * 256 || q.split >= 8)) {
        const bool vec = q.sc[2] == 1 && q.sc[1] % 4 == 0 && (q.batch == 1 || (q.sc[0] % 4 == 0 && (q.bh <= 1 || q.sc_h % 4 == 0))) &&
                         (reinterpret_cast<uintptr_t>(q.c) & 7) == 0;
        const unsigned blocks = (unsigned)std::min<int64_t>((total / 4 + 255) / 256, 8192);
        if (vec) hipLaunchKernelGGL((gemm_split_reduce4_kernel<DT, true>), dim3(blocks), dim3(256), 0, s, q);
        else hipLaunchKernelGGL((gemm_split_reduce4_kernel<DT, false>), dim3(blocks), dim3(256), 0, s, q);
        return;
    }
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(gemm_split_reduce_kernel<DT>, dim3(blocks), dim3(256), 0, s, q);
}

// Out-of-range buffer offset: the hardware returns zeros for it.
constexpr uint32_t kOOB = 0x80000000u;

__device__ inline u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ inline uint32_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// Eight consecutive elements of one operand along its contiguous dimension.
// VEC: one 16-byte load (alignment and extent are multiples of 8 elements);
// otherwise eight 2-byte loads, each range-checked.
template <bool VEC>
__device__ inline u32x4 load_chunk(__amdgpu_buffer_rsrc_t r, bool row_ok, int64_t elem_off, int64_t step, int valid) {
    if constexpr (VEC) {
        return buf_load16(r, (row_ok && valid > 0) ? (uint32_t)(elem_off * 2) : kOOB);
    } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            h[e] = buf_load2(r, (row_ok && e < valid) ? (uint32_t)((elem_off + e * step) * 2) : kOOB);
        u32x4 v;
        v.x = h[0] | (h[1] << 16);
        v.y = h[2] | (h[3] << 16);
        v.z = h[4] | (h[5] << 16);
        v.w = h[6] | (h[7] << 16);
        return v;
    }
}


// Tile kernel with operands fetched straight into LDS (gemm_dma.hip).
// dma_applies: the operands meet its alignment and K granularity; launch_dma
// returns hipSuccess or the launch error.
bool dma_applies(const GemmArgs& p, bool a_kmajor, bool b_kmajor);
// tile: 256 (256x256), 128 (128x128), DMA_TILE_128X256 or DMA_TILE_256X128
constexpr int DMA_TILE_128X256 = 1, DMA_TILE_256X128 = 2;
hipError_t launch_dma(int dtype, GemmArgs& p, bool a_kmajor, bool b_kmajor, int tile, hipStream_t s, int stages = 4);

// Channels-last convolution on the LDS ring (conv_nhwc.hip); mode 0 forward,
// 1 grad input, 2 grad weight.
bool conv_ring_applies(const tvk_conv_desc& d, int mode);
tvk_status conv_ring_run(const tvk_conv_desc& d, int mode, const char* who);
// Stride-1 3x3 padding-1 forward / grad input from NCHW through an LDS halo
// (conv_nhwc.hip); mode 0 or 1.
bool conv_halo_applies(const tvk_conv_desc& d, int mode);
tvk_status conv_halo_run(const tvk_conv_desc& d, int mode, const char* who);
// Few input channels (conv_stem.hip): cin * kh * kw <= 32; same modes.
bool conv_small_applies(const tvk_conv_desc& d, int mode);
tvk_status conv_small_run(const tvk_conv_desc& d, int mode, const char* who);

// float64 and integer products (gemm_wide.hip): one kernel, any strides, no
// scratch; the dtype's own accumulate type, float64 in k order.
bool gemm_wide_dtype(int dtype);
const char* gemm_wide_name(int dtype);
tvk_status gemm_wide_run(const tvk_gemm_desc& d);

// M <= 16 streaming kernel (gemm_skinny.hip). b_kmajor: B's k stride is 1.
// vec: 16-byte loads are legal for A and B. `part`: skinny_scratch_bytes of
// caller-provided scratch for split-K partials, or NULL to lease them from the
// library's pool. Returns hipSuccess or the launch error.
hipError_t launch_skinny(int dtype, const GemmArgs& p, bool b_kmajor, bool vec, hipStream_t s, float* part = nullptr);
// Scratch bytes launch_skinny needs for this product (0: none).
size_t skinny_scratch_bytes(const GemmArgs& p, bool b_kmajor, bool vec);
const char* skinny_name(const GemmArgs& p, bool b_kmajor, bool vec);
bool skinny_applies(int64_t M, int64_t N, int64_t K, int64_t batch);

}  // namespace tvk
