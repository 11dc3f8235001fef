// Scaled dot-product attention for the shapes the MFMA kernels of
// attention.hip do not take: float32 as well as float16/bfloat16, any head
// dims up to 512 (query/key and value dims may differ), any element strides,
// and the gradient of the scores when the caller wants the bias gradient.
//
// Semantics are those of tvk_attention_fwd / tvk_attention_bwd (the
// reference's fused and chunked paths, src/api/ops/attention.cpp:115-199,
// 434-500): scores scale*q.k + bias in float32, causal mask j > i, rows with
// no unmasked key give out = 0 and lse = +inf; float16/bfloat16 stage the
// probabilities (and the score gradient) in the dtype before their products,
// as the cooperative-matrix kernels do (src/shaders/ops/attention_coop.slang).
//
// Layout: a workgroup of 256 threads owns 16 rows (queries in the forward and
// the query-gradient pass, keys in the key/value-gradient pass); 16 threads
// share a row, thread `lane` of a row takes columns lane, lane+16, ... of
// every 32-wide tile of the other side and output columns lane + 16*i. Both
// sides are staged through LDS in 64-column chunks of the head dimension as
// float32, so the dot products of any head dim are chunked sums; the running
// softmax of a row is reduced over its 16 threads with lane shuffles.
// Every output element has one writer (no atomics): the same bits each run.
#include "attention_any.h"

#include <algorithm>
#include <cmath>

namespace tvk {
namespace {

constexpr int AY_ROWS = 16;        // rows per workgroup
constexpr int AY_TILE = 32;        // columns of the other side per tile
constexpr int AY_DC = 64;          // head-dim chunk staged in LDS
constexpr int AY_LD = AY_DC + 1;   // padded LDS row (floats)
constexpr int AY_THREADS = 256;

template <int DT>
__device__ inline float ld(const void* base, int64_t off) {
    if constexpr (DT == TVK_F32) return static_cast<const float*>(base)[off];
    else if constexpr (DT == TVK_F16) return (float)static_cast<const _Float16*>(base)[off];
    else return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[off]);
}

template <int DT>
__device__ inline void st(void* base, int64_t off, float v) {
    if constexpr (DT == TVK_F32) static_cast<float*>(base)[off] = v;
    else if constexpr (DT == TVK_F16) static_cast<_Float16*>(base)[off] = (_Float16)v;
    else static_cast<uint16_t*>(base)[off] = f32_to_bf16_bits(v);
}

// A float32 value as the dtype would hold it (the staging of P and dS).
template <int DT>
__device__ inline float round_dt(float v) {
    if constexpr (DT == TVK_F32) return v;
    else if constexpr (DT == TVK_F16) return (float)(_Float16)v;
    else return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

__device__ inline float row_max16(float v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 16));
    return v;
}
__device__ inline float row_sum16(float v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, 16);
    return v;
}

// Stages rows [r0, r0+nrows) x columns [c0, c0+64) of a [rows][dim] view
// (row stride rs, unit or `cs` column stride) into lds[nrows][AY_LD] as
// float32; rows or columns past the end read 0.
template <int DT>
__device__ inline void stage(float* lds, int nrows, const void* base, int64_t rs, int64_t cs, int r0, int rows, int c0,
                             int dim) {
    for (int i = threadIdx.x; i < nrows * AY_DC; i += AY_THREADS) {
        const int r = i / AY_DC, c = i % AY_DC;
        float v = 0.0f;
        if (r0 + r < rows && c0 + c < dim) v = ld<DT>(base, (int64_t)(r0 + r) * rs + (int64_t)(c0 + c) * cs);
        lds[r * AY_LD + c] = v;
    }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------

template <int DT, int NV>
__global__ __launch_bounds__(AY_THREADS) void attn_any_fwd_kernel(AnyAttnArgs p) {
    __shared__ float qs[AY_ROWS * AY_LD];
    __shared__ float ks[AY_TILE * AY_LD];
    __shared__ float ps[AY_ROWS * (AY_TILE + 1)];
    const int r = threadIdx.x / 16, lane = threadIdx.x % 16;
    const int h = blockIdx.y, b = blockIdx.z, hk = h / p.group;
    const int q0 = blockIdx.x * AY_ROWS, qi = q0 + r;
    const char* qb = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * p.es;
    const char* kb = static_cast<const char*>(p.k) + (b * p.sk[0] + hk * p.sk[1]) * p.es;
    const char* vb = static_cast<const char*>(p.v) + (b * p.sv[0] + hk * p.sv[1]) * p.es;
    const char* bb = p.bias ? static_cast<const char*>(p.bias) + (b * p.sb[0] + h * p.sb[1]) * p.es : nullptr;

    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    // keys past the row's causal limit contribute nothing: the workgroup's
    // last query bounds the tiles it visits
    const int kend = p.causal ? std::min(p.S, q0 + AY_ROWS) : p.S;
    for (int k0 = 0; k0 < kend; k0 += AY_TILE) {
        float s0 = 0.0f, s1 = 0.0f;
        for (int c0 = 0; c0 < p.D; c0 += AY_DC) {
            __syncthreads();
            stage<DT>(qs, AY_ROWS, qb, p.sq[2], p.sq[3], q0, p.L, c0, p.D);
            stage<DT>(ks, AY_TILE, kb, p.sk[2], p.sk[3], k0, p.S, c0, p.D);
            __syncthreads();
            const int n = std::min(AY_DC, p.D - c0);
#pragma unroll 4
            for (int c = 0; c < n; ++c) {
                const float qv = qs[r * AY_LD + c];
                s0 = fmaf(qv, ks[lane * AY_LD + c], s0);
                s1 = fmaf(qv, ks[(lane + 16) * AY_LD + c], s1);
            }
        }
        float sc[2] = {s0, s1};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int kj = k0 + lane + 16 * j;
            float s = sc[j] * p.scale;
            if (bb && qi < p.L && kj < p.S) s += ld<DT>(bb, qi * p.sb[2] + kj * p.sb[3]);
            if (kj >= p.S || qi >= p.L || (p.causal && kj > qi)) s = -INFINITY;
            sc[j] = s;
        }
        const float m_new = fmaxf(m_run, row_max16(fmaxf(sc[0], sc[1])));
        const float base = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - base);
        const float p0 = sc[0] == -INFINITY ? 0.0f : expf(sc[0] - base);
        const float p1 = sc[1] == -INFINITY ? 0.0f : expf(sc[1] - base);
        m_run = m_new;
        l_run = l_run * alpha + p0 + p1;
#pragma unroll
        for (int i = 0; i < NV; ++i) acc[i] *= alpha;
        ps[r * (AY_TILE + 1) + lane] = round_dt<DT>(p0);
        ps[r * (AY_TILE + 1) + lane + 16] = round_dt<DT>(p1);
        // O += P V, V by 64-column chunks; a thread's columns of chunk ch are lane + 16*i
#pragma unroll
        for (int ch = 0; ch < NV / 4; ++ch) {
            if (ch * AY_DC >= p.Dv) break;
            __syncthreads();
            stage<DT>(ks, AY_TILE, vb, p.sv[2], p.sv[3], k0, p.S, ch * AY_DC, p.Dv);
            __syncthreads();
#pragma unroll 2
            for (int j = 0; j < AY_TILE; ++j) {
                const float pj = ps[r * (AY_TILE + 1) + j];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[ch * 4 + i] = fmaf(pj, ks[j * AY_LD + lane + 16 * i], acc[ch * 4 + i]);
            }
        }
    }
    const float l = row_sum16(l_run);
    if (qi >= p.L) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    char* ob = static_cast<char*>(p.out) + (b * p.so[0] + h * p.so[1] + qi * p.so[2]) * p.es;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (i / 4) * AY_DC + lane + 16 * (i % 4);
        if (c < p.Dv) st<DT>(ob, c * p.so[3], acc[i] * inv);
    }
    if (lane == 0) p.lse[b * p.sl[0] + h * p.sl[1] + qi * p.sl[2]] = l > 0.0f ? m_run + logf(l) : INFINITY;
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------

// delta[b, h, i] = sum_c dout[i, c] * out[i, c] (float32), one thread a row.
template <int DT>
__global__ __launch_bounds__(256) void attn_any_delta_kernel(AnyAttnArgs p) {
    const int64_t rows = (int64_t)p.B * p.Hq * p.L;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows) return;
    const int i = (int)(idx % p.L), h = (int)((idx / p.L) % p.Hq), b = (int)(idx / ((int64_t)p.L * p.Hq));
    const char* o = static_cast<const char*>(p.out) + (b * p.so[0] + h * p.so[1] + i * p.so[2]) * p.es;
    const char* g = static_cast<const char*>(p.dout) + (b * p.sdo[0] + h * p.sdo[1] + i * p.sdo[2]) * p.es;
    float s = 0.0f;
    for (int c = 0; c < p.Dv; ++c) s = fmaf(ld<DT>(g, c * p.sdo[3]), ld<DT>(o, c * p.so[3]), s);
    p.delta[idx] = s;
}

// P and dS of one (row, column) pair from the raw dot products.
struct PdS {
    float p, ds;
};

// dQ (and the score gradient): a workgroup owns 16 queries of one head.
template <int DT, int ND>
__global__ __launch_bounds__(AY_THREADS) void attn_any_dq_kernel(AnyAttnArgs p) {
    __shared__ float as_[AY_ROWS * AY_LD];   // q chunk, then dout chunk
    __shared__ float bs[AY_TILE * AY_LD];    // k chunk, v chunk, k chunk
    __shared__ float dss[AY_ROWS * (AY_TILE + 1)];
    const int r = threadIdx.x / 16, lane = threadIdx.x % 16;
    const int h = blockIdx.y, b = blockIdx.z, hk = h / p.group;
    const int q0 = blockIdx.x * AY_ROWS, qi = q0 + r;
    const char* qb = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * p.es;
    const char* kb = static_cast<const char*>(p.k) + (b * p.sk[0] + hk * p.sk[1]) * p.es;
    const char* vb = static_cast<const char*>(p.v) + (b * p.sv[0] + hk * p.sv[1]) * p.es;
    const char* gb = static_cast<const char*>(p.dout) + (b * p.sdo[0] + h * p.sdo[1]) * p.es;
    const char* bb = p.bias ? static_cast<const char*>(p.bias) + (b * p.sb[0] + h * p.sb[1]) * p.es : nullptr;
    const int64_t row = ((int64_t)b * p.Hq + h) * p.L + qi;
    const float lse = qi < p.L ? p.lse[b * p.sl[0] + h * p.sl[1] + qi * p.sl[2]] : INFINITY;
    const float delta = qi < p.L ? p.delta[row] : 0.0f;

    float acc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[i] = 0.0f;
    const int kend = p.causal ? std::min(p.S, q0 + AY_ROWS) : p.S;
    for (int k0 = 0; k0 < kend; k0 += AY_TILE) {
        float s0 = 0.0f, s1 = 0.0f, g0 = 0.0f, g1 = 0.0f;
        for (int c0 = 0; c0 < p.D; c0 += AY_DC) {
            __syncthreads();
            stage<DT>(as_, AY_ROWS, qb, p.sq[2], p.sq[3], q0, p.L, c0, p.D);
            stage<DT>(bs, AY_TILE, kb, p.sk[2], p.sk[3], k0, p.S, c0, p.D);
            __syncthreads();
            const int n = std::min(AY_DC, p.D - c0);
#pragma unroll 4
            for (int c = 0; c < n; ++c) {
                const float a = as_[r * AY_LD + c];
                s0 = fmaf(a, bs[lane * AY_LD + c], s0);
                s1 = fmaf(a, bs[(lane + 16) * AY_LD + c], s1);
            }
        }
        for (int c0 = 0; c0 < p.Dv; c0 += AY_DC) {
            __syncthreads();
            stage<DT>(as_, AY_ROWS, gb, p.sdo[2], p.sdo[3], q0, p.L, c0, p.Dv);
            stage<DT>(bs, AY_TILE, vb, p.sv[2], p.sv[3], k0, p.S, c0, p.Dv);
            __syncthreads();
            const int n = std::min(AY_DC, p.Dv - c0);
#pragma unroll 4
            for (int c = 0; c < n; ++c) {
                const float a = as_[r * AY_LD + c];
                g0 = fmaf(a, bs[lane * AY_LD + c], g0);
                g1 = fmaf(a, bs[(lane + 16) * AY_LD + c], g1);
            }
        }
        const float sc[2] = {s0, s1}, gc[2] = {g0, g1};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int kj = k0 + lane + 16 * j;
            float pj = 0.0f;
            if (qi < p.L && kj < p.S && !(p.causal && kj > qi) && lse != INFINITY) {
                float s = sc[j] * p.scale;
                if (bb) s += ld<DT>(bb, qi * p.sb[2] + kj * p.sb[3]);
                pj = expf(s - lse);
            }
            const float ds = pj * (gc[j] - delta);
            if (p.ds && qi < p.L && kj < p.S)
                p.ds[b * p.sds[0] + h * p.sds[1] + qi * p.sds[2] + (int64_t)kj * p.sds[3]] = ds;
            dss[r * (AY_TILE + 1) + lane + 16 * j] = round_dt<DT>(ds);
        }
        // dQ += dS K, K by 64-column chunks
#pragma unroll
        for (int ch = 0; ch < ND / 4; ++ch) {
            if (ch * AY_DC >= p.D) break;
            __syncthreads();
            stage<DT>(bs, AY_TILE, kb, p.sk[2], p.sk[3], k0, p.S, ch * AY_DC, p.D);
            __syncthreads();
#pragma unroll 2
            for (int j = 0; j < AY_TILE; ++j) {
                const float dj = dss[r * (AY_TILE + 1) + j];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[ch * 4 + i] = fmaf(dj, bs[j * AY_LD + lane + 16 * i], acc[ch * 4 + i]);
            }
        }
    }
    // score gradients of keys the causal bound skipped are zero
    if (p.ds && qi < p.L)
        for (int kj = kend + lane; kj < p.S; kj += 16) p.ds[b * p.sds[0] + h * p.sds[1] + qi * p.sds[2] + (int64_t)kj * p.sds[3]] = 0.0f;
    if (qi >= p.L) return;
    char* ob = static_cast<char*>(p.dq) + (b * p.sdq[0] + h * p.sdq[1] + qi * p.sdq[2]) * p.es;
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const int c = (i / 4) * AY_DC + lane + 16 * (i % 4);
        if (c < p.D) st<DT>(ob, c * p.sdq[3], acc[i] * p.scale);
    }
}

// dK and dV: a workgroup owns 16 keys of one key/value head and visits every
// query of every query head that reads it.
template <int DT, int N>
__global__ __launch_bounds__(AY_THREADS) void attn_any_dkv_kernel(AnyAttnArgs p) {
    __shared__ float as_[AY_ROWS * AY_LD];   // k chunk, then v chunk
    __shared__ float bs[AY_TILE * AY_LD];    // q chunk, dout chunk, dout chunk, q chunk
    __shared__ float pts[AY_ROWS * (AY_TILE + 1)];
    __shared__ float dsts[AY_ROWS * (AY_TILE + 1)];
    const int r = threadIdx.x / 16, lane = threadIdx.x % 16;
    const int hk = blockIdx.y, b = blockIdx.z;
    const int k0 = blockIdx.x * AY_ROWS, kj = k0 + r;
    const char* kb = static_cast<const char*>(p.k) + (b * p.sk[0] + hk * p.sk[1]) * p.es;
    const char* vb = static_cast<const char*>(p.v) + (b * p.sv[0] + hk * p.sv[1]) * p.es;

    float dk[N], dv[N];
#pragma unroll
    for (int i = 0; i < N; ++i) dk[i] = dv[i] = 0.0f;
    for (int g = 0; g < p.group; ++g) {
        const int h = hk * p.group + g;
        const char* qb = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * p.es;
        const char* gb = static_cast<const char*>(p.dout) + (b * p.sdo[0] + h * p.sdo[1]) * p.es;
        const char* bb = p.bias ? static_cast<const char*>(p.bias) + (b * p.sb[0] + h * p.sb[1]) * p.es : nullptr;
        // queries before the block's first key see none of its keys under the causal mask
        const int qstart = p.causal ? (k0 / AY_TILE) * AY_TILE : 0;
        for (int q0 = qstart; q0 < p.L; q0 += AY_TILE) {
            float s0 = 0.0f, s1 = 0.0f, g0 = 0.0f, g1 = 0.0f;
            for (int c0 = 0; c0 < p.D; c0 += AY_DC) {
                __syncthreads();
                stage<DT>(as_, AY_ROWS, kb, p.sk[2], p.sk[3], k0, p.S, c0, p.D);
                stage<DT>(bs, AY_TILE, qb, p.sq[2], p.sq[3], q0, p.L, c0, p.D);
                __syncthreads();
                const int n = std::min(AY_DC, p.D - c0);
    #pragma unroll 4
            for (int c = 0; c < n; ++c) {
                    const float a = as_[r * AY_LD + c];
                    s0 = fmaf(a, bs[lane * AY_LD + c], s0);
                    s1 = fmaf(a, bs[(lane + 16) * AY_LD + c], s1);
                }
            }
            for (int c0 = 0; c0 < p.Dv; c0 += AY_DC) {
                __syncthreads();
                stage<DT>(as_, AY_ROWS, vb, p.sv[2], p.sv[3], k0, p.S, c0, p.Dv);
                stage<DT>(bs, AY_TILE, gb, p.sdo[2], p.sdo[3], q0, p.L, c0, p.Dv);
                __syncthreads();
                const int n = std::min(AY_DC, p.Dv - c0);
    #pragma unroll 4
            for (int c = 0; c < n; ++c) {
                    const float a = as_[r * AY_LD + c];
                    g0 = fmaf(a, bs[lane * AY_LD + c], g0);
                    g1 = fmaf(a, bs[(lane + 16) * AY_LD + c], g1);
                }
            }
            const float sc[2] = {s0, s1}, gc[2] = {g0, g1};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int qi = q0 + lane + 16 * j;
                float pj = 0.0f, ds = 0.0f;
                if (qi < p.L && kj < p.S && !(p.causal && kj > qi)) {
                    const float lse = p.lse[b * p.sl[0] + h * p.sl[1] + qi * p.sl[2]];
                    if (lse != INFINITY) {
                        float s = sc[j] * p.scale;
                        if (bb) s += ld<DT>(bb, qi * p.sb[2] + kj * p.sb[3]);
                        pj = expf(s - lse);
                        ds = pj * (gc[j] - p.delta[((int64_t)b * p.Hq + h) * p.L + qi]);
                    }
                }
                pts[r * (AY_TILE + 1) + lane + 16 * j] = round_dt<DT>(pj);
                dsts[r * (AY_TILE + 1) + lane + 16 * j] = round_dt<DT>(ds);
            }
            // dV += P^T dout and dK += dS^T q, both by 64-column chunks
#pragma unroll
            for (int ch = 0; ch < N / 4; ++ch) {
                if (ch * AY_DC >= p.Dv) break;
                __syncthreads();
                stage<DT>(bs, AY_TILE, gb, p.sdo[2], p.sdo[3], q0, p.L, ch * AY_DC, p.Dv);
                __syncthreads();
    #pragma unroll 2
            for (int j = 0; j < AY_TILE; ++j) {
                    const float pj = pts[r * (AY_TILE + 1) + j];
#pragma unroll
                    for (int i = 0; i < 4; ++i) dv[ch * 4 + i] = fmaf(pj, bs[j * AY_LD + lane + 16 * i], dv[ch * 4 + i]);
                }
            }
#pragma unroll
            for (int ch = 0; ch < N / 4; ++ch) {
                if (ch * AY_DC >= p.D) break;
                __syncthreads();
                stage<DT>(bs, AY_TILE, qb, p.sq[2], p.sq[3], q0, p.L, ch * AY_DC, p.D);
                __syncthreads();
    #pragma unroll 2
            for (int j = 0; j < AY_TILE; ++j) {
                    const float dj = dsts[r * (AY_TILE + 1) + j];
#pragma unroll
                    for (int i = 0; i < 4; ++i) dk[ch * 4 + i] = fmaf(dj, bs[j * AY_LD + lane + 16 * i], dk[ch * 4 + i]);
                }
            }
        }
    }
    if (kj >= p.S) return;
    char* kout = static_cast<char*>(p.dk) + (b * p.sdk[0] + hk * p.sdk[1] + kj * p.sdk[2]) * p.es;
    char* vout = static_cast<char*>(p.dv) + (b * p.sdv[0] + hk * p.sdv[1] + kj * p.sdv[2]) * p.es;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int c = (i / 4) * AY_DC + lane + 16 * (i % 4);
        if (c < p.D) st<DT>(kout, c * p.sdk[3], dk[i] * p.scale);
        if (c < p.Dv) st<DT>(vout, c * p.sdv[3], dv[i]);
    }
}

// Accumulators a thread needs for a head dim (16 threads share a row).
int acc_slots(int64_t dim) { return dim <= 64 ? 4 : dim <= 128 ? 8 : dim <= 256 ? 16 : 32; }

#define TVK_AY_LAUNCH(KERNEL, DT_, N_, GRID, ARGS, S_)                                                   \
    do {                                                                                                 \
        switch (N_) {                                                                                    \
        case 4: hipLaunchKernelGGL((KERNEL<DT_, 4>), GRID, dim3(AY_THREADS), 0, S_, ARGS); break;        \
        case 8: hipLaunchKernelGGL((KERNEL<DT_, 8>), GRID, dim3(AY_THREADS), 0, S_, ARGS); break;        \
        case 16: hipLaunchKernelGGL((KERNEL<DT_, 16>), GRID, dim3(AY_THREADS), 0, S_, ARGS); break;      \
        default: hipLaunchKernelGGL((KERNEL<DT_, 32>), GRID, dim3(AY_THREADS), 0, S_, ARGS); break;      \
        }                                                                                                \
    } while (0)

template <int DT>
void launch_fwd(const AnyAttnArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.L + AY_ROWS - 1) / AY_ROWS), (unsigned)a.Hq, (unsigned)a.B);
    TVK_AY_LAUNCH(attn_any_fwd_kernel, DT, acc_slots(a.Dv), grid, a, s);
}

template <int DT>
void launch_bwd(const AnyAttnArgs& a, int heads_kv, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.Hq * a.L;
    if (rows > 0) hipLaunchKernelGGL(attn_any_delta_kernel<DT>, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, a);
    const dim3 gq((unsigned)((a.L + AY_ROWS - 1) / AY_ROWS), (unsigned)a.Hq, (unsigned)a.B);
    if (a.L > 0) TVK_AY_LAUNCH(attn_any_dq_kernel, DT, acc_slots(a.D), gq, a, s);
    const dim3 gkv((unsigned)((a.S + AY_ROWS - 1) / AY_ROWS), (unsigned)heads_kv, (unsigned)a.B);
    if (a.S > 0) TVK_AY_LAUNCH(attn_any_dkv_kernel, DT, acc_slots(std::max(a.D, a.Dv)), gkv, a, s);
}

}  // namespace

bool attn_any_applies(const tvk_attention_desc* d) {
    return (d->dtype == TVK_F32 || d->dtype == TVK_F16 || d->dtype == TVK_BF16) && d->head_dim >= 1 && d->head_dim <= 512 &&
           d->head_dim_v >= 1 && d->head_dim_v <= 512 && d->batch <= 65535 && d->heads_q <= 65535 &&
           d->len_q <= (int64_t)1 << 30 && d->len_kv <= (int64_t)1 << 30;
}

AnyAttnArgs attn_any_args(const tvk_attention_desc* d) {
    AnyAttnArgs a{};
    a.q = d->q; a.k = d->k; a.v = d->v; a.bias = d->bias; a.out = d->out;
    a.lse = d->lse;
    for (int i = 0; i < 4; ++i) {
        a.sq[i] = d->q_stride[i];
        a.sk[i] = d->k_stride[i];
        a.sv[i] = d->v_stride[i];
        a.sb[i] = d->bias ? d->bias_stride[i] : 0;
        a.so[i] = d->out_stride[i];
    }
    for (int i = 0; i < 3; ++i) a.sl[i] = d->lse_stride[i];
    a.B = (int)d->batch;
    a.Hq = (int)d->heads_q;
    a.group = (int)(d->heads_q / d->heads_kv);
    a.L = (int)d->len_q;
    a.S = (int)d->len_kv;
    a.D = (int)d->head_dim;
    a.Dv = (int)d->head_dim_v;
    a.causal = d->causal != 0;
    a.scale = (float)d->scale;
    a.es = (int64_t)dtype_size(d->dtype);
    return a;
}

tvk_status attn_any_fwd(const tvk_attention_desc* d, hipStream_t s) {
    const AnyAttnArgs a = attn_any_args(d);
    switch (d->dtype) {
    case TVK_F32: launch_fwd<TVK_F32>(a, s); break;
    case TVK_F16: launch_fwd<TVK_F16>(a, s); break;
    default: launch_fwd<TVK_BF16>(a, s); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_attention_fwd: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status attn_any_bwd(const tvk_attention_bwd_desc* desc, float* delta, hipStream_t s) {
    const tvk_attention_desc* d = &desc->fwd;
    AnyAttnArgs a = attn_any_args(d);
    a.dout = desc->dout;
    a.dq = desc->dq;
    a.dk = desc->dk;
    a.dv = desc->dv;
    a.ds = desc->dscores;
    for (int i = 0; i < 4; ++i) {
        a.sdo[i] = desc->dout_stride[i];
        a.sdq[i] = desc->dq_stride[i];
        a.sdk[i] = desc->dk_stride[i];
        a.sdv[i] = desc->dv_stride[i];
        a.sds[i] = desc->dscores ? desc->dscores_stride[i] : 0;
    }
    a.delta = delta;
    switch (d->dtype) {
    case TVK_F32: launch_bwd<TVK_F32>(a, (int)d->heads_kv, s); break;
    case TVK_F16: launch_bwd<TVK_F16>(a, (int)d->heads_kv, s); break;
    default: launch_bwd<TVK_BF16>(a, (int)d->heads_kv, s); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_attention_bwd: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

}  // namespace tvk
