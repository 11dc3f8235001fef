// Fused scaled dot-product attention forward (tvk_attention_fwd) for gfx950.
//
// Reference semantics: chunked_forward / the fused kernel behind
// _scaled_dot_product_fused_attention_overrideable
// (src/api/ops/attention.cpp:115-139,434-500,697-719): scores
// scale*q.k (+ bias) in float32, causal mask j > i, softmax over keys, a row
// with no unmasked key gives 0 and lse = +inf; the probabilities are staged
// in the dtype before the product with v (src/shaders/ops/attention_coop.slang).
//
// Kernel: one workgroup of 4 waves owns 128 queries of one (batch, head);
// each wave owns 32 of them as two 16-query columns. Keys go by tiles of 64:
// K and V tiles are loaded into registers one tile ahead and parked in a
// double-buffered LDS pair. Per tile each wave computes the transposed scores
// S^T = K Q^T with v_mfma_f32_16x16x32 (keys on rows, queries on columns):
// lane l then holds query l%16 and keys 4(l/16)+r of every 16-key block, so
// the softmax row statistics need one lane-local pass and two cross-lane
// steps (xor 16, xor 32). The same accumulator layout is already the B
// operand of O^T = V^T P^T once rounded to the dtype: the 32 k-slots of one
// product are keys {4g..4g+3, 16+4g..16+4g+3} of the 16-lane group g, and
// V^T is read in exactly that key order with ds_read_b64_tr_b16 (four keys
// of one dv column per lane). Online softmax: the running max m and sum l of
// each query rescale O by exp(m_old - m_new) per tile; exp is v_exp_f32 on
// log2-scaled arguments.
#include "gemm_common.h"

#include <cmath>

namespace tvk {
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define TVK_LDS __attribute__((address_space(3)))

constexpr int AT_WAVES = 4;
constexpr int AT_BM = 32 * AT_WAVES;   // queries per workgroup
constexpr int AT_BN = 64;              // keys per tile
constexpr float AT_LOG2E = 1.4426950408889634f;

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* bias;
    uint16_t* out;
    float* lse;
    int64_t sq[4], sk[4], sv[4], sb[4], so[4], sl[3];
    int L, S, Hq, group;
    float scale;
    int causal;
    int out_vec;   // out rows 8-byte aligned with unit dv stride
};

template <int DT>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int DT>
__device__ inline uint32_t pack2(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, elem<DT>::from_f32(lo)) |
           ((uint32_t)__builtin_bit_cast(uint16_t, elem<DT>::from_f32(hi)) << 16);
}

__device__ inline float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m)); }
__device__ inline float xor_sum(float v, int m) { return v + __shfl_xor(v, m); }

template <int DT, int D, bool CAUSAL, bool BIAS>
__global__ __launch_bounds__(64 * AT_WAVES) void attn_fwd_kernel(AttnArgs p) {
    constexpr int DS = D / 32;          // 32-wide d steps of the score product
    constexpr int DT16 = D / 16;        // 16-wide dv tiles of the output
    constexpr int LDK = D + 8;          // LDS row pitch (halfs)
    constexpr int CH = AT_BN * D / 8;   // 16-byte chunks per K (or V) tile
    constexpr int CPT = CH / (64 * AT_WAVES);
    static_assert(CPT * 64 * AT_WAVES == CH, "whole chunks per thread");
    __shared__ __attribute__((aligned(16))) uint16_t ks[2][AT_BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t vs[2][AT_BN * LDK];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int g = lane / 16, c16 = lane % 16;
    const int b = blockIdx.z, h = blockIdx.y;
    const int hk = h / p.group;
    const int q0 = blockIdx.x * AT_BM + wave * 32;   // this wave's first query

    const uint16_t* Q = p.q + (int64_t)b * p.sq[0] + (int64_t)h * p.sq[1];
    const uint16_t* K = p.k + (int64_t)b * p.sk[0] + (int64_t)hk * p.sk[1];
    const uint16_t* V = p.v + (int64_t)b * p.sv[0] + (int64_t)hk * p.sv[1];

    // Q^T as the B operand: lane holds query q0+16qt+c16, d = 32ds + 8g .. +7
    u32x4 qf[2][DS];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + 16 * qt + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
            qf[qt][ds] = qi < p.L ? *reinterpret_cast<const u32x4*>(Q + (int64_t)qi * p.sq[2] + 32 * ds + 8 * g)
                                  : u32x4{0, 0, 0, 0};
    }

    f32x4 oacc[DT16][2];
#pragma unroll
    for (int i = 0; i < DT16; ++i)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) oacc[i][qt] = f32x4{0, 0, 0, 0};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};

    int ntiles = (p.S + AT_BN - 1) / AT_BN;
    if (CAUSAL) {
        const int last_q = min(p.L, (int)blockIdx.x * AT_BM + AT_BM) - 1;   // keys beyond it are masked for the block
        ntiles = min(ntiles, last_q / AT_BN + 1);
    }

    u32x4 kreg[CPT], vreg[CPT];
    auto load_tile = [&](int j) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 64 * AT_WAVES;
            const int key = c / (D / 8), d8 = (c % (D / 8)) * 8;
            const int kj = j * AT_BN + key;
            if (kj < p.S) {
                kreg[i] = *reinterpret_cast<const u32x4*>(K + (int64_t)kj * p.sk[2] + d8);
                vreg[i] = *reinterpret_cast<const u32x4*>(V + (int64_t)kj * p.sv[2] + d8);
            } else {
                kreg[i] = u32x4{0, 0, 0, 0};
                vreg[i] = u32x4{0, 0, 0, 0};
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 64 * AT_WAVES;
            const int key = c / (D / 8), d8 = (c % (D / 8)) * 8;
            *reinterpret_cast<u32x4*>(&ks[buf][key * LDK + d8]) = kreg[i];
            *reinterpret_cast<u32x4*>(&vs[buf][key * LDK + d8]) = vreg[i];
        }
    };

    if (ntiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();

    for (int j = 0; j < ntiles; ++j) {
        const int buf = j & 1;
        if (j + 1 < ntiles) load_tile(j + 1);   // in flight while this tile computes

        // ---- S^T = K Q^T over 4 key blocks x 2 query columns
        f32x4 sacc[4][2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) sacc[kt][qt] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const u32x4 kf = *reinterpret_cast<const u32x4*>(&ks[buf][(kt * 16 + c16) * LDK + 32 * ds + 8 * g]);
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) sacc[kt][qt] = mfma16<DT>(kf, qf[qt][ds], sacc[kt][qt]);
            }
        }

        // ---- scale, bias, masks; online softmax per query column
        float alpha[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const int qi = q0 + 16 * qt + c16;
            float tmax = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kj = j * AT_BN + kt * 16 + 4 * g + r;
                    float s = sacc[kt][qt][r] * p.scale;
                    if (BIAS && kj < p.S && qi < p.L) {
                        const uint16_t bv = p.bias[(int64_t)b * p.sb[0] + (int64_t)h * p.sb[1] + (int64_t)qi * p.sb[2] + (int64_t)kj * p.sb[3]];
                        s = s + elem<DT>::to_f32(__builtin_bit_cast(typename elem<DT>::T, bv));
                    }
                    if (kj >= p.S || (CAUSAL && kj > qi)) s = -INFINITY;
                    sacc[kt][qt][r] = s;
                    tmax = fmaxf(tmax, s);
                }
            tmax = xor_max(xor_max(tmax, 16), 32);
            const float m_new = fmaxf(m_run[qt], tmax);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            alpha[qt] = __builtin_amdgcn_exp2f((m_run[qt] - m_use) * AT_LOG2E);
            float rsum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f((sacc[kt][qt][r] - m_use) * AT_LOG2E);
                    sacc[kt][qt][r] = e;
                    rsum += e;
                }
            rsum = xor_sum(xor_sum(rsum, 16), 32);
            l_run[qt] = l_run[qt] * alpha[qt] + rsum;
            m_run[qt] = m_new;
        }
#pragma unroll
        for (int i = 0; i < DT16; ++i)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int r = 0; r < 4; ++r) oacc[i][qt][r] *= alpha[qt];

        // ---- O^T += V^T P^T: two 32-key products, k-slots in the S^T lane order
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            u32x4 pf[2];
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                const f32x4 a = sacc[2 * kk][qt], c = sacc[2 * kk + 1][qt];
                pf[qt] = u32x4{pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]), pack2<DT>(c[2], c[3])};
            }
#pragma unroll
            for (int i = 0; i < DT16; ++i) {
                // lane c16 of group g: column dv = 16i + c16, keys 32kk + {4g..4g+3, 16+4g..16+4g+3}
                u32x4 vf;
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const int kr = 32 * kk + 16 * rr + 4 * g + c16 / 4;
                    TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(TVK_LDS uint16_t*)&vs[buf][kr * LDK + 16 * i + (c16 % 4) * 4];
                    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
                    vf[2 * rr] = w.x;
                    vf[2 * rr + 1] = w.y;
                }
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) oacc[i][qt] = mfma16<DT>(vf, pf[qt], oacc[i][qt]);
            }
        }

        // buffer buf^1 was last read in iteration j-1, which every wave left
        // through the barrier below: it can take tile j+1 now
        if (j + 1 < ntiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- O = O^T / l; lse = m + log l (+inf for a row that attended to nothing)
    uint16_t* O = p.out + (int64_t)b * p.so[0] + (int64_t)h * p.so[1];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + 16 * qt + c16;
        if (qi >= p.L) continue;
        const float inv = l_run[qt] > 0.0f ? 1.0f / l_run[qt] : 0.0f;
#pragma unroll
        for (int i = 0; i < DT16; ++i) {
            const int dv = 16 * i + 4 * g;   // four consecutive dv of column qi
            const f32x4 o = oacc[i][qt];
            uint16_t* op = O + (int64_t)qi * p.so[2] + (int64_t)dv * p.so[3];
            if (p.out_vec) {
                *reinterpret_cast<u32x2*>(op) = u32x2{pack2<DT>(o[0] * inv, o[1] * inv), pack2<DT>(o[2] * inv, o[3] * inv)};
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    op[(int64_t)r * p.so[3]] = __builtin_bit_cast(uint16_t, elem<DT>::from_f32(o[r] * inv));
            }
        }
        if (g == 0)
            p.lse[(int64_t)b * p.sl[0] + (int64_t)h * p.sl[1] + (int64_t)qi * p.sl[2]] =
                l_run[qt] > 0.0f ? m_run[qt] + logf(l_run[qt]) : INFINITY;
    }
}

template <int DT, int D>
void launch_attn(const AttnArgs& a, bool causal, bool bias, dim3 grid, hipStream_t s) {
    const dim3 block(64 * AT_WAVES);
    if (causal) {
        if (bias) hipLaunchKernelGGL((attn_fwd_kernel<DT, D, true, true>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((attn_fwd_kernel<DT, D, true, false>), grid, block, 0, s, a);
    } else {
        if (bias) hipLaunchKernelGGL((attn_fwd_kernel<DT, D, false, true>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((attn_fwd_kernel<DT, D, false, false>), grid, block, 0, s, a);
    }
}

}  // namespace
}  // namespace tvk

using namespace tvk;

extern "C" tvk_status tvk_attention_fwd(const tvk_attention_desc* d) {
    if (!d) return fail(TVK_ERR_INVALID, "tvk_attention_fwd: desc is NULL");
    if (d->dtype != TVK_F16 && d->dtype != TVK_BF16)
        return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: dtype must be float16 or bfloat16");
    if (d->batch < 0 || d->heads_q < 0 || d->heads_kv <= 0 || d->len_q < 0 || d->len_kv < 0)
        return fail(TVK_ERR_INVALID, "tvk_attention_fwd: negative size");
    if (d->heads_q % d->heads_kv != 0)
        return fail(TVK_ERR_INVALID, "tvk_attention_fwd: heads_q is not a multiple of heads_kv");
    if (d->head_dim != d->head_dim_v || (d->head_dim != 64 && d->head_dim != 128))
        return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: head_dim == head_dim_v in {64, 128} only");
    if (d->batch > 65535 || d->heads_q > 65535 || d->len_q > (int64_t)0x7fffffff || d->len_kv > (int64_t)0x7fffffff)
        return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: grid too large");
    if (d->batch == 0 || d->heads_q == 0 || d->len_q == 0) return TVK_OK;
    if (!d->q || !d->k || !d->v || !d->out || !d->lse) return fail(TVK_ERR_INVALID, "tvk_attention_fwd: NULL tensor");
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    for (const int64_t* st : {d->q_stride, d->k_stride, d->v_stride}) {
        if (st[3] != 1) return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: q, k, v need unit stride along the head dimension");
        for (int i = 0; i < 3; ++i)
            if (st[i] % 8 != 0) return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: q, k, v rows must be 16-byte aligned");
    }
    if (!al16(d->q) || !al16(d->k) || !al16(d->v)) return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: unaligned q, k or v");
    AttnArgs a{};
    a.q = static_cast<const uint16_t*>(d->q);
    a.k = static_cast<const uint16_t*>(d->k);
    a.v = static_cast<const uint16_t*>(d->v);
    a.bias = static_cast<const uint16_t*>(d->bias);
    a.out = static_cast<uint16_t*>(d->out);
    a.lse = d->lse;
    for (int i = 0; i < 4; ++i) {
        a.sq[i] = d->q_stride[i];
        a.sk[i] = d->k_stride[i];
        a.sv[i] = d->v_stride[i];
        a.sb[i] = d->bias ? d->bias_stride[i] : 0;
        a.so[i] = d->out_stride[i];
    }
    for (int i = 0; i < 3; ++i) a.sl[i] = d->lse_stride[i];
    a.L = (int)d->len_q;
    a.S = (int)d->len_kv;
    a.Hq = (int)d->heads_q;
    a.group = (int)(d->heads_q / d->heads_kv);
    a.scale = (float)d->scale;
    a.causal = d->causal != 0;
    a.out_vec = d->out_stride[3] == 1 && (reinterpret_cast<uintptr_t>(d->out) & 7) == 0 && d->out_stride[2] % 4 == 0 &&
                d->out_stride[1] % 4 == 0 && d->out_stride[0] % 4 == 0;
    const dim3 grid((unsigned)((d->len_q + AT_BM - 1) / AT_BM), (unsigned)d->heads_q, (unsigned)d->batch);
    const hipStream_t s = resolve_stream(d->stream);
    const bool bias = d->bias != nullptr;
    if (d->dtype == TVK_F16) {
        if (d->head_dim == 64) launch_attn<TVK_F16, 64>(a, a.causal, bias, grid, s);
        else launch_attn<TVK_F16, 128>(a, a.causal, bias, grid, s);
    } else {
        if (d->head_dim == 64) launch_attn<TVK_BF16, 64>(a, a.causal, bias, grid, s);
        else launch_attn<TVK_BF16, 128>(a, a.causal, bias, grid, s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_attention_fwd: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}
