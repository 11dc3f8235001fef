// Fused scaled dot-product attention forward (tvk_attention_fwd) for gfx950.
//
// Reference semantics: chunked_forward / the fused kernel behind
// _scaled_dot_product_fused_attention_overrideable
// (src/api/ops/attention.cpp:115-139,434-500,697-719): scores
// scale*q.k (+ bias) in float32, causal mask j > i, softmax over keys, a row
// with no unmasked key gives 0 and lse = +inf; the probabilities are staged
// in the dtype before the product with v (src/shaders/ops/attention_coop.slang).
//
// Kernel: one workgroup of 4 waves owns 64 or 128 queries of one (batch, head);
// each wave owns one or two 16-query columns of them. Keys go by tiles of 64:
// K and V tiles are loaded into registers one tile ahead and parked in a
// double-buffered LDS pair. Per tile each wave computes the transposed scores
// S^T = K Q^T with v_mfma_f32_16x16x32 (keys on rows, queries on columns):
// lane l then holds query l%16 and keys 4(l/16)+r of every 16-key block, so
// a query's row statistics are one lane-local pass plus two lane swaps
// (v_permlane32_swap, v_permlane16_swap). The same accumulator layout is
// already the B operand of O^T = V^T P^T once rounded to the dtype (one
// v_cvt_pk per pair): the 32 k-slots of one product are keys
// {4g..4g+3, 16+4g..16+4g+3} of the 16-lane group g, and V^T is read in
// exactly that key order with ds_read_b64_tr_b16 (four keys of one dv column
// per lane).
//
// Online softmax in log2 units: with c = |scale|*log2(e) (q negated when the
// scale is negative, which is exact), the running max m of c*q.k and the
// probabilities exp2(c*q.k - m) come from the raw accumulators with one fma
// each. Masks are applied only on the tiles that reach past the last key or
// cross the causal diagonal; a bias switches every tile to the explicit
// scale*q.k + bias path. O is rescaled by exp2(m_old - m_new) only when some
// query's max moved (a factor of exactly 1 otherwise), and each lane keeps
// its own partial row sum l, reduced across the four lane groups once at the
// end (l and O share every rescale factor).
#include "gemm_common.h"
#include "attention_any.h"

#include <algorithm>
#include <cmath>

namespace tvk {
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
#define TVK_LDS __attribute__((address_space(3)))

constexpr int AT_WAVES = 4;
constexpr int AT_BN = 64;              // keys per tile
constexpr float AT_LOG2E = 1.4426950408889634f;
constexpr float AT_LN2 = 0.6931471805599453f;

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* bias;
    uint16_t* out;
    float* lse;
    int64_t sq[4], sk[4], sv[4], sb[4], so[4], sl[3];
    int L, S, Hq, group;
    int nqb, BH;       // query tiles per (batch, head); batch * heads
    float scale;       // signed scale (bias path)
    float c2;          // |scale| * log2(e) (no-bias path)
    uint32_t qflip;    // sign bits flipped into q on the no-bias path when scale < 0
    int out_vec;       // out rows 8-byte aligned with unit dv stride
};

template <int DT>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Two floats rounded to nearest even into one packed pair (v_cvt_pk_f16_f32 /
// v_cvt_pk_bf16_f32), lo in the low half.
template <int DT>
__device__ inline uint32_t pack2(float lo, float hi) {
    if constexpr (DT == TVK_F16)
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{lo, hi}, f16x2v));
    else
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{lo, hi}, bf16x2v));
}

__device__ inline float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m)); }
__device__ inline float xor_sum(float v, int m) { return v + __shfl_xor(v, m); }

// Max / sum over lanes {l, l^16, l^32, l^48}: permlane32_swap of a value with
// itself hands each lane its partner l^32, permlane16_swap then l^16. Every
// lane of the four ends with the same bits.
__device__ inline float lanes4_max(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
    const uint32_t w = __builtin_bit_cast(uint32_t, v);
    const auto c = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)c[0]), __builtin_bit_cast(float, (uint32_t)c[1]));
}
__device__ inline float lanes4_sum(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
    const uint32_t w = __builtin_bit_cast(uint32_t, v);
    const auto c = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return __builtin_bit_cast(float, (uint32_t)c[0]) + __builtin_bit_cast(float, (uint32_t)c[1]);
}

// Workgroup -> (query tile qb, batch*head bh). Workgroups are dealt to the 8
// XCDs round robin (id % 8); when batch*heads is a multiple of 8 each
// (batch, head) stays on one XCD, so its K and V tiles are shared in that
// XCD's L2. Causal rows do work in proportion to their query tile: the
// heaviest tiles are dealt first, every XCD taking the same mix.
template <bool CAUSAL, class Args>
__device__ inline void attn_block(const Args& p, int& qb, int& bh) {
    const int id = blockIdx.x;
    if (p.BH % 8 == 0) {
        const int xcd = id % 8, local = id / 8, per = p.BH / 8;
        if (CAUSAL) {
            qb = p.nqb - 1 - local / per;
            bh = (local % per) * 8 + xcd;
        } else {
            qb = local % p.nqb;
            bh = (local / p.nqb) * 8 + xcd;
        }
    } else if (CAUSAL) {
        qb = p.nqb - 1 - id / p.BH;
        bh = id % p.BH;
    } else {
        qb = id % p.nqb;
        bh = id / p.nqb;
    }
}

// One key tile of the online softmax for QPW query columns: scores from the
// accumulators (PLAIN: no mask reaches the tile and no bias, so max and
// exponent work on the raw products), running max m and per-lane sum l
// updated, probabilities left in sacc, rescale factors in alpha.
template <int DT, bool PLAIN, bool BIAS, bool CAUSAL, int QPW>
__device__ inline void softmax_tile(const AttnArgs& p, f32x4 (&sacc)[4][QPW], float (&m_run)[QPW], float (&l_run)[QPW],
                                    float (&alpha)[QPW], int k0, int q0, int b, int h, int g, int c16) {
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) {
        float tmax = -INFINITY;
        if (PLAIN) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sacc[kt][qt][r]);
            tmax = lanes4_max(tmax) * p.c2;
        } else {
            const int qi = q0 + 16 * qt + c16;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kj = k0 + kt * 16 + 4 * g + r;
                    float s;
                    if (BIAS) {
                        s = sacc[kt][qt][r] * p.scale;
                        if (kj < p.S && qi < p.L) {
                            const uint16_t bv = p.bias[(int64_t)b * p.sb[0] + (int64_t)h * p.sb[1] + (int64_t)qi * p.sb[2] + (int64_t)kj * p.sb[3]];
                            s = s + elem<DT>::to_f32(__builtin_bit_cast(typename elem<DT>::T, bv));
                        }
                        s *= AT_LOG2E;
                    } else {
                        s = sacc[kt][qt][r] * p.c2;
                    }
                    if (kj >= p.S || (CAUSAL && kj > qi)) s = -INFINITY;
                    sacc[kt][qt][r] = s;
                    tmax = fmaxf(tmax, s);
                }
            tmax = lanes4_max(tmax);
        }
        const float m_old = m_run[qt];
        const float m_new = fmaxf(m_old, tmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        // O and l are still 0 while m_old is -inf
        alpha[qt] = (m_old == m_new || m_old == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_old - m_use);
        float rsum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = PLAIN ? __builtin_fmaf(sacc[kt][qt][r], p.c2, -m_use) : sacc[kt][qt][r] - m_use;
                const float e = __builtin_amdgcn_exp2f(x);
                sacc[kt][qt][r] = e;
                rsum += e;
            }
        l_run[qt] = l_run[qt] * alpha[qt] + rsum;
        m_run[qt] = m_new;
    }
}

// One 16-query column per wave at head_dim 64 without a bias fits 128 VGPRs: four waves per
// SIMD, the occupancy the 39 KB of LDS per workgroup allows.
template <int DT, int D, bool CAUSAL, bool BIAS, int QPW>
__global__ __launch_bounds__(64 * AT_WAVES) __attribute__((amdgpu_waves_per_eu(D == 64 && QPW == 1 && !BIAS ? 4 : 1)))
void attn_fwd_kernel(AttnArgs p) {
    constexpr int BMQ = 16 * QPW * AT_WAVES;   // queries per workgroup
    constexpr int DS = D / 32;          // 32-wide d steps of the score product
    constexpr int DT16 = D / 16;        // 16-wide dv tiles of the output
    // LDS row pitches (halfs): K rows step 4 banks (16-byte reads of 8
    // consecutive rows cover all 32 banks once), V rows step 8 banks (the
    // transposed 8-byte reads of 4 consecutive rows cover all 32 banks once)
    constexpr int LDK = D + 8;
    constexpr int LDV = D + 16;
    constexpr int CH = AT_BN * D / 8;   // 16-byte chunks per K (or V) tile
    constexpr int CPT = CH / (64 * AT_WAVES);
    static_assert(CPT * 64 * AT_WAVES == CH, "whole chunks per thread");
    __shared__ __attribute__((aligned(16))) uint16_t ks[2][AT_BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t vs[2][AT_BN * LDV];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int g = lane / 16, c16 = lane % 16;
    int qb, bh;
    attn_block<CAUSAL>(p, qb, bh);
    const int b = bh / p.Hq, h = bh % p.Hq;
    const int hk = h / p.group;
    const int q0 = qb * BMQ + wave * 16 * QPW;   // this wave's first query

    const uint16_t* Q = p.q + (int64_t)b * p.sq[0] + (int64_t)h * p.sq[1];

    // Q^T as the B operand: lane holds query q0+16qt+c16, d = 32ds + 8g .. +7
    u32x4 qf[QPW][DS];
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) {
        const int qi = q0 + 16 * qt + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            u32x4 x = qi < p.L ? *reinterpret_cast<const u32x4*>(Q + (int64_t)qi * p.sq[2] + 32 * ds + 8 * g)
                               : u32x4{0, 0, 0, 0};
            if (!BIAS) x ^= p.qflip;
            qf[qt][ds] = x;
        }
    }

    f32x4 oacc[DT16][QPW];
#pragma unroll
    for (int i = 0; i < DT16; ++i)
#pragma unroll
        for (int qt = 0; qt < QPW; ++qt) oacc[i][qt] = f32x4{0, 0, 0, 0};
    float m_run[QPW], l_run[QPW];   // m in log2 units; l a per-lane partial sum
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.0f;
    }

    int ntiles = (p.S + AT_BN - 1) / AT_BN;
    if (CAUSAL) {
        const int last_q = min(p.L, qb * BMQ + BMQ) - 1;   // keys beyond it are masked for the block
        ntiles = min(ntiles, last_q / AT_BN + 1);
    }

    // K/V tile loads: a uniform base per tile plus a 32-bit byte offset per chunk
    const char* Kh = reinterpret_cast<const char*>(p.k + (int64_t)b * p.sk[0] + (int64_t)hk * p.sk[1]);
    const char* Vh = reinterpret_cast<const char*>(p.v + (int64_t)b * p.sv[0] + (int64_t)hk * p.sv[1]);
    const int64_t kstep = (int64_t)AT_BN * p.sk[2] * 2, vstep = (int64_t)AT_BN * p.sv[2] * 2;
    uint32_t koff[CPT], voff[CPT];
    int krow[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * 64 * AT_WAVES;
        krow[i] = c / (D / 8);
        const int d8 = (c % (D / 8)) * 8;
        koff[i] = (uint32_t)(((int64_t)krow[i] * p.sk[2] + d8) * 2);
        voff[i] = (uint32_t)(((int64_t)krow[i] * p.sv[2] + d8) * 2);
    }
    // two register sets: tile j+2 is in flight while tile j computes and tile
    // j+1 waits in registers for its LDS buffer
    u32x4 kra[CPT], vra[CPT], krb[CPT], vrb[CPT];
    auto load_tile = [&](int j, u32x4 (&kreg)[CPT], u32x4 (&vreg)[CPT]) {
        const char* kt = Kh + (int64_t)j * kstep;
        const char* vt = Vh + (int64_t)j * vstep;
        if (j * AT_BN + AT_BN <= p.S) {
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                kreg[i] = *reinterpret_cast<const u32x4*>(kt + koff[i]);
                vreg[i] = *reinterpret_cast<const u32x4*>(vt + voff[i]);
            }
        } else {
            // rows past the last key are zeros: P is 0 there and V must be finite
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                if (j * AT_BN + krow[i] < p.S) {
                    kreg[i] = *reinterpret_cast<const u32x4*>(kt + koff[i]);
                    vreg[i] = *reinterpret_cast<const u32x4*>(vt + voff[i]);
                } else {
                    kreg[i] = u32x4{0, 0, 0, 0};
                    vreg[i] = u32x4{0, 0, 0, 0};
                }
            }
        }
    };
    auto store_tile = [&](int buf, const u32x4 (&kreg)[CPT], const u32x4 (&vreg)[CPT]) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 64 * AT_WAVES;
            const int key = c / (D / 8), d8 = (c % (D / 8)) * 8;
            *reinterpret_cast<u32x4*>(&ks[buf][key * LDK + d8]) = kreg[i];
            *reinterpret_cast<u32x4*>(&vs[buf][key * LDV + d8]) = vreg[i];
        }
    };

    auto compute_tile = [&](int j, int buf) {
        const int k0 = j * AT_BN;
        // a causal wave whose queries all precede the tile has nothing to add
        if (CAUSAL && k0 > q0 + 16 * QPW - 1) return;
        // ---- S^T = K Q^T over 4 key blocks x QPW query columns
        f32x4 sacc[4][QPW];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int qt = 0; qt < QPW; ++qt) sacc[kt][qt] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const u32x4 kf = *reinterpret_cast<const u32x4*>(&ks[buf][(kt * 16 + c16) * LDK + 32 * ds + 8 * g]);
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt) sacc[kt][qt] = mfma16<DT>(kf, qf[qt][ds], sacc[kt][qt]);
            }
        }

        // ---- online softmax per query column
        float alpha[QPW];
        if (!BIAS && k0 + AT_BN <= p.S && !(CAUSAL && k0 + AT_BN - 1 > q0))
            softmax_tile<DT, true, false, CAUSAL, QPW>(p, sacc, m_run, l_run, alpha, k0, q0, b, h, g, c16);
        else
            softmax_tile<DT, false, BIAS, CAUSAL, QPW>(p, sacc, m_run, l_run, alpha, k0, q0, b, h, g, c16);
        bool rescale = false;
#pragma unroll
        for (int qt = 0; qt < QPW; ++qt) rescale = rescale || alpha[qt] != 1.0f;
        if (__any(rescale)) {
#pragma unroll
            for (int i = 0; i < DT16; ++i)
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) oacc[i][qt][r] *= alpha[qt];
        }

        // ---- O^T += V^T P^T: two 32-key products, k-slots in the S^T lane order
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            u32x4 pf[QPW];
#pragma unroll
            for (int qt = 0; qt < QPW; ++qt) {
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
                    TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(TVK_LDS uint16_t*)&vs[buf][kr * LDV + 16 * i + (c16 % 4) * 4];
                    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
                    vf[2 * rr] = w.x;
                    vf[2 * rr + 1] = w.y;
                }
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt) oacc[i][qt] = mfma16<DT>(vf, pf[qt], oacc[i][qt]);
            }
        }
    };

    if (ntiles > 0) {
        load_tile(0, kra, vra);
        if (ntiles > 1) load_tile(1, krb, vrb);
        store_tile(0, kra, vra);
    }
    __syncthreads();

    // Two tiles per trip so the register sets stay fixed: LDS buffer j%2
    // holds tile j. Each store goes to the buffer that the iteration before
    // the last barrier finished reading.
    for (int j = 0; j < ntiles; j += 2) {
        if (j + 2 < ntiles) load_tile(j + 2, kra, vra);
        compute_tile(j, 0);
        if (j + 1 < ntiles) store_tile(1, krb, vrb);
        __syncthreads();
        if (j + 1 >= ntiles) break;
        if (j + 3 < ntiles) load_tile(j + 3, krb, vrb);
        compute_tile(j + 1, 1);
        if (j + 2 < ntiles) store_tile(0, kra, vra);
        __syncthreads();
    }

    // ---- O = O^T / l; lse = m ln2 + log l (+inf for a row that attended to nothing)
    float l_tot[QPW];
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) l_tot[qt] = lanes4_sum(l_run[qt]);   // every lane, before any divergence
    uint16_t* O = p.out + (int64_t)b * p.so[0] + (int64_t)h * p.so[1];
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) {
        const int qi = q0 + 16 * qt + c16;
        if (qi >= p.L) continue;
        const float inv = l_tot[qt] > 0.0f ? 1.0f / l_tot[qt] : 0.0f;
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
                l_tot[qt] > 0.0f ? m_run[qt] * AT_LN2 + logf(l_tot[qt]) : INFINITY;
    }
}

template <int DT, int D, int QPW>
void launch_attn_q(AttnArgs a, bool causal, bool bias, int64_t bh, int64_t L, hipStream_t s) {
    constexpr int BMQ = 16 * QPW * AT_WAVES;
    a.nqb = (int)((L + BMQ - 1) / BMQ);
    a.BH = (int)bh;
    const dim3 grid((unsigned)(a.nqb * bh)), block(64 * AT_WAVES);
    if (causal) {
        if (bias) hipLaunchKernelGGL((attn_fwd_kernel<DT, D, true, true, QPW>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((attn_fwd_kernel<DT, D, true, false, QPW>), grid, block, 0, s, a);
    } else {
        if (bias) hipLaunchKernelGGL((attn_fwd_kernel<DT, D, false, true, QPW>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((attn_fwd_kernel<DT, D, false, false, QPW>), grid, block, 0, s, a);
    }
}

// Query columns per wave: at head_dim 64, two (128 queries per workgroup) when
// that still gives the device plenty of workgroups, else one (64 per
// workgroup). At head_dim 128 two columns need over 256 VGPRs (one wave per
// SIMD), so it is always one.
template <int DT, int D>
void launch_attn(const AttnArgs& a, bool causal, bool bias, int64_t batch, int64_t heads, int64_t L, hipStream_t s) {
    if constexpr (D == 64) {
        if (batch * heads * ((L + 127) / 128) >= 2048) {
            launch_attn_q<DT, D, 2>(a, causal, bias, batch * heads, L, s);
            return;
        }
    }
    launch_attn_q<DT, D, 1>(a, causal, bias, batch * heads, L, s);
}


// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------

struct AttnBwdArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* bias;
    const uint16_t* out;
    const uint16_t* dout;
    const float* lse;
    float* delta;          // [B][Hq][L], dense
    uint16_t* dq;
    uint16_t* dk;
    uint16_t* dv;
    int64_t sq[4], sk[4], sv[4], sb[4], so[4], sdo[4], sdq[4], sdk[4], sdv[4], sl[3];
    int L, S, Hq, group;
    int nqb, BH;       // dQ pass: query tiles per (batch, head), batch * heads
    float scale;
    float c2;          // scale * log2(e)
    int o_vec;         // out: unit stride along the head dim and 16-byte aligned rows
};

// 64-bit stores of four consecutive elements along the head dimension
template <int DT>
__device__ inline void store4(uint16_t* dst, f32x4 v, float mul) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{pack2<DT>(v[0] * mul, v[1] * mul), pack2<DT>(v[2] * mul, v[3] * mul)};
}

// Reads, with ds_read_b64_tr_b16, the A operand M^T for M^T X where M is an
// LDS tile [row][LDK] of 16-bit values: lane c16 of group g gets column
// 16*i + c16 at rows 32*kk + {4g..4g+3, 16+4g..16+4g+3} (the k-slot order of
// a transposed-score accumulator).
template <int LDK>
__device__ inline u32x4 read_tr(const uint16_t* tile, int kk, int i, int g, int c16) {
    u32x4 f;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const int kr = 32 * kk + 16 * rr + 4 * g + c16 / 4;
        TVK_LDS s16x4* ptr = (TVK_LDS s16x4*)(uintptr_t)(TVK_LDS const uint16_t*)&tile[kr * LDK + 16 * i + (c16 % 4) * 4];
        const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(ptr));
        f[2 * rr] = w.x;
        f[2 * rr + 1] = w.y;
    }
    return f;
}

// dQ pass (and delta): the forward's orientation. 4 waves x 16 or 32 queries
// of one (batch, head), workgroups dealt as the forward's; key tiles of 64
// through double-buffered LDS. Per tile: S^T = K Q^T, P^T = exp(s - lse),
// dP^T = V dO^T, dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T (K read
// transposed in the dS^T k-slot order). As in the reference's scoreGradients
// (src/shaders/ops/attention_coop.slang:283-305), P and dS are formed in
// float32 and rounded to the dtype for their products. Without a bias and away
// from the sequence end and the causal diagonal, P is one fma and one exp2 of
// the raw product (scale*log2(e) and lse*log2(e) folded in).
template <int DT, int D, bool CAUSAL, bool BIAS, int QPW>
__global__ __launch_bounds__(64 * AT_WAVES) void attn_bwd_dq_kernel(AttnBwdArgs p) {
    constexpr int BMQ = 16 * QPW * AT_WAVES;
    constexpr int DS = D / 32, DT16 = D / 16, LDK = D + 8;
    constexpr int CH = AT_BN * D / 8, CPT = CH / (64 * AT_WAVES);
    __shared__ __attribute__((aligned(16))) uint16_t ks[2][AT_BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t vs[2][AT_BN * LDK];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int g = lane / 16, c16 = lane % 16;
    int qb, bh;
    attn_block<CAUSAL>(p, qb, bh);
    const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
    const int q0 = qb * BMQ + wave * 16 * QPW;
    const uint16_t* Q = p.q + (int64_t)b * p.sq[0] + (int64_t)h * p.sq[1];
    const uint16_t* K = p.k + (int64_t)b * p.sk[0] + (int64_t)hk * p.sk[1];
    const uint16_t* V = p.v + (int64_t)b * p.sv[0] + (int64_t)hk * p.sv[1];
    const uint16_t* O = p.out + (int64_t)b * p.so[0] + (int64_t)h * p.so[1];
    const uint16_t* dO = p.dout + (int64_t)b * p.sdo[0] + (int64_t)h * p.sdo[1];

    int ntiles = (p.S + AT_BN - 1) / AT_BN;
    if (CAUSAL) {
        const int last_q = min(p.L, qb * BMQ + BMQ) - 1;
        ntiles = min(ntiles, last_q / AT_BN + 1);
    }
    u32x4 kreg[CPT], vreg[CPT];
    auto load_tile = [&](int j) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 64 * AT_WAVES;
            const int key = c / (D / 8), d8 = (c % (D / 8)) * 8;
            const int kj = j * AT_BN + key;
            kreg[i] = kj < p.S ? *reinterpret_cast<const u32x4*>(K + (int64_t)kj * p.sk[2] + d8) : u32x4{0, 0, 0, 0};
            vreg[i] = kj < p.S ? *reinterpret_cast<const u32x4*>(V + (int64_t)kj * p.sv[2] + d8) : u32x4{0, 0, 0, 0};
        }
    };
    // the first key tile is requested before the query side: its latency then
    // overlaps the q / dout / out loads and delta (the delta store would
    // otherwise keep the compiler from issuing these loads earlier)
    if (ntiles > 0) load_tile(0);

    u32x4 qf[QPW][DS], df[QPW][DS];
    float lse[QPW], lse2[QPW], dlt[QPW];
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) {
        const int qi = q0 + 16 * qt + c16;
        const bool in = qi < p.L;
        float part = 0.0f;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const int d0 = 32 * ds + 8 * g;
            qf[qt][ds] = in ? *reinterpret_cast<const u32x4*>(Q + (int64_t)qi * p.sq[2] + d0) : u32x4{0, 0, 0, 0};
            df[qt][ds] = in ? *reinterpret_cast<const u32x4*>(dO + (int64_t)qi * p.sdo[2] + d0) : u32x4{0, 0, 0, 0};
            if (in) {
                uint16_t ob[8];
                if (p.o_vec) {
                    const u32x4 ow = *reinterpret_cast<const u32x4*>(O + (int64_t)qi * p.so[2] + d0);
#pragma unroll
                    for (int e = 0; e < 8; ++e) ob[e] = (uint16_t)(ow[e / 2] >> (16 * (e % 2)));
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) ob[e] = O[(int64_t)qi * p.so[2] + (int64_t)(d0 + e) * p.so[3]];
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint16_t db = (uint16_t)(df[qt][ds][e / 2] >> (16 * (e % 2)));
                    part += elem<DT>::to_f32(__builtin_bit_cast(typename elem<DT>::T, db)) *
                            elem<DT>::to_f32(__builtin_bit_cast(typename elem<DT>::T, ob[e]));
                }
            }
        }
        dlt[qt] = lanes4_sum(part);
        lse[qt] = in ? p.lse[(int64_t)b * p.sl[0] + (int64_t)h * p.sl[1] + (int64_t)qi * p.sl[2]] : INFINITY;
        lse2[qt] = lse[qt] * AT_LOG2E;
        if (in && g == 0) p.delta[((int64_t)b * p.Hq + h) * p.L + qi] = dlt[qt];
    }

    f32x4 acc[DT16][QPW];
#pragma unroll
    for (int i = 0; i < DT16; ++i)
#pragma unroll
        for (int qt = 0; qt < QPW; ++qt) acc[i][qt] = f32x4{0, 0, 0, 0};

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 64 * AT_WAVES;
            const int key = c / (D / 8), d8 = (c % (D / 8)) * 8;
            *reinterpret_cast<u32x4*>(&ks[buf][key * LDK + d8]) = kreg[i];
            *reinterpret_cast<u32x4*>(&vs[buf][key * LDK + d8]) = vreg[i];
        }
    };
    if (ntiles > 0) store_tile(0);
    __syncthreads();

    for (int j = 0; j < ntiles; ++j) {
        const int buf = j & 1;
        const int k0 = j * AT_BN;
        if (j + 1 < ntiles) load_tile(j + 1);
        // a causal wave whose queries all precede the tile has nothing to add
        if (!CAUSAL || k0 <= q0 + 16 * QPW - 1) {
            f32x4 sacc[4][QPW], pacc[4][QPW];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt) {
                    sacc[kt][qt] = f32x4{0, 0, 0, 0};
                    pacc[kt][qt] = f32x4{0, 0, 0, 0};
                }
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const u32x4 kf = *reinterpret_cast<const u32x4*>(&ks[buf][(kt * 16 + c16) * LDK + 32 * ds + 8 * g]);
                    const u32x4 vf = *reinterpret_cast<const u32x4*>(&vs[buf][(kt * 16 + c16) * LDK + 32 * ds + 8 * g]);
#pragma unroll
                    for (int qt = 0; qt < QPW; ++qt) {
                        sacc[kt][qt] = mfma16<DT>(kf, qf[qt][ds], sacc[kt][qt]);
                        pacc[kt][qt] = mfma16<DT>(vf, df[qt][ds], pacc[kt][qt]);
                    }
                }
            }
            // dS^T = P^T (dP^T - delta), P^T = exp(s - lse); masked entries give 0
            if (!BIAS && k0 + AT_BN <= p.S && !(CAUSAL && k0 + AT_BN - 1 > q0)) {
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt)
#pragma unroll
                    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][qt][r], p.c2, -lse2[qt]));
                            sacc[kt][qt][r] = pe * (pacc[kt][qt][r] - dlt[qt]);
                        }
            } else {
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt) {
                    const int qi = q0 + 16 * qt + c16;
#pragma unroll
                    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int kj = k0 + kt * 16 + 4 * g + r;
                            float s = sacc[kt][qt][r] * p.scale;
                            if (BIAS && kj < p.S && qi < p.L) {
                                const uint16_t bv = p.bias[(int64_t)b * p.sb[0] + (int64_t)h * p.sb[1] + (int64_t)qi * p.sb[2] + (int64_t)kj * p.sb[3]];
                                s = s + elem<DT>::to_f32(__builtin_bit_cast(typename elem<DT>::T, bv));
                            }
                            if (kj >= p.S || (CAUSAL && kj > qi)) s = -INFINITY;
                            // dS from the float32 P; only dS is rounded to the dtype (when packed)
                            const float pe = __builtin_amdgcn_exp2f((s - lse[qt]) * AT_LOG2E);
                            sacc[kt][qt][r] = pe * (pacc[kt][qt][r] - dlt[qt]);
                        }
                }
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                u32x4 sf[QPW];
#pragma unroll
                for (int qt = 0; qt < QPW; ++qt) {
                    const f32x4 a = sacc[2 * kk][qt], c = sacc[2 * kk + 1][qt];
                    sf[qt] = u32x4{pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]), pack2<DT>(c[2], c[3])};
                }
#pragma unroll
                for (int i = 0; i < DT16; ++i) {
                    const u32x4 kf = read_tr<LDK>(ks[buf], kk, i, g, c16);
#pragma unroll
                    for (int qt = 0; qt < QPW; ++qt) acc[i][qt] = mfma16<DT>(kf, sf[qt], acc[i][qt]);
                }
            }
        }
        if (j + 1 < ntiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    uint16_t* dQ = p.dq + (int64_t)b * p.sdq[0] + (int64_t)h * p.sdq[1];
#pragma unroll
    for (int qt = 0; qt < QPW; ++qt) {
        const int qi = q0 + 16 * qt + c16;
        if (qi >= p.L) continue;
#pragma unroll
        for (int i = 0; i < DT16; ++i) store4<DT>(dQ + (int64_t)qi * p.sdq[2] + 16 * i + 4 * g, acc[i][qt], p.scale);
    }
}

// dK / dV pass: one workgroup owns 4 waves x KPW x 16 keys of one (batch, kv
// head) per wave group. Small grids run two groups of 4 waves on 64 keys
// (head_dim 64; at 128 a second group would overflow the registers); large
// ones one group whose waves own two 16-key columns (128 keys), so each q and
// dout fragment read from LDS feeds twice the MFMAs (one column per wave
// leaves the pass bound by LDS reads). The query tiles (64 queries) of every
// head of the group form one list, and the wave groups take alternate
// entries, each through double-buffered LDS of its own (q, dout, lse, delta).
// Per tile: S = Q K^T (a lane owns one key), P = exp(s - lse),
// dP = dO V^T, dS = P (dP - delta), then dV^T += dO^T P and dK^T += Q^T dS
// with dO and Q read transposed in the k-slot order of the S accumulator. At
// the end the second group's partial dK and dV go through LDS and are added to
// the first group's, in that order. Causal workgroups are dealt heaviest
// first (the first keys see every query tile) with each (batch, kv head) on
// one XCD, as in the forward.
template <int D, int KPW>
constexpr int dkv_groups() { return D == 64 && KPW == 1 ? 2 : 1; }

template <int DT, int D, bool CAUSAL, bool BIAS, int KPW>
__global__ __launch_bounds__((64 * AT_WAVES * dkv_groups<D, KPW>())) void attn_bwd_dkv_kernel(AttnBwdArgs p) {
    constexpr int KW = AT_WAVES;
    constexpr int DKV_GROUPS = dkv_groups<D, KPW>();
    constexpr int KB = 16 * KPW * KW;   // keys per workgroup
    constexpr int DS = D / 32, DT16 = D / 16, LDK = D + 8;
    constexpr int QT = 64;   // queries per tile
    constexpr int NT = 64 * KW;   // threads of one wave group
    constexpr int CH = QT * D / 8, CPT = CH / NT;
    // tl[group][0 = q, 1 = dout][buffer]: one array, so that a group's tiles are
    // one contiguous region (the partial exchange below reuses group 1's)
    __shared__ __attribute__((aligned(16))) uint16_t tl[DKV_GROUPS][2][2][QT * LDK];
    __shared__ __attribute__((aligned(16))) float lses[DKV_GROUPS][2][QT];
    __shared__ __attribute__((aligned(16))) float dls[DKV_GROUPS][2][QT];
    static_assert(DKV_GROUPS == 1 || sizeof(tl[0]) >= KW * KPW * DT16 * 2 * 64 * sizeof(f32x4), "partials fit a group's tiles");

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int grp = wave / KW, kw = wave % KW, tg = tid % NT;
    const int g = lane / 16, c16 = lane % 16;
    int kblk, bhk;
    attn_block<CAUSAL>(p, kblk, bhk);
    if (CAUSAL) kblk = p.nqb - 1 - kblk;   // the heaviest key blocks are the first ones
    const int b = bhk / (p.Hq / p.group), hk = bhk % (p.Hq / p.group);
    const int kb0 = kblk * KB, kw0 = kb0 + kw * 16 * KPW;   // this wave's first key
    const uint16_t* K = p.k + (int64_t)b * p.sk[0] + (int64_t)hk * p.sk[1];
    const uint16_t* V = p.v + (int64_t)b * p.sv[0] + (int64_t)hk * p.sv[1];

    // kc-th 16-key column of the wave: lane key kw0 + 16 kc + c16
    u32x4 kf[KPW][DS], vf[KPW][DS];
#pragma unroll
    for (int kc = 0; kc < KPW; ++kc) {
        const int kj = kw0 + 16 * kc + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            kf[kc][ds] = kj < p.S ? *reinterpret_cast<const u32x4*>(K + (int64_t)kj * p.sk[2] + 32 * ds + 8 * g) : u32x4{0, 0, 0, 0};
            vf[kc][ds] = kj < p.S ? *reinterpret_cast<const u32x4*>(V + (int64_t)kj * p.sv[2] + 32 * ds + 8 * g) : u32x4{0, 0, 0, 0};
        }
    }
    f32x4 dka[KPW][DT16], dva[KPW][DT16];
#pragma unroll
    for (int kc = 0; kc < KPW; ++kc)
#pragma unroll
        for (int i = 0; i < DT16; ++i) {
            dka[kc][i] = f32x4{0, 0, 0, 0};
            dva[kc][i] = f32x4{0, 0, 0, 0};
        }

    // query tiles of all heads of the group; under the causal mask the tiles
    // wholly before this block's first key see none of its keys
    const int first_t = CAUSAL ? kb0 / QT : 0;
    const int per_head = max(0, (p.L + QT - 1) / QT - first_t);
    const int ntiles = p.group * per_head;
    const int nsteps = (ntiles + DKV_GROUPS - 1) / DKV_GROUPS;
    u32x4 qreg[CPT], dreg[CPT];
    float lreg = INFINITY, dreg1 = 0.0f;
    auto tile_pos = [&](int n, int& hq, int& t) {
        hq = hk * p.group + n / max(1, per_head);
        t = first_t + n % max(1, per_head);
    };
    auto load_tile = [&](int n) {
        if (n >= ntiles) return;
        int hq, t;
        tile_pos(n, hq, t);
        const uint16_t* Q = p.q + (int64_t)b * p.sq[0] + (int64_t)hq * p.sq[1];
        const uint16_t* dO = p.dout + (int64_t)b * p.sdo[0] + (int64_t)hq * p.sdo[1];
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tg + i * NT;
            const int row = c / (D / 8), d8 = (c % (D / 8)) * 8;
            const int qi = t * QT + row;
            qreg[i] = qi < p.L ? *reinterpret_cast<const u32x4*>(Q + (int64_t)qi * p.sq[2] + d8) : u32x4{0, 0, 0, 0};
            dreg[i] = qi < p.L ? *reinterpret_cast<const u32x4*>(dO + (int64_t)qi * p.sdo[2] + d8) : u32x4{0, 0, 0, 0};
        }
        if (tg < QT) {
            const int qi = t * QT + tg;
            // lse in log2 units; +inf past the last query gives P = 0 there
            lreg = qi < p.L ? p.lse[(int64_t)b * p.sl[0] + (int64_t)hq * p.sl[1] + (int64_t)qi * p.sl[2]] * AT_LOG2E : INFINITY;
            dreg1 = qi < p.L ? p.delta[((int64_t)b * p.Hq + hq) * p.L + qi] : 0.0f;
        }
    };
    auto store_tile = [&](int n, int buf) {
        if (n >= ntiles) return;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tg + i * NT;
            const int row = c / (D / 8), d8 = (c % (D / 8)) * 8;
            *reinterpret_cast<u32x4*>(&tl[grp][0][buf][row * LDK + d8]) = qreg[i];
            *reinterpret_cast<u32x4*>(&tl[grp][1][buf][row * LDK + d8]) = dreg[i];
        }
        if (tg < QT) {
            lses[grp][buf][tg] = lreg;
            dls[grp][buf][tg] = dreg1;
        }
    };
    load_tile(grp);
    store_tile(grp, 0);
    __syncthreads();

    for (int st = 0; st < nsteps; ++st) {
        const int buf = st & 1;
        const int n = st * DKV_GROUPS + grp;   // this group's tile
        load_tile(n + DKV_GROUPS);
        int hq = 0, t = 0;
        if (n < ntiles) tile_pos(n, hq, t);
        const int qt0 = t * QT;
        // nothing to add: no tile left for this group, or every key of the wave follows every query
        if (n < ntiles && !(CAUSAL && kw0 > qt0 + QT - 1)) {
            // S and dP: 4 blocks of 16 queries (rows) x the wave's KPW 16-key columns
            f32x4 sacc[4][KPW], pacc[4][KPW];
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
#pragma unroll
                for (int kc = 0; kc < KPW; ++kc) {
                    sacc[qt][kc] = f32x4{0, 0, 0, 0};
                    pacc[qt][kc] = f32x4{0, 0, 0, 0};
                }
#pragma unroll
                for (int ds = 0; ds < DS; ++ds) {
                    const u32x4 qa = *reinterpret_cast<const u32x4*>(&tl[grp][0][buf][(qt * 16 + c16) * LDK + 32 * ds + 8 * g]);
                    const u32x4 da = *reinterpret_cast<const u32x4*>(&tl[grp][1][buf][(qt * 16 + c16) * LDK + 32 * ds + 8 * g]);
#pragma unroll
                    for (int kc = 0; kc < KPW; ++kc) {
                        sacc[qt][kc] = mfma16<DT>(qa, kf[kc][ds], sacc[qt][kc]);
                        pacc[qt][kc] = mfma16<DT>(da, vf[kc][ds], pacc[qt][kc]);
                    }
                }
            }
            // P (rounded to the dtype when packed) into sacc, dS into pacc;
            // rows 4g..4g+3 of each 16-query block share one 16-byte LDS read
            const bool plain = !BIAS && kw0 + 16 * KPW - 1 < p.S && !(CAUSAL && kw0 + 16 * KPW - 1 > qt0);
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
                const f32x4 l4 = *reinterpret_cast<const f32x4*>(&lses[grp][buf][qt * 16 + 4 * g]);
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dls[grp][buf][qt * 16 + 4 * g]);
#pragma unroll
                for (int kc = 0; kc < KPW; ++kc) {
                    const int kj = kw0 + 16 * kc + c16;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x;
                        if (plain) {
                            x = __builtin_fmaf(sacc[qt][kc][r], p.c2, -l4[r]);
                        } else {
                            const int qi = qt0 + qt * 16 + 4 * g + r;
                            float s = sacc[qt][kc][r] * p.scale;
                            if (BIAS && kj < p.S && qi < p.L) {
                                const uint16_t bv = p.bias[(int64_t)b * p.sb[0] + (int64_t)hq * p.sb[1] + (int64_t)qi * p.sb[2] + (int64_t)kj * p.sb[3]];
                                s = s + elem<DT>::to_f32(__builtin_bit_cast(typename elem<DT>::T, bv));
                            }
                            if (kj >= p.S || (CAUSAL && kj > qi)) s = -INFINITY;
                            x = s * AT_LOG2E - l4[r];
                        }
                        // P and dS from the float32 P; each is rounded to the dtype when packed
                        const float pe = __builtin_amdgcn_exp2f(x);
                        sacc[qt][kc][r] = pe;
                        pacc[qt][kc][r] = pe * (pacc[qt][kc][r] - d4[r]);
                    }
                }
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                u32x4 pf[KPW], sf[KPW];
#pragma unroll
                for (int kc = 0; kc < KPW; ++kc) {
                    const f32x4 a = sacc[2 * kk][kc], c = sacc[2 * kk + 1][kc];
                    pf[kc] = u32x4{pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]), pack2<DT>(c[2], c[3])};
                    const f32x4 e = pacc[2 * kk][kc], f = pacc[2 * kk + 1][kc];
                    sf[kc] = u32x4{pack2<DT>(e[0], e[1]), pack2<DT>(e[2], e[3]), pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3])};
                }
#pragma unroll
                for (int i = 0; i < DT16; ++i) {
                    const u32x4 dot = read_tr<LDK>(tl[grp][1][buf], kk, i, g, c16);
                    const u32x4 qtr = read_tr<LDK>(tl[grp][0][buf], kk, i, g, c16);
#pragma unroll
                    for (int kc = 0; kc < KPW; ++kc) {
                        dva[kc][i] = mfma16<DT>(dot, pf[kc], dva[kc][i]);
                        dka[kc][i] = mfma16<DT>(qtr, sf[kc], dka[kc][i]);
                    }
                }
            }
        }
        // buffer buf^1 was last read in step st-1, which every wave left through the barrier below
        store_tile(n + DKV_GROUPS, buf ^ 1);
        __syncthreads();
    }

    if constexpr (DKV_GROUPS == 2) {
        // second group's partials through LDS (its tile buffers are free now), added in group order
        f32x4* part = reinterpret_cast<f32x4*>(&tl[1][0][0][0]);
        if (grp == 1) {
#pragma unroll
            for (int kc = 0; kc < KPW; ++kc)
#pragma unroll
                for (int i = 0; i < DT16; ++i) {
                    part[(((kw * KPW + kc) * DT16 + i) * 2 + 0) * 64 + lane] = dka[kc][i];
                    part[(((kw * KPW + kc) * DT16 + i) * 2 + 1) * 64 + lane] = dva[kc][i];
                }
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int kc = 0; kc < KPW; ++kc)
#pragma unroll
            for (int i = 0; i < DT16; ++i) {
                dka[kc][i] += part[(((kw * KPW + kc) * DT16 + i) * 2 + 0) * 64 + lane];
                dva[kc][i] += part[(((kw * KPW + kc) * DT16 + i) * 2 + 1) * 64 + lane];
            }
    }
#pragma unroll
    for (int kc = 0; kc < KPW; ++kc) {
        const int kj = kw0 + 16 * kc + c16;
        if (kj >= p.S) continue;
        uint16_t* dK = p.dk + (int64_t)b * p.sdk[0] + (int64_t)hk * p.sdk[1] + (int64_t)kj * p.sdk[2];
        uint16_t* dV = p.dv + (int64_t)b * p.sdv[0] + (int64_t)hk * p.sdv[1] + (int64_t)kj * p.sdv[2];
#pragma unroll
        for (int i = 0; i < DT16; ++i) {
            store4<DT>(dK + 16 * i + 4 * g, dka[kc][i], p.scale);
            store4<DT>(dV + 16 * i + 4 * g, dva[kc][i], 1.0f);
        }
    }
}


template <int DT, int D, bool C, bool B>
void launch_attn_bwd_cb(AttnBwdArgs a, int64_t batch, int64_t heads, int64_t L, int64_t S, hipStream_t s) {
    const dim3 block(64 * AT_WAVES);
    if (L > 0) {
        a.BH = (int)(batch * heads);
        // query columns per wave as in the forward: two at head_dim 64 on large grids
        bool two = false;
        if constexpr (D == 64) two = batch * heads * ((L + 127) / 128) >= 2048;
        if (two) {
            a.nqb = (int)((L + 127) / 128);
            hipLaunchKernelGGL((attn_bwd_dq_kernel<DT, D, C, B, 2>), dim3((unsigned)(a.nqb * a.BH)), block, 0, s, a);
        } else {
            a.nqb = (int)((L + 63) / 64);
            hipLaunchKernelGGL((attn_bwd_dq_kernel<DT, D, C, B, 1>), dim3((unsigned)(a.nqb * a.BH)), block, 0, s, a);
        }
    }
    if (S > 0) {
        // workgroups dealt by attn_block: nqb = key blocks per (batch, kv head), BH = batch * kv heads
        a.BH = (int)(batch * heads / a.group);
        bool wide = false;
        if constexpr (D == 64) {
            if ((int64_t)a.BH * ((S + 127) / 128) >= 512) {
                wide = true;
                a.nqb = (int)((S + 127) / 128);
                hipLaunchKernelGGL((attn_bwd_dkv_kernel<DT, D, C, B, 2>), dim3((unsigned)(a.nqb * a.BH)), dim3(64 * AT_WAVES), 0, s, a);
            }
        }
        if (!wide) {
            a.nqb = (int)((S + 63) / 64);
            hipLaunchKernelGGL((attn_bwd_dkv_kernel<DT, D, C, B, 1>), dim3((unsigned)(a.nqb * a.BH)),
                               dim3(64 * AT_WAVES * dkv_groups<D, 1>()), 0, s, a);
        }
    }
}

template <int DT, int D>
void launch_attn_bwd(const AttnBwdArgs& a, bool causal, bool bias, int64_t batch, int64_t heads, int64_t L, int64_t S,
                     hipStream_t s) {
    if (causal) {
        if (bias) launch_attn_bwd_cb<DT, D, true, true>(a, batch, heads, L, S, s);
        else launch_attn_bwd_cb<DT, D, true, false>(a, batch, heads, L, S, s);
    } else {
        if (bias) launch_attn_bwd_cb<DT, D, false, true>(a, batch, heads, L, S, s);
        else launch_attn_bwd_cb<DT, D, false, false>(a, batch, heads, L, S, s);
    }
}

}  // namespace
}  // namespace tvk

using namespace tvk;

namespace {

// The MFMA forward (float16/bfloat16, head dims 64/128, 16-byte rows);
// TVK_ERR_UNSUPPORTED when the case is not one it takes.
tvk_status fused_fwd(const tvk_attention_desc* d) {
    if (d->dtype != TVK_F16 && d->dtype != TVK_BF16)
        return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: dtype must be float16 or bfloat16");
    if (d->batch < 0 || d->heads_q < 0 || d->heads_kv <= 0 || d->len_q < 0 || d->len_kv < 0)
        return fail(TVK_ERR_INVALID, "tvk_attention_fwd: negative size");
    if (d->heads_q % d->heads_kv != 0)
        return fail(TVK_ERR_INVALID, "tvk_attention_fwd: heads_q is not a multiple of heads_kv");
    if (d->head_dim != d->head_dim_v || (d->head_dim != 64 && d->head_dim != 128))
        return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: head_dim == head_dim_v in {64, 128} only");
    if (d->len_q > ((int64_t)1 << 30) || d->len_kv > ((int64_t)1 << 30) ||
        d->batch * d->heads_q * ((d->len_q + 63) / 64) > (int64_t)0x7fffffff)
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
    // a key tile's rows are addressed by 32-bit byte offsets from the tile's first row
    for (const int64_t row : {d->k_stride[2], d->v_stride[2]})
        if (row < 0 || (63 * row + d->head_dim) * 2 > (int64_t)0xffffffff)
            return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: k or v row stride too large");
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
    a.c2 = std::fabs(a.scale) * AT_LOG2E;
    a.qflip = a.scale < 0.0f ? 0x80008000u : 0u;
    const bool causal = d->causal != 0;
    a.out_vec = d->out_stride[3] == 1 && (reinterpret_cast<uintptr_t>(d->out) & 7) == 0 && d->out_stride[2] % 4 == 0 &&
                d->out_stride[1] % 4 == 0 && d->out_stride[0] % 4 == 0;
    const hipStream_t s = resolve_stream(d->stream);
    const bool bias = d->bias != nullptr;
    if (d->dtype == TVK_F16) {
        if (d->head_dim == 64) launch_attn<TVK_F16, 64>(a, causal, bias, d->batch, d->heads_q, d->len_q, s);
        else launch_attn<TVK_F16, 128>(a, causal, bias, d->batch, d->heads_q, d->len_q, s);
    } else {
        if (d->head_dim == 64) launch_attn<TVK_BF16, 64>(a, causal, bias, d->batch, d->heads_q, d->len_q, s);
        else launch_attn<TVK_BF16, 128>(a, causal, bias, d->batch, d->heads_q, d->len_q, s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_attention_fwd: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status check_attention(const tvk_attention_desc* d, const char* who) {
    auto bad = [&](tvk_status st, const char* m) { return fail(st, std::string(who) + ": " + m); };
    if (d->dtype != TVK_F16 && d->dtype != TVK_BF16) return bad(TVK_ERR_UNSUPPORTED, "dtype must be float16 or bfloat16");
    if (d->batch < 0 || d->heads_q < 0 || d->heads_kv <= 0 || d->len_q < 0 || d->len_kv < 0) return bad(TVK_ERR_INVALID, "negative size");
    if (d->heads_q % d->heads_kv != 0) return bad(TVK_ERR_INVALID, "heads_q is not a multiple of heads_kv");
    if (d->head_dim != d->head_dim_v || (d->head_dim != 64 && d->head_dim != 128))
        return bad(TVK_ERR_UNSUPPORTED, "head_dim == head_dim_v in {64, 128} only");
    if (d->batch > 65535 || d->heads_q > 65535 || d->len_q > ((int64_t)1 << 30) || d->len_kv > ((int64_t)1 << 30) ||
        d->batch * d->heads_q * ((d->len_q + 63) / 64) > (int64_t)0x7fffffff)
        return bad(TVK_ERR_UNSUPPORTED, "grid too large");
    return TVK_OK;
}

bool rows_ok(const void* ptr, const int64_t* st) {
    if ((reinterpret_cast<uintptr_t>(ptr) & 15) != 0 || st[3] != 1) return false;
    for (int i = 0; i < 3; ++i)
        if (st[i] % 8 != 0) return false;
    return true;
}

// The MFMA backward passes; TVK_ERR_UNSUPPORTED when the case is not one they take.
tvk_status fused_bwd(const tvk_attention_bwd_desc* desc) {
    const tvk_attention_desc* d = &desc->fwd;
    tvk_status st = check_attention(d, "tvk_attention_bwd");
    if (st != TVK_OK) return st;
    if (d->batch == 0 || d->heads_q == 0 || (d->len_q == 0 && d->len_kv == 0)) return TVK_OK;
    if (!d->q || !d->k || !d->v || !d->out || !d->lse || !desc->dout || !desc->dq || !desc->dk || !desc->dv)
        return fail(TVK_ERR_INVALID, "tvk_attention_bwd: NULL tensor");
    if (!rows_ok(d->q, d->q_stride) || !rows_ok(d->k, d->k_stride) || !rows_ok(d->v, d->v_stride) ||
        !rows_ok(desc->dout, desc->dout_stride) || !rows_ok(desc->dq, desc->dq_stride) ||
        !rows_ok(desc->dk, desc->dk_stride) || !rows_ok(desc->dv, desc->dv_stride))
        return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_bwd: q, k, v, dout, dq, dk, dv need unit stride along the head dimension and 16-byte aligned rows");
    AttnBwdArgs a{};
    a.q = static_cast<const uint16_t*>(d->q);
    a.k = static_cast<const uint16_t*>(d->k);
    a.v = static_cast<const uint16_t*>(d->v);
    a.bias = static_cast<const uint16_t*>(d->bias);
    a.out = static_cast<const uint16_t*>(d->out);
    a.dout = static_cast<const uint16_t*>(desc->dout);
    a.lse = d->lse;
    a.dq = static_cast<uint16_t*>(desc->dq);
    a.dk = static_cast<uint16_t*>(desc->dk);
    a.dv = static_cast<uint16_t*>(desc->dv);
    for (int i = 0; i < 4; ++i) {
        a.sq[i] = d->q_stride[i];
        a.sk[i] = d->k_stride[i];
        a.sv[i] = d->v_stride[i];
        a.sb[i] = d->bias ? d->bias_stride[i] : 0;
        a.so[i] = d->out_stride[i];
        a.sdo[i] = desc->dout_stride[i];
        a.sdq[i] = desc->dq_stride[i];
        a.sdk[i] = desc->dk_stride[i];
        a.sdv[i] = desc->dv_stride[i];
    }
    for (int i = 0; i < 3; ++i) a.sl[i] = d->lse_stride[i];
    a.L = (int)d->len_q;
    a.S = (int)d->len_kv;
    a.Hq = (int)d->heads_q;
    a.group = (int)(d->heads_q / d->heads_kv);
    a.scale = (float)d->scale;
    a.c2 = a.scale * AT_LOG2E;
    a.o_vec = rows_ok(d->out, d->out_stride) ? 1 : 0;
    const hipStream_t s = resolve_stream(d->stream);
    Scratch scratch;
    a.delta = static_cast<float*>(scratch.get((size_t)std::max<int64_t>(1, d->batch * d->heads_q * d->len_q) * 4, s));
    if (!a.delta) return fail(TVK_ERR_OOM, "tvk_attention_bwd: workspace allocation failed");
    const bool bias = d->bias != nullptr;
    if (d->dtype == TVK_F16) {
        if (d->head_dim == 64) launch_attn_bwd<TVK_F16, 64>(a, d->causal != 0, bias, d->batch, d->heads_q, d->len_q, d->len_kv, s);
        else launch_attn_bwd<TVK_F16, 128>(a, d->causal != 0, bias, d->batch, d->heads_q, d->len_q, d->len_kv, s);
    } else {
        if (d->head_dim == 64) launch_attn_bwd<TVK_BF16, 64>(a, d->causal != 0, bias, d->batch, d->heads_q, d->len_q, d->len_kv, s);
        else launch_attn_bwd<TVK_BF16, 128>(a, d->causal != 0, bias, d->batch, d->heads_q, d->len_q, d->len_kv, s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_attention_bwd: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

// Validation shared by both directions: every case that passes runs on the
// device, in the MFMA kernels when they take it, else in the general kernels
// of attention_any.hip.
tvk_status check_any(const tvk_attention_desc* d, const char* who) {
    auto bad = [&](tvk_status st, const std::string& m) { return fail(st, std::string(who) + ": " + m); };
    if (d->dtype != TVK_F32 && d->dtype != TVK_F16 && d->dtype != TVK_BF16)
        return bad(TVK_ERR_UNSUPPORTED, "dtype must be float32, float16 or bfloat16");
    if (d->batch < 0 || d->heads_q < 0 || d->heads_kv <= 0 || d->len_q < 0 || d->len_kv < 0 || d->head_dim < 0 ||
        d->head_dim_v < 0)
        return bad(TVK_ERR_INVALID, "negative size");
    if (d->heads_q % d->heads_kv != 0) return bad(TVK_ERR_INVALID, "heads_q is not a multiple of heads_kv");
    if (!attn_any_applies(d))
        return bad(TVK_ERR_UNSUPPORTED, "head dims above 512, or batch or heads above 65535, or sequences above 2^30");
    return TVK_OK;
}

}  // namespace

extern "C" tvk_status tvk_attention_fwd(const tvk_attention_desc* d) {
    if (!d) return fail(TVK_ERR_INVALID, "tvk_attention_fwd: desc is NULL");
    tvk_status st = check_any(d, "tvk_attention_fwd");
    if (st != TVK_OK) return st;
    if (d->batch == 0 || d->heads_q == 0 || d->len_q == 0) return TVK_OK;
    if (!d->q || !d->k || !d->v || !d->out || !d->lse) return fail(TVK_ERR_INVALID, "tvk_attention_fwd: NULL tensor");
    if (d->head_dim == 0 && d->len_kv > 0) return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_fwd: empty head dim");
    st = fused_fwd(d);
    if (st != TVK_ERR_UNSUPPORTED) return st;
    clear_error();
    return attn_any_fwd(d, resolve_stream(d->stream));
}

extern "C" tvk_status tvk_attention_bwd(const tvk_attention_bwd_desc* desc) {
    if (!desc) return fail(TVK_ERR_INVALID, "tvk_attention_bwd: desc is NULL");
    const tvk_attention_desc* d = &desc->fwd;
    tvk_status st = check_any(d, "tvk_attention_bwd");
    if (st != TVK_OK) return st;
    if (d->batch == 0 || d->heads_q == 0 || (d->len_q == 0 && d->len_kv == 0)) return TVK_OK;
    if (!d->q || !d->k || !d->v || !d->out || !d->lse || !desc->dout || !desc->dq || !desc->dk || !desc->dv)
        return fail(TVK_ERR_INVALID, "tvk_attention_bwd: NULL tensor");
    if (d->head_dim == 0 || d->head_dim_v == 0) return fail(TVK_ERR_UNSUPPORTED, "tvk_attention_bwd: empty head dim");
    if (!desc->dscores) {
        st = fused_bwd(desc);
        if (st != TVK_ERR_UNSUPPORTED) return st;
        clear_error();
    }
    const hipStream_t s = resolve_stream(d->stream);
    Scratch scratch;
    float* delta = static_cast<float*>(scratch.get((size_t)std::max<int64_t>(1, d->batch * d->heads_q * d->len_q) * 4, s));
    if (!delta) return fail(TVK_ERR_OOM, "tvk_attention_bwd: workspace allocation failed");
    return attn_any_bwd(desc, delta, s);
}
