// Convolution as implicit GEMM on gfx950: forward, grad-input and
// grad-weight, NC(D)HW, 2 or 3 spatial dimensions, any stride / padding /
// dilation / groups.
//
// Reference semantics (file:line under the reference tree):
//   forward     y[n, g*Cy+m, o] = sum_{c,tap} W[g*Cy+m, c, tap] x[n, g*Cx+c, o*s-p+tap*d]
//               + bias, zero padding; GEMM M = Cy, N = n*prod(out), K = Cx*taps with
//               k = (c, [kd,] kh, kw) (src/shaders/helpers/conv.slang:93-117,198-207,
//               280-312, src/api/ops/conv.cpp:1014-1022, bias epilogue conv_simd.slang:8-19)
//   grad input  dx[n, g*Cx+c, i] = sum_{m,tap} W[g*Cy+m, c, tap] dy[n, g*Cy+m, (i+p-tap*d)/s]
//               where the division is exact and in range; M = Cx, N = n*prod(in),
//               K = Cy*taps (conv.slang:320-362, conv.cpp:1024-1032)
//   grad weight dW[g*Cy+m, c, tap] = sum_{n,o} dy[n, g*Cy+m, o] x[n, g*Cx+c, o*s-p+tap*d];
//               M = Cy, N = Cx*taps, K = n*prod(out), K split into float32 partials that
//               are summed and cast to the storage type (conv.cpp:1034-1060)
// The reference takes up to three spatial dimensions (conv.cpp:295-311); its
// geometry block pads the shapes to three (conv.cpp:313-343). Here the 2-D and
// 3-D kernels are separate instantiations (ND), so the 2-D gathers carry no
// depth arithmetic; one spatial dimension runs as 2-D with a height of 1.
//
// Both operands of every mode are gathered element by element (buffer loads
// whose out-of-range offset reads zero, which is the padding) into LDS tiles
// laid out k-contiguous, the layout the GEMM kernels' MFMA fragments read.
// Each thread gathers 8 consecutive k of one GEMM row or column; the column
// decompositions are computed once per tile and the k decompositions are
// wave-uniform, so the inner gather is an add, two (three) range tests and a
// load. float16/bfloat16 use v_mfma_f32_32x32x16; float32 (and
// TVK_GEMM_EXACT) use the rank-1 v_mfma_f32_32x32x1f32 so every output
// accumulates in k order.
#include "gemm_common.h"
#include "tune_table.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace tvk {
namespace {

enum { FWD = 0, DGRAD = 1, WGRAD = 2 };
static_assert(FWD == 0 && DGRAD == 1 && WGRAD == 2, "mode numbers shared with conv_nhwc.hip");

struct ConvArgs {
    const void* x;
    const void* w;
    const void* bias;
    const void* y;
    void* out;      // y (FWD), x (DGRAD), w (WGRAD)
    float* part;    // WGRAD float32 partials [split][Cout][Cx*taps] when split > 1
    int n, cin, h, wd, cout, kh, kw, sh, sw, ph, pw, dh, dw, groups, ho, wo;
    int dp, kd, sd, pd, dd, dop;   // depth: input, kernel, stride, padding, dilation, output (3-D only)
    int si, so;                    // spatial elements per channel: input, output
    int cx, cy, taps;
    int M, N, K;
    int k_chunk;    // WGRAD: k per split
    int split;
    int has_bias;
    int x_bytes, w_bytes, y_bytes;
};

constexpr int C_BK = 32;   // k per LDS stage
constexpr int C_BN = 128;  // GEMM columns per block

// ---------------------------------------------------------------------------
// gathers
// ---------------------------------------------------------------------------

// Per-row (A) or per-column (B) part of an element address, fixed for the tile.
struct Lane {
    int base;       // element offset of the (row, k = 0) origin
    int db, hb, wb; // spatial offsets (meaning depends on mode; db only in 3-D)
    bool ok;        // the row/column exists
};

// k decomposition, wave-uniform; advanced by one k at a time.
struct KPos {
    int a, z, b, c;   // FWD B / DGRAD A,B: (channel, kd, kh, kw); WGRAD A,B: (n, od, oh, ow)
};

template <int ND, int MODE, bool IS_A>
__device__ inline Lane lane_info(const ConvArgs& p, int g, int idx) {
    Lane L{0, 0, 0, 0, false};
    if constexpr (IS_A) {
        if (idx >= p.M) return L;
        L.ok = true;
        if constexpr (MODE == FWD) L.base = (g * p.cy + idx) * p.cx * p.taps;                 // W row
        else if constexpr (MODE == DGRAD) L.base = (g * p.cy * p.cx + idx) * p.taps;         // W[g*Cy][c]
        else L.base = (g * p.cy + idx) * p.so;                                               // dy[0][g*Cy+m]
    } else {
        if (idx >= p.N) return L;
        L.ok = true;
        if constexpr (MODE == FWD) {
            const int o = idx % p.so, n = idx / p.so;
            const int plane = ND == 3 ? o % (p.ho * p.wo) : o;
            L.base = (n * p.cin + g * p.cx) * p.si;
            if constexpr (ND == 3) L.db = (o / (p.ho * p.wo)) * p.sd - p.pd;
            L.hb = (plane / p.wo) * p.sh - p.ph;
            L.wb = (plane % p.wo) * p.sw - p.pw;
        } else if constexpr (MODE == DGRAD) {
            const int o = idx % p.si, n = idx / p.si;
            const int plane = ND == 3 ? o % (p.h * p.wd) : o;
            L.base = (n * p.cout + g * p.cy) * p.so;
            if constexpr (ND == 3) L.db = o / (p.h * p.wd) + p.pd;
            L.hb = plane / p.wd + p.ph;
            L.wb = plane % p.wd + p.pw;
        } else {
            const int t = idx % p.taps, c = idx / p.taps;
            const int tp = ND == 3 ? t % (p.kh * p.kw) : t;
            L.base = (g * p.cx + c) * p.si;
            if constexpr (ND == 3) L.db = (t / (p.kh * p.kw)) * p.dd - p.pd;
            L.hb = (tp / p.kw) * p.dh - p.ph;
            L.wb = (tp % p.kw) * p.dw - p.pw;
        }
    }
    return L;
}

template <int ND, int MODE, bool IS_A>
__device__ inline KPos kpos_of(const ConvArgs& p, int k) {
    KPos q{0, 0, 0, 0};
    if constexpr (MODE == WGRAD) {
        const int o = k % p.so;
        const int plane = ND == 3 ? o % (p.ho * p.wo) : o;
        q.a = k / p.so;
        if constexpr (ND == 3) q.z = o / (p.ho * p.wo);
        q.b = plane / p.wo;
        q.c = plane % p.wo;
    } else if constexpr (!(IS_A && MODE == FWD)) {
        const int t = k % p.taps;
        const int tp = ND == 3 ? t % (p.kh * p.kw) : t;
        q.a = k / p.taps;
        if constexpr (ND == 3) q.z = t / (p.kh * p.kw);
        q.b = tp / p.kw;
        q.c = tp % p.kw;
    } else {
        q.a = k;
    }
    return q;
}

template <int ND, int MODE, bool IS_A>
__device__ inline void kpos_next(const ConvArgs& p, KPos& q) {
    if constexpr (MODE == WGRAD) {
        if (++q.c == p.wo) {
            q.c = 0;
            if (++q.b == p.ho) {
                q.b = 0;
                if constexpr (ND == 3) {
                    if (++q.z == p.dop) { q.z = 0; ++q.a; }
                } else {
                    ++q.a;
                }
            }
        }
    } else if constexpr (!(IS_A && MODE == FWD)) {
        if (++q.c == p.kw) {
            q.c = 0;
            if (++q.b == p.kh) {
                q.b = 0;
                if constexpr (ND == 3) {
                    if (++q.z == p.kd) { q.z = 0; ++q.a; }
                } else {
                    ++q.a;
                }
            }
        }
    } else {
        ++q.a;
    }
}

// Element offset (in elements) of operand element (row/col lane L, k = q), or
// -1 when it is padding / out of range.
template <int ND, int MODE, bool IS_A>
__device__ inline int elem_offset(const ConvArgs& p, const Lane& L, const KPos& q, bool kvalid) {
    if (!L.ok || !kvalid) return -1;
    if constexpr (IS_A) {
        const int tap = ND == 3 ? (q.z * p.kh + q.b) * p.kw + q.c : q.b * p.kw + q.c;
        const int opix = ND == 3 ? (q.z * p.ho + q.b) * p.wo + q.c : q.b * p.wo + q.c;
        if constexpr (MODE == FWD) return L.base + q.a;
        else if constexpr (MODE == DGRAD) return L.base + q.a * p.cx * p.taps + tap;
        else return L.base + q.a * p.cout * p.so + opix;
    } else {
        if constexpr (MODE == FWD) {
            const int ih = L.hb + q.b * p.dh, iw = L.wb + q.c * p.dw;
            if ((unsigned)ih >= (unsigned)p.h || (unsigned)iw >= (unsigned)p.wd) return -1;
            if constexpr (ND == 3) {
                const int id = L.db + q.z * p.dd;
                if ((unsigned)id >= (unsigned)p.dp) return -1;
                return L.base + q.a * p.si + (id * p.h + ih) * p.wd + iw;
            }
            return L.base + q.a * p.si + ih * p.wd + iw;
        } else if constexpr (MODE == DGRAD) {
            const int th = L.hb - q.b * p.dh, tw = L.wb - q.c * p.dw;
            if (th < 0 || tw < 0) return -1;
            const int oh = th / p.sh, ow = tw / p.sw;
            if (oh * p.sh != th || ow * p.sw != tw || oh >= p.ho || ow >= p.wo) return -1;
            if constexpr (ND == 3) {
                const int td = L.db - q.z * p.dd;
                if (td < 0) return -1;
                const int od = td / p.sd;
                if (od * p.sd != td || od >= p.dop) return -1;
                return L.base + q.a * p.so + (od * p.ho + oh) * p.wo + ow;
            }
            return L.base + q.a * p.so + oh * p.wo + ow;
        } else {
            const int ih = q.b * p.sh + L.hb, iw = q.c * p.sw + L.wb;
            if ((unsigned)ih >= (unsigned)p.h || (unsigned)iw >= (unsigned)p.wd) return -1;
            if constexpr (ND == 3) {
                const int id = q.z * p.sd + L.db;
                if ((unsigned)id >= (unsigned)p.dp) return -1;
                return L.base + q.a * p.cin * p.si + (id * p.h + ih) * p.wd + iw;
            }
            return L.base + q.a * p.cin * p.si + ih * p.wd + iw;
        }
    }
}

// Gathers operand tiles of R rows x C_BK k: thread t owns row t % R and the
// k chunks (t / R) + (256 / R) * i of 8 elements each; the chunk index is
// wave-uniform (R is 64 or 128).
template <int DT, int ND, int MODE, bool IS_A, int R>
struct Gather {
    static constexpr int ES = DT == TVK_F32 ? 4 : 2;
    static constexpr int NCH = R * (C_BK / 8) / 256;
    Lane lane;
    uint32_t raw[NCH][8];

    __device__ inline void init(const ConvArgs& p, int g, int row0, int tid) {
        lane = lane_info<ND, MODE, IS_A>(p, g, row0 + tid % R);
    }

    __device__ inline void load(const ConvArgs& p, __amdgpu_buffer_rsrc_t rsrc, int k0, int kend, int tid) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int kc = __builtin_amdgcn_readfirstlane(tid / R + (256 / R) * i);
            const int kb = k0 + kc * 8;
            KPos q = kpos_of<ND, MODE, IS_A>(p, kb);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int off = elem_offset<ND, MODE, IS_A>(p, lane, q, kb + e < kend);
                const uint32_t bo = off < 0 ? kOOB : (uint32_t)off * ES;
                if constexpr (ES == 4) raw[i][e] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)bo, 0, 0);
                else raw[i][e] = buf_load2(rsrc, bo);
                kpos_next<ND, MODE, IS_A>(p, q);
            }
        }
    }

    // 16-bit storage: [R][LD] halfs
    template <int LD>
    __device__ inline void store16(uint16_t* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int kc = tid / R + (256 / R) * i;
            u32x4 v{raw[i][0] | (raw[i][1] << 16), raw[i][2] | (raw[i][3] << 16), raw[i][4] | (raw[i][5] << 16),
                    raw[i][6] | (raw[i][7] << 16)};
            *reinterpret_cast<u32x4*>(lds + (tid % R) * LD + kc * 8) = v;
        }
    }

    // float32 storage (operands widened exactly): [R][LD] floats
    template <int LD>
    __device__ inline void store32(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int kc = tid / R + (256 / R) * i;
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (DT == TVK_F32) f[e] = __builtin_bit_cast(float, raw[i][e]);
                else if constexpr (DT == TVK_F16) f[e] = (float)__builtin_bit_cast(half_t, (uint16_t)raw[i][e]);
                else f[e] = __builtin_bit_cast(float, raw[i][e] << 16);
            }
            float* d = lds + (tid % R) * LD + kc * 8;
            *reinterpret_cast<f32x4*>(d) = f32x4{f[0], f[1], f[2], f[3]};
            *reinterpret_cast<f32x4*>(d + 4) = f32x4{f[4], f[5], f[6], f[7]};
        }
    }
};

// ---------------------------------------------------------------------------
// epilogue: GEMM (row, col) of group g -> tensor element
// ---------------------------------------------------------------------------

template <int DT, int MODE>
__device__ inline void conv_store(const ConvArgs& p, int g, int split, int row, int col, float acc) {
    if (row >= p.M || col >= p.N) return;
    typedef typename elem<DT>::T T;
    if constexpr (MODE == FWD) {
        const int o = col % p.so, n = col / p.so;
        const int ch = g * p.cy + row;
        float v = acc;
        if (p.has_bias) {
#pragma clang fp contract(off)
            v = v + elem<DT>::to_f32(reinterpret_cast<const T*>(p.bias)[ch]);
        }
        reinterpret_cast<T*>(p.out)[(int64_t)(n * p.cout + ch) * p.so + o] = elem<DT>::from_f32(v);
    } else if constexpr (MODE == DGRAD) {
        const int o = col % p.si, n = col / p.si;
        reinterpret_cast<T*>(p.out)[(int64_t)(n * p.cin + g * p.cx + row) * p.si + o] = elem<DT>::from_f32(acc);
    } else {
        const int64_t idx = (int64_t)(g * p.cy + row) * p.cx * p.taps + col;
        if (p.split > 1) p.part[(int64_t)split * p.cout * p.cx * p.taps + idx] = acc;
        else reinterpret_cast<T*>(p.out)[idx] = elem<DT>::from_f32(acc);
    }
}

__device__ inline void block_coords(const ConvArgs& p, int& g, int& split, int& kbeg, int& kend) {
    g = blockIdx.z % p.groups;
    split = blockIdx.z / p.groups;
    kbeg = 0;
    kend = p.K;
    if (p.split > 1) {
        kbeg = split * p.k_chunk;
        kend = min(p.K, kbeg + p.k_chunk);
    }
}

template <int MODE>
__device__ inline void operand_rsrc(const ConvArgs& p, __amdgpu_buffer_rsrc_t& ra, __amdgpu_buffer_rsrc_t& rb) {
    const void* a = MODE == WGRAD ? p.y : p.w;
    const void* b = MODE == DGRAD ? p.y : p.x;
    const int ab = MODE == WGRAD ? p.y_bytes : p.w_bytes;
    const int bb = MODE == DGRAD ? p.y_bytes : p.x_bytes;
    ra = __builtin_amdgcn_make_buffer_rsrc((void*)a, 0, ab, 0x00020000);
    rb = __builtin_amdgcn_make_buffer_rsrc((void*)b, 0, bb, 0x00020000);
}

// ---------------------------------------------------------------------------
// float16 / bfloat16 kernel: v_mfma_f32_32x32x16, BM x 128 tile, 4 waves
// ---------------------------------------------------------------------------

constexpr int C_LDK = C_BK + 8;   // 80-byte rows: conflict-free 16-byte fragment reads

template <int DT>
__device__ inline f32x16 cmfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (DT == TVK_F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int DT, int ND, int MODE, int BM>
__global__ __launch_bounds__(256) void conv16_kernel(ConvArgs p) {
    constexpr int WGM = BM / 64;                 // waves along M (1 or 2)
    constexpr int WGN = 4 / WGM;                 // waves along N
    constexpr int WN = C_BN / WGN;               // wave tile 64 x WN
    constexpr int FM = 2, FN = WN / 32;
    __shared__ __attribute__((aligned(16))) uint16_t lds[2][(BM + C_BN) * C_LDK];

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / WGN, wn = wave % WGN;
    int g, split, kbeg, kend;
    block_coords(p, g, split, kbeg, kend);
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * C_BN;
    __amdgpu_buffer_rsrc_t ra, rb;
    operand_rsrc<MODE>(p, ra, rb);

    Gather<DT, ND, MODE, true, BM> ga;
    Gather<DT, ND, MODE, false, C_BN> gb;
    ga.init(p, g, m0, tid);
    gb.init(p, g, n0, tid);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = (kend - kbeg + C_BK - 1) / C_BK;
    ga.load(p, ra, kbeg, kend, tid);
    gb.load(p, rb, kbeg, kend, tid);
    ga.template store16<C_LDK>(lds[0], tid);
    gb.template store16<C_LDK>(lds[0] + BM * C_LDK, tid);
    __syncthreads();
    const int frag_row = lane % 32, frag_k = (lane / 32) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) {
            ga.load(p, ra, kbeg + (kt + 1) * C_BK, kend, tid);
            gb.load(p, rb, kbeg + (kt + 1) * C_BK, kend, tid);
        }
        const uint16_t* As = lds[buf];
        const uint16_t* Bs = lds[buf] + BM * C_LDK;
#pragma unroll
        for (int kk = 0; kk < C_BK; kk += 16) {
            u32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const u32x4*>(As + (wm * 64 + i * 32 + frag_row) * C_LDK + kk + frag_k);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const u32x4*>(Bs + (wn * WN + j * 32 + frag_row) * C_LDK + kk + frag_k);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = cmfma32<DT>(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < nk) {
            ga.template store16<C_LDK>(lds[buf ^ 1], tid);
            gb.template store16<C_LDK>(lds[buf ^ 1] + BM * C_LDK, tid);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * WN + j * 32 + lane % 32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + i * 32 + (r / 4) * 8 + (lane / 32) * 4 + (r % 4);
                conv_store<DT, MODE>(p, g, split, row, col, acc[i][j][r]);
            }
        }
}

// ---------------------------------------------------------------------------
// sequential-k kernel (float32, exact mode): v_mfma_f32_32x32x1f32, 128 x 128
// ---------------------------------------------------------------------------

constexpr int S_LDK = C_BK + 4;   // float rows of 144 bytes

template <int DT, int ND, int MODE>
__global__ __launch_bounds__(256) void conv_seq_kernel(ConvArgs p) {
    constexpr int BM = 128;
    __shared__ __attribute__((aligned(16))) float lds[2][(BM + C_BN) * S_LDK];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / 2, wn = wave % 2;
    int g, split, kbeg, kend;
    block_coords(p, g, split, kbeg, kend);
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * C_BN;
    __amdgpu_buffer_rsrc_t ra, rb;
    operand_rsrc<MODE>(p, ra, rb);

    Gather<DT, ND, MODE, true, BM> ga;
    Gather<DT, ND, MODE, false, C_BN> gb;
    ga.init(p, g, m0, tid);
    gb.init(p, g, n0, tid);

    f32x32 acc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 32; ++r) acc[i][r] = 0.0f;

    const int nk = (kend - kbeg + C_BK - 1) / C_BK;
    ga.load(p, ra, kbeg, kend, tid);
    gb.load(p, rb, kbeg, kend, tid);
    ga.template store32<S_LDK>(lds[0], tid);
    gb.template store32<S_LDK>(lds[0] + BM * S_LDK, tid);
    __syncthreads();
    const int arow = wm * 64 + lane % 32;
    const int bcol = wn * 64 + lane;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) {
            ga.load(p, ra, kbeg + (kt + 1) * C_BK, kend, tid);
            gb.load(p, rb, kbeg + (kt + 1) * C_BK, kend, tid);
        }
        const float* As = lds[buf];
        const float* Bs = lds[buf] + BM * S_LDK;
#pragma unroll
        for (int k4 = 0; k4 < C_BK; k4 += 4) {
            const f32x4 a0 = *reinterpret_cast<const f32x4*>(As + arow * S_LDK + k4);
            const f32x4 a1 = *reinterpret_cast<const f32x4*>(As + (arow + 32) * S_LDK + k4);
            const f32x4 bv = *reinterpret_cast<const f32x4*>(Bs + bcol * S_LDK + k4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(a0[q], bv[q], acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_32x32x1f32(a1[q], bv[q], acc[1], 0, 0, 0);
            }
        }
        if (kt + 1 < nk) {
            ga.template store32<S_LDK>(lds[buf ^ 1], tid);
            gb.template store32<S_LDK>(lds[buf ^ 1] + BM * S_LDK, tid);
        }
        __syncthreads();
    }
    // block r/16 of the rank-1 MFMA: row (rr/4)*8 + (lane/32)*4 + rr%4, column (r/16)*32 + lane%32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 32; ++r) {
            const int rr = r % 16;
            const int row = m0 + wm * 64 + 32 * i + (rr / 4) * 8 + (lane / 32) * 4 + rr % 4;
            const int col = n0 + wn * 64 + (r / 16) * 32 + lane % 32;
            conv_store<DT, MODE>(p, g, split, row, col, acc[i][r]);
        }
}

__global__ __launch_bounds__(256) void zero_fill_kernel(uint16_t* out, int64_t halfs) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < halfs; i += (int64_t)gridDim.x * 256) out[i] = 0;
}

// Sums the grad-weight partials over the splits and rounds once. Few outputs
// with many splits (the 3-channel stem: 1728 outputs of 512 partials) would
// leave a thread per output summing serially, so each output gets one wave:
// lane l sums splits l, l+64, ... in order, then the 64 lane sums are added
// by a fixed butterfly, so the result does not depend on timing.
template <int DT>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* part, void* out, int64_t count, int split) {
    typedef typename elem<DT>::T T;
    const int lane = threadIdx.x % 64;
    for (int64_t i = (int64_t)blockIdx.x * 4 + threadIdx.x / 64; i < count; i += (int64_t)gridDim.x * 4) {
        float v = 0.0f;
        for (int s = lane; s < split; s += 64) v += part[(int64_t)s * count + i];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
        if (lane == 0) reinterpret_cast<T*>(out)[i] = elem<DT>::from_f32(v);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

tvk_status check_dtype_flags(int32_t dtype, uint32_t flags, const std::string& w) {
    if (dtype != TVK_F32 && dtype != TVK_F16 && dtype != TVK_BF16)
        return fail(TVK_ERR_UNSUPPORTED, w + ": unsupported dtype " + std::to_string(dtype));
    if (flags & ~TVK_GEMM_EXACT) return fail(TVK_ERR_INVALID, w + ": unknown flags");
    return TVK_OK;
}

tvk_status conv_validate(const tvk_conv_desc* d, const char* who) {
    const std::string w(who);
    if (!d) return fail(TVK_ERR_INVALID, w + ": desc is NULL");
    tvk_status st = check_dtype_flags(d->dtype, d->flags, w);
    if (st != TVK_OK) return st;
    if (d->n < 0 || d->c_in <= 0 || d->c_out <= 0 || d->h <= 0 || d->w <= 0 || d->kh <= 0 || d->kw <= 0 || d->groups <= 0)
        return fail(TVK_ERR_INVALID, w + ": sizes must be positive");
    if (d->c_in % d->groups || d->c_out % d->groups)
        return fail(TVK_ERR_INVALID, w + ": channels must be divisible by groups");
    for (int i = 0; i < 2; ++i)
        if (d->stride[i] <= 0 || d->dilation[i] <= 0 || d->padding[i] < 0)
            return fail(TVK_ERR_INVALID, w + ": stride and dilation must be positive, padding non-negative");
    const int64_t ho = (d->h + 2 * d->padding[0] - d->dilation[0] * (d->kh - 1) - 1) / d->stride[0] + 1;
    const int64_t wo = (d->w + 2 * d->padding[1] - d->dilation[1] * (d->kw - 1) - 1) / d->stride[1] + 1;
    if (ho <= 0 || wo <= 0 || ho != d->h_out || wo != d->w_out)
        return fail(TVK_ERR_INVALID, w + ": h_out/w_out do not match the geometry (expected " + std::to_string(ho) + "x" +
                                         std::to_string(wo) + ")");
    const int64_t es = dtype_size(d->dtype);
    const int64_t xb = d->n * d->c_in * d->h * d->w * es, yb = d->n * d->c_out * ho * wo * es;
    const int64_t wb = d->c_out * (d->c_in / d->groups) * d->kh * d->kw * es;
    if (xb >= 0x7fffffff || yb >= 0x7fffffff || wb >= 0x7fffffff)
        return fail(TVK_ERR_UNSUPPORTED, w + ": an operand exceeds 2 GiB (32-bit buffer offsets)");
    return TVK_OK;
}

ConvArgs make_args(const tvk_conv_desc& d) {
    ConvArgs p;
    memset(&p, 0, sizeof(p));
    p.x = d.x; p.w = d.weight; p.bias = d.bias; p.y = d.y;
    p.n = (int)d.n; p.cin = (int)d.c_in; p.h = (int)d.h; p.wd = (int)d.w;
    p.cout = (int)d.c_out; p.kh = (int)d.kh; p.kw = (int)d.kw;
    p.sh = (int)d.stride[0]; p.sw = (int)d.stride[1]; p.ph = (int)d.padding[0]; p.pw = (int)d.padding[1];
    p.dh = (int)d.dilation[0]; p.dw = (int)d.dilation[1]; p.groups = (int)d.groups;
    p.ho = (int)d.h_out; p.wo = (int)d.w_out;
    p.dp = 1; p.kd = 1; p.sd = 1; p.pd = 0; p.dd = 1; p.dop = 1;
    p.si = p.h * p.wd; p.so = p.ho * p.wo;
    p.cx = p.cin / p.groups; p.cy = p.cout / p.groups; p.taps = p.kh * p.kw;
    const int64_t es = dtype_size(d.dtype);
    p.x_bytes = (int)(d.n * d.c_in * d.h * d.w * es);
    p.y_bytes = (int)(d.n * d.c_out * d.h_out * d.w_out * es);
    p.w_bytes = (int)(d.c_out * p.cx * d.kh * d.kw * es);
    p.split = 1;
    return p;
}

template <int DT, int ND, int MODE>
void launch(const ConvArgs& p, bool seq, hipStream_t s) {
    if (seq || DT == TVK_F32) {
        dim3 grid((p.N + C_BN - 1) / C_BN, (p.M + 127) / 128, p.groups * p.split);
        hipLaunchKernelGGL((conv_seq_kernel<DT, ND, MODE>), grid, dim3(256), 0, s, p);
    } else if constexpr (DT != TVK_F32) {
        if (p.M <= 64) {
            dim3 grid((p.N + C_BN - 1) / C_BN, (p.M + 63) / 64, p.groups * p.split);
            hipLaunchKernelGGL((conv16_kernel<DT, ND, MODE, 64>), grid, dim3(256), 0, s, p);
        } else {
            dim3 grid((p.N + C_BN - 1) / C_BN, (p.M + 127) / 128, p.groups * p.split);
            hipLaunchKernelGGL((conv16_kernel<DT, ND, MODE, 128>), grid, dim3(256), 0, s, p);
        }
    }
}

template <int MODE>
void set_gemm_shape(ConvArgs& p) {
    if (MODE == FWD) { p.M = p.cy; p.N = p.n * p.so; p.K = p.cx * p.taps; }
    else if (MODE == DGRAD) { p.M = p.cx; p.N = p.n * p.si; p.K = p.cy * p.taps; }
    else { p.M = p.cy; p.N = p.cx * p.taps; p.K = p.n * p.so; }
}

// The generic implicit-GEMM kernels: the grad-weight split, the launch, and
// the split reduction. p carries the geometry and the GEMM shape.
template <int ND, int MODE>
tvk_status run_generic(ConvArgs& p, int32_t dtype, bool seq, void* out, hipStream_t s, const char* who) {
    const size_t es = dtype_size(dtype);
    if (p.N == 0 || p.M == 0) return TVK_OK;
    if (p.K == 0) {
        // empty reduction (grad weight of an empty batch): zeros, written by a
        // kernel rather than a memset so the call can be graph-captured
        const int64_t count = (int64_t)p.cout * p.cx * p.taps;
        const unsigned blocks = (unsigned)std::min<int64_t>((count * (int64_t)es / 4 + 255) / 256 + 1, 4096);
        hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, s, static_cast<uint16_t*>(out), count * (int64_t)es / 2);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
        return TVK_OK;
    }
    Scratch scratch;
    if (MODE == WGRAD) {
        // split the long reduction so the grid covers the device: about 512
        // blocks, each with at least 8 k stages
        const int bm = (seq || dtype == TVK_F32 || p.M > 64) ? 128 : 64;
        const int64_t tiles = (int64_t)((p.M + bm - 1) / bm) * ((p.N + C_BN - 1) / C_BN) * p.groups;
        int64_t split = std::max<int64_t>(1, std::min<int64_t>(512 / std::max<int64_t>(1, tiles), p.K / (8 * C_BK)));
        split = std::min<int64_t>(split, 65535 / p.groups);
        int64_t chunk = (p.K + split - 1) / split;
        chunk = (chunk + C_BK - 1) / C_BK * C_BK;
        split = (p.K + chunk - 1) / chunk;
        p.split = (int)split;
        p.k_chunk = (int)chunk;
        if (split > 1) {
            p.part = static_cast<float*>(scratch.get((size_t)split * p.cout * p.cx * p.taps * sizeof(float), s));
            if (!p.part) return fail(TVK_ERR_OOM, std::string(who) + ": no workspace for the split-k partials");
        }
    }
    switch (dtype) {
    case TVK_F32: launch<TVK_F32, ND, MODE>(p, true, s); break;
    case TVK_F16: launch<TVK_F16, ND, MODE>(p, seq, s); break;
    default: launch<TVK_BF16, ND, MODE>(p, seq, s); break;
    }
    if (MODE == WGRAD && p.split > 1) {
        const int64_t count = (int64_t)p.cout * p.cx * p.taps;
        const unsigned blocks = (unsigned)std::min<int64_t>((count + 3) / 4, 8192);
        switch (dtype) {
        case TVK_F32: hipLaunchKernelGGL(wgrad_reduce_kernel<TVK_F32>, dim3(blocks), dim3(256), 0, s, p.part, out, count, p.split); break;
        case TVK_F16: hipLaunchKernelGGL(wgrad_reduce_kernel<TVK_F16>, dim3(blocks), dim3(256), 0, s, p.part, out, count, p.split); break;
        default: hipLaunchKernelGGL(wgrad_reduce_kernel<TVK_BF16>, dim3(blocks), dim3(256), 0, s, p.part, out, count, p.split); break;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string(who) + ": launch failed: " + hipGetErrorString(e));
    return TVK_OK;
}

// ---------------------------------------------------------------------------
// Kernel choice. A 2-D problem can run on up to four kernel families:
//   conv_stem           few input channels, one k step, straight from NCHW (conv_stem.hip)
//   conv_halo           3x3 (stride 1 and 2) and 1x1 kernels through an LDS halo of the
//                       NCHW source (conv_nhwc.hip)
//   conv_ring           channels-last implicit GEMM on the LDS ring (conv_nhwc.hip)
//   conv_implicit_gemm  the element-gathering implicit GEMM here, every problem
// The shape rule takes the first that applies in that order; the kernel-choice
// table (the GEMMs' table, kind "conv") may record another candidate for the
// problem's shape class, as the reference tunes its conv tilings per problem
// through the matmul autotuner (src/api/ops/conv.cpp:499-659). Only the
// implicit GEMM runs float32 and TVK_GEMM_EXACT (the others are float16 /
// bfloat16 kernels of another summation order), so a recorded choice never
// changes an exact result.
// ---------------------------------------------------------------------------

enum class ConvFamily { SMALL, HALO, RING, GENERIC };

const char* family_name(ConvFamily f) {
    switch (f) {
    case ConvFamily::SMALL: return "conv_stem";
    case ConvFamily::HALO: return "conv_halo";
    case ConvFamily::RING: return "conv_ring";
    default: return "conv_implicit_gemm";
    }
}

template <int MODE>
ConvArgs gemm_args(const tvk_conv_desc& d) {
    ConvArgs p = make_args(d);
    p.out = MODE == FWD ? d.y : MODE == DGRAD ? d.x : d.weight;
    p.has_bias = (MODE == FWD && d.bias) ? 1 : 0;
    set_gemm_shape<MODE>(p);
    return p;
}

// Every family that computes the (validated) problem, the shape rule's first.
template <int MODE>
std::vector<ConvFamily> conv_candidates(const tvk_conv_desc& d) {
    std::vector<ConvFamily> out;
    const ConvArgs p = gemm_args<MODE>(d);
    if (p.N != 0 && p.M != 0 && p.K != 0) {
        if (conv_small_applies(d, MODE)) out.push_back(ConvFamily::SMALL);
        if (conv_halo_applies(d, MODE)) out.push_back(ConvFamily::HALO);
        if (conv_ring_applies(d, MODE)) out.push_back(ConvFamily::RING);
    }
    out.push_back(ConvFamily::GENERIC);
    return out;
}

// Shape class, after the reference's conv tune key (conv.cpp:643-644: mode,
// ceil(log2) of the GEMM rows, columns, depth and planes, of the taps, padding,
// unit stride): here mode, dtype, exact flag, bias, grouping, which families
// apply, ceil(log2) of the GEMM M, N, K and of the taps, padding, unit stride
// and unit dilation.
template <int MODE>
uint64_t conv_tune_key(const tvk_conv_desc& d, const std::vector<ConvFamily>& cands) {
    const ConvArgs p = gemm_args<MODE>(d);
    auto lg = [](int64_t v) {
        uint64_t r = 0;
        while (r < 63 && (int64_t(1) << r) < v) ++r;
        return r;
    };
    uint64_t fam = 0;
    for (ConvFamily f : cands) fam |= uint64_t(1) << (int)f;
    const bool padded = d.padding[0] != 0 || d.padding[1] != 0;
    const bool unit_stride = d.stride[0] == 1 && d.stride[1] == 1;
    const bool unit_dil = d.dilation[0] == 1 && d.dilation[1] == 1;
    return (uint64_t)MODE | (uint64_t)(d.dtype & 15) << 2 | (uint64_t)(d.flags & 1) << 6 | (uint64_t)(p.has_bias & 1) << 7 |
           (uint64_t)(d.groups > 1) << 8 | fam << 9 | (uint64_t)padded << 13 | (uint64_t)unit_stride << 14 |
           (uint64_t)unit_dil << 15 | lg(p.M) << 16 | lg(p.N) << 24 | lg(p.K) << 32 | lg(p.taps) << 40;
}

// The tensors a direction reads must be given (an empty batch reads no x or y).
template <int MODE>
bool inputs_given(int64_t n, const void* x, const void* weight, const void* y) {
    if (MODE == FWD) return (n == 0 || x) && weight;
    if (MODE == DGRAD) return (n == 0 || y) && weight;
    return n == 0 || (x && y);
}

template <int MODE>
tvk_status run_family(const tvk_conv_desc& d, ConvFamily f, const char* who) {
    ConvArgs p = gemm_args<MODE>(d);
    if (!p.out) return fail(TVK_ERR_INVALID, std::string(who) + ": output pointer is NULL");
    if (!inputs_given<MODE>(d.n, d.x, d.weight, d.y)) return fail(TVK_ERR_INVALID, std::string(who) + ": an input pointer is NULL");
    if (p.N != 0 && p.M != 0 && p.K != 0) {
        if (f == ConvFamily::SMALL) return conv_small_run(d, MODE, who);
        if (f == ConvFamily::HALO) return conv_halo_run(d, MODE, who);
        if (f == ConvFamily::RING) return conv_ring_run(d, MODE, who);
    }
    return run_generic<2, MODE>(p, d.dtype, (d.flags & TVK_GEMM_EXACT) != 0, p.out, resolve_stream(d.stream), who);
}

// The shape rule's family unless the table records another candidate for the
// shape class (a recorded family that does not apply is ignored).
template <int MODE>
ConvFamily choose_family(const tvk_conv_desc& d, const std::vector<ConvFamily>& cands) {
    std::string id;
    if (cands.size() > 1 && tune_lookup("conv", conv_tune_key<MODE>(d, cands), id))
        for (ConvFamily f : cands)
            if (id == family_name(f)) return f;
    return cands[0];
}

template <int MODE>
tvk_status run_conv(const tvk_conv_desc* desc, const char* who) {
    tvk_status st = conv_validate(desc, who);
    if (st != TVK_OK) return st;
    const tvk_conv_desc& d = *desc;
    const std::vector<ConvFamily> cands = conv_candidates<MODE>(d);
    return run_family<MODE>(d, choose_family<MODE>(d, cands), who);
}

// Times every candidate and returns the fastest: the first candidate runs for
// about 2 ms first (the clock ramps up after an idle spell), then each takes
// the median of five timed calls after one untimed call, as tvk_gemm_tune
// does. The timed calls write the problem's own output.
template <int MODE>
tvk_status time_families(const tvk_conv_desc& d, const std::vector<ConvFamily>& cands, ConvFamily& best, const char* who) {
    const hipStream_t s = resolve_stream(d.stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        (void)hipGetLastError();
        if (e0) (void)hipEventDestroy(e0);
        return fail(TVK_ERR_DEVICE, std::string(who) + ": hipEventCreate failed");
    }
    if (hipEventRecord(e0, s) == hipSuccess) {
        for (int i = 0; i < 200; ++i) {
            if (run_family<MODE>(d, cands[0], who) != TVK_OK) break;
            float ms = 0.0f;
            if (i % 8 == 7 && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                               hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms > 2.0f))
                break;
        }
        (void)hipGetLastError();
    }
    float best_ms = INFINITY;
    best = cands[0];
    for (ConvFamily f : cands) {
        float spans[5];
        bool ok = run_family<MODE>(d, f, who) == TVK_OK;
        for (int i = 0; ok && i < 5; ++i)
            ok = hipEventRecord(e0, s) == hipSuccess && run_family<MODE>(d, f, who) == TVK_OK &&
                 hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
                 hipEventElapsedTime(&spans[i], e0, e1) == hipSuccess;
        if (!ok) {
            (void)hipGetLastError();
            continue;
        }
        std::nth_element(spans, spans + 2, spans + 5);
        if (spans[2] < best_ms) {
            best_ms = spans[2];
            best = f;
        }
    }
    (void)hipStreamSynchronize(s);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return TVK_OK;
}

// ---------------------------------------------------------------------------
// N-d entry points: 1 and 2 spatial dimensions run the 2-D dispatch (1-D as a
// height of 1), 3 run the 3-D generic kernels
// ---------------------------------------------------------------------------

tvk_status convnd_validate(const tvk_convnd_desc* d, const char* who) {
    const std::string w(who);
    if (!d) return fail(TVK_ERR_INVALID, w + ": desc is NULL");
    if (d->spatial_dims < 1 || d->spatial_dims > 3)
        return fail(TVK_ERR_UNSUPPORTED, w + ": spatial_dims must be 1, 2 or 3 (got " + std::to_string(d->spatial_dims) + ")");
    tvk_status st = check_dtype_flags(d->dtype, d->flags, w);
    if (st != TVK_OK) return st;
    if (d->n < 0 || d->c_in <= 0 || d->c_out <= 0 || d->groups <= 0)
        return fail(TVK_ERR_INVALID, w + ": sizes must be positive");
    if (d->c_in % d->groups || d->c_out % d->groups)
        return fail(TVK_ERR_INVALID, w + ": channels must be divisible by groups");
    int64_t si = 1, so = 1, taps = 1;
    for (int i = 0; i < d->spatial_dims; ++i) {
        if (d->in_size[i] <= 0 || d->kernel[i] <= 0) return fail(TVK_ERR_INVALID, w + ": sizes must be positive");
        if (d->stride[i] <= 0 || d->dilation[i] <= 0 || d->padding[i] < 0)
            return fail(TVK_ERR_INVALID, w + ": stride and dilation must be positive, padding non-negative");
        const int64_t o = (d->in_size[i] + 2 * d->padding[i] - d->dilation[i] * (d->kernel[i] - 1) - 1) / d->stride[i] + 1;
        if (o <= 0 || o != d->out_size[i])
            return fail(TVK_ERR_INVALID, w + ": out_size[" + std::to_string(i) + "] does not match the geometry (expected " +
                                             std::to_string(o) + ")");
        si *= d->in_size[i];
        so *= o;
        taps *= d->kernel[i];
    }
    const int64_t es = dtype_size(d->dtype);
    const int64_t xb = d->n * d->c_in * si * es, yb = d->n * d->c_out * so * es, wb = d->c_out * (d->c_in / d->groups) * taps * es;
    if (xb >= 0x7fffffff || yb >= 0x7fffffff || wb >= 0x7fffffff)
        return fail(TVK_ERR_UNSUPPORTED, w + ": an operand exceeds 2 GiB (32-bit buffer offsets)");
    return TVK_OK;
}

// The 2-D descriptor of a 1-D or 2-D problem (1-D: height 1, kernel height 1).
tvk_conv_desc as_2d(const tvk_convnd_desc& d) {
    tvk_conv_desc c;
    memset(&c, 0, sizeof(c));
    c.dtype = d.dtype; c.flags = d.flags;
    c.n = d.n; c.c_in = d.c_in; c.c_out = d.c_out; c.groups = d.groups;
    const int o = d.spatial_dims == 1 ? 1 : 0;   // first 2-D slot taken from the descriptor
    c.h = o ? 1 : d.in_size[0];
    c.kh = o ? 1 : d.kernel[0];
    c.stride[0] = o ? 1 : d.stride[0];
    c.padding[0] = o ? 0 : d.padding[0];
    c.dilation[0] = o ? 1 : d.dilation[0];
    c.h_out = o ? 1 : d.out_size[0];
    const int j = d.spatial_dims - 1;
    c.w = d.in_size[j]; c.kw = d.kernel[j]; c.stride[1] = d.stride[j]; c.padding[1] = d.padding[j];
    c.dilation[1] = d.dilation[j]; c.w_out = d.out_size[j];
    c.x = d.x; c.weight = d.weight; c.bias = d.bias; c.y = d.y; c.stream = d.stream;
    return c;
}

ConvArgs make_args3(const tvk_convnd_desc& d) {
    ConvArgs p;
    memset(&p, 0, sizeof(p));
    p.x = d.x; p.w = d.weight; p.bias = d.bias; p.y = d.y;
    p.n = (int)d.n; p.cin = (int)d.c_in; p.cout = (int)d.c_out; p.groups = (int)d.groups;
    p.dp = (int)d.in_size[0]; p.h = (int)d.in_size[1]; p.wd = (int)d.in_size[2];
    p.kd = (int)d.kernel[0]; p.kh = (int)d.kernel[1]; p.kw = (int)d.kernel[2];
    p.sd = (int)d.stride[0]; p.sh = (int)d.stride[1]; p.sw = (int)d.stride[2];
    p.pd = (int)d.padding[0]; p.ph = (int)d.padding[1]; p.pw = (int)d.padding[2];
    p.dd = (int)d.dilation[0]; p.dh = (int)d.dilation[1]; p.dw = (int)d.dilation[2];
    p.dop = (int)d.out_size[0]; p.ho = (int)d.out_size[1]; p.wo = (int)d.out_size[2];
    p.si = p.dp * p.h * p.wd; p.so = p.dop * p.ho * p.wo;
    p.cx = p.cin / p.groups; p.cy = p.cout / p.groups; p.taps = p.kd * p.kh * p.kw;
    const int64_t es = dtype_size(d.dtype);
    p.x_bytes = (int)(d.n * d.c_in * p.si * es);
    p.y_bytes = (int)(d.n * d.c_out * p.so * es);
    p.w_bytes = (int)(d.c_out * p.cx * p.taps * es);
    p.split = 1;
    return p;
}

template <int MODE>
tvk_status run_convnd(const tvk_convnd_desc* desc, const char* who) {
    tvk_status st = convnd_validate(desc, who);
    if (st != TVK_OK) return st;
    const tvk_convnd_desc& d = *desc;
    if (d.spatial_dims < 3) {
        const tvk_conv_desc c = as_2d(d);
        return run_conv<MODE>(&c, who);
    }
    void* out = MODE == FWD ? d.y : MODE == DGRAD ? d.x : d.weight;
    if (!out) return fail(TVK_ERR_INVALID, std::string(who) + ": output pointer is NULL");
    if (!inputs_given<MODE>(d.n, d.x, d.weight, d.y)) return fail(TVK_ERR_INVALID, std::string(who) + ": an input pointer is NULL");
    ConvArgs p = make_args3(d);
    p.out = out;
    p.has_bias = (MODE == FWD && d.bias) ? 1 : 0;
    set_gemm_shape<MODE>(p);
    return run_generic<3, MODE>(p, d.dtype, (d.flags & TVK_GEMM_EXACT) != 0, out, resolve_stream(d.stream), who);
}

}  // namespace
}  // namespace tvk

using namespace tvk;

namespace tvk {
namespace {

void put_conv_name(char* name, size_t name_len, const std::string& n) {
    if (name && name_len) snprintf(name, name_len, "%s", n.c_str());
}

// The 2-D view of a validated N-d problem, or false for three spatial
// dimensions (one family: the 3-D implicit GEMM).
bool nd_as_2d(const tvk_convnd_desc& d, tvk_conv_desc& c) {
    if (d.spatial_dims >= 3) return false;
    c = as_2d(d);
    return true;
}

template <int MODE>
tvk_status conv_candidates_nd(const tvk_convnd_desc* desc, char* names, size_t names_len, const char* who) {
    tvk_status st = convnd_validate(desc, who);
    if (st != TVK_OK) return st;
    if (!names || names_len == 0) return fail(TVK_ERR_INVALID, std::string(who) + ": name buffer is empty");
    std::string all;
    tvk_conv_desc c;
    if (!nd_as_2d(*desc, c)) all = family_name(ConvFamily::GENERIC);
    else
        for (ConvFamily f : conv_candidates<MODE>(c)) all += (all.empty() ? "" : "\n") + std::string(family_name(f));
    if (all.size() + 1 > names_len)
        return fail(TVK_ERR_INVALID, std::string(who) + ": the names need " + std::to_string(all.size() + 1) + " bytes");
    snprintf(names, names_len, "%s", all.c_str());
    return TVK_OK;
}

template <int MODE>
tvk_status conv_choose_nd(const tvk_convnd_desc* desc, const char* kernel, int persist, const char* who) {
    tvk_status st = convnd_validate(desc, who);
    if (st != TVK_OK) return st;
    if (!kernel) return fail(TVK_ERR_INVALID, std::string(who) + ": kernel is NULL");
    tvk_conv_desc c;
    if (!nd_as_2d(*desc, c)) {
        // one family: nothing to record
        if (std::string(kernel) == family_name(ConvFamily::GENERIC)) return TVK_OK;
        return fail(TVK_ERR_INVALID, std::string(who) + ": " + kernel + " does not compute this convolution");
    }
    const std::vector<ConvFamily> cands = conv_candidates<MODE>(c);
    for (ConvFamily f : cands)
        if (std::string(kernel) == family_name(f)) {
            tune_record("conv", conv_tune_key<MODE>(c, cands), family_name(f), persist != 0);
            return TVK_OK;
        }
    return fail(TVK_ERR_INVALID, std::string(who) + ": " + kernel + " does not compute this convolution");
}

template <int MODE>
tvk_status conv_tune_nd(const tvk_convnd_desc* desc, char* name, size_t name_len, const char* who) {
    tvk_status st = convnd_validate(desc, who);
    if (st != TVK_OK) return st;
    tvk_conv_desc c;
    if (!nd_as_2d(*desc, c)) {
        put_conv_name(name, name_len, family_name(ConvFamily::GENERIC));
        return run_convnd<MODE>(desc, who);
    }
    const std::vector<ConvFamily> cands = conv_candidates<MODE>(c);
    ConvFamily best = cands[0];
    if (cands.size() > 1) {
        const uint64_t key = conv_tune_key<MODE>(c, cands);
        std::string id;
        bool known = false;
        if (tune_lookup("conv", key, id))
            for (ConvFamily f : cands)
                if (id == family_name(f)) {
                    best = f;
                    known = true;
                    break;
                }
        if (!known) {
            st = time_families<MODE>(c, cands, best, who);
            if (st != TVK_OK) return st;
            tune_record("conv", key, family_name(best), true);
        }
    }
    put_conv_name(name, name_len, family_name(best));
    return run_family<MODE>(c, best, who);
}

int conv_mode_ok(int mode) { return mode == FWD || mode == DGRAD || mode == WGRAD; }

}  // namespace
}  // namespace tvk

extern "C" tvk_status tvk_conv_candidates(const tvk_convnd_desc* desc, int mode, char* names, size_t names_len) {
    if (!conv_mode_ok(mode)) return fail(TVK_ERR_INVALID, "tvk_conv_candidates: mode must be TVK_CONV_FWD, _DGRAD or _WGRAD");
    if (mode == FWD) return conv_candidates_nd<FWD>(desc, names, names_len, "tvk_conv_candidates");
    if (mode == DGRAD) return conv_candidates_nd<DGRAD>(desc, names, names_len, "tvk_conv_candidates");
    return conv_candidates_nd<WGRAD>(desc, names, names_len, "tvk_conv_candidates");
}

extern "C" tvk_status tvk_conv_choose(const tvk_convnd_desc* desc, int mode, const char* kernel, int persist) {
    if (!conv_mode_ok(mode)) return fail(TVK_ERR_INVALID, "tvk_conv_choose: mode must be TVK_CONV_FWD, _DGRAD or _WGRAD");
    if (mode == FWD) return conv_choose_nd<FWD>(desc, kernel, persist, "tvk_conv_choose");
    if (mode == DGRAD) return conv_choose_nd<DGRAD>(desc, kernel, persist, "tvk_conv_choose");
    return conv_choose_nd<WGRAD>(desc, kernel, persist, "tvk_conv_choose");
}

extern "C" tvk_status tvk_conv_tune(const tvk_convnd_desc* desc, int mode, char* name, size_t name_len) {
    if (!conv_mode_ok(mode)) return fail(TVK_ERR_INVALID, "tvk_conv_tune: mode must be TVK_CONV_FWD, _DGRAD or _WGRAD");
    if (mode == FWD) return conv_tune_nd<FWD>(desc, name, name_len, "tvk_conv_tune");
    if (mode == DGRAD) return conv_tune_nd<DGRAD>(desc, name, name_len, "tvk_conv_tune");
    return conv_tune_nd<WGRAD>(desc, name, name_len, "tvk_conv_tune");
}

extern "C" tvk_status tvk_conv2d_fwd(const tvk_conv_desc* desc) { return run_conv<FWD>(desc, "tvk_conv2d_fwd"); }
extern "C" tvk_status tvk_conv2d_dgrad(const tvk_conv_desc* desc) { return run_conv<DGRAD>(desc, "tvk_conv2d_dgrad"); }
extern "C" tvk_status tvk_conv2d_wgrad(const tvk_conv_desc* desc) { return run_conv<WGRAD>(desc, "tvk_conv2d_wgrad"); }
extern "C" tvk_status tvk_conv_fwd(const tvk_convnd_desc* desc) { return run_convnd<FWD>(desc, "tvk_conv_fwd"); }
extern "C" tvk_status tvk_conv_dgrad(const tvk_convnd_desc* desc) { return run_convnd<DGRAD>(desc, "tvk_conv_dgrad"); }
extern "C" tvk_status tvk_conv_wgrad(const tvk_convnd_desc* desc) { return run_convnd<WGRAD>(desc, "tvk_conv_wgrad"); }
