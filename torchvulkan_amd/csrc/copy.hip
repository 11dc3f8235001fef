// Strided element-wise copy with dtype conversion (tvk_copy): the copy and
// cast kernels on both sides of every contraction (operand .to() and
// .contiguous(), .out copies, conv's NCHW .contiguous()).
//
// Reference semantics: dispatch_copy_shader (src/api/tensor/transfer.cpp:16-56)
// walks a TensorIterator-coalesced index space and copies T -> T;
// dispatch_cast_shader (src/api/tensor/cast.cpp:8-56) does the same through
// castValue (src/shaders/core/cast.slang:49-52): the source widens to int64,
// uint64, float or double and the destination is built from that one wide
// value (src/shaders/core/dtype.slang:122-282); with a bool on either side the
// value is (src != 0) ? 1 : 0 (src/shaders/ops/cast.slang:29-33).
//
// The host plan merges dimensions the way TensorIterator coalesces them
// (innermost first, by destination strides), then picks one of five kernels:
//   cast_contig: both sides dense: 8 elements per thread, vector loads/stores;
//   broadcast:   a dense destination from one source element (an expanded
//                scalar, stride 0 everywhere): converted once per thread and
//                stored 16 bytes at a time;
//   rows:        same dtype, the innermost dimension contiguous on both sides
//                in whole 16-byte vectors (a permute of outer dimensions): one
//                16-byte vector per thread;
//   transpose:   destination contiguous along a dimension the source is not,
//                source contiguous along another: 64x64 tiles through LDS, so
//                both the loads and the stores are coalesced (W.t().contiguous(),
//                NCHW <-> NHWC);
//   strided:     anything else: one element per thread, offsets from the
//                linear index by multiply-high division.
// Same-dtype dense copies are a hipMemcpyAsync. Same-dtype copies move raw bits
// (integer lanes of the element's size), so NaN payloads are kept.
#include "convert.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

namespace tvk {
namespace {


// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

struct Shape {
    int nd;
    int64_t size[kMaxDims], ss[kMaxDims], ds[kMaxDims];   // innermost first, elements
};

struct StridedArgs {
    const char* src;
    char* dst;
    int sdt, ddt;
    int ss_bytes, ds_bytes;   // element sizes
    int nd;
    int64_t numel;
    Div32 div[kMaxDims];
    int64_t ss[kMaxDims], ds[kMaxDims];
    int64_t size[kMaxDims];
};

// One element per thread; dimension 0 is the destination's innermost, so
// neighbouring threads write neighbouring elements where dst allows it.
template <int SDT, int DDT, bool IDX32>
__global__ __launch_bounds__(256) void copy_strided_kernel(StridedArgs p) {
    const Dts<SDT, DDT> t(p.sdt, p.ddt);
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t li = (int64_t)blockIdx.x * 256 + threadIdx.x; li < p.numel; li += step) {
        int64_t so = 0, dof = 0;
        if constexpr (IDX32) {
            uint32_t rem = (uint32_t)li;
#pragma unroll 1
            for (int k = 0; k < p.nd - 1; ++k) {
                const uint32_t q = div32(rem, p.div[k]);
                const uint32_t c = rem - q * p.div[k].d;
                so += (int64_t)c * p.ss[k];
                dof += (int64_t)c * p.ds[k];
                rem = q;
            }
            so += (int64_t)rem * p.ss[p.nd - 1];
            dof += (int64_t)rem * p.ds[p.nd - 1];
        } else {
            int64_t rem = li;
#pragma unroll 1
            for (int k = 0; k < p.nd - 1; ++k) {
                const int64_t q = rem / p.size[k];
                const int64_t c = rem - q * p.size[k];
                so += c * p.ss[k];
                dof += c * p.ds[k];
                rem = q;
            }
            so += rem * p.ss[p.nd - 1];
            dof += rem * p.ds[p.nd - 1];
        }
        convert(p.src + so * p.ss_bytes, t.s, p.dst + dof * p.ds_bytes, t.d);
    }
}

// Same-dtype copies whose innermost dimension is contiguous on both sides in
// whole 16-byte vectors (a permute of the outer dimensions, such as
// [B, L, H, D] -> [B, H, L, D]): one 16-byte vector per thread; the vector
// index is split into the position inside its run and the run's outer
// coordinates, whose offsets are in bytes.
struct RowsArgs {
    const char* src;
    char* dst;
    int nd;                   // outer dimensions (the run dimension excluded)
    int64_t nvec;             // 16-byte vectors in all
    Div32 vdiv;               // vectors per run
    Div32 div[kMaxDims];
    int64_t size[kMaxDims], ss[kMaxDims], ds[kMaxDims];   // outer extents; strides in bytes
};

__global__ __launch_bounds__(256) void copy_rows_kernel(RowsArgs p) {
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < p.nvec; v += step) {
        uint32_t run = div32((uint32_t)v, p.vdiv);
        const uint32_t w = (uint32_t)v - run * p.vdiv.d;
        int64_t so = (int64_t)w * 16, dof = (int64_t)w * 16;
#pragma unroll 1
        for (int k = 0; k < p.nd - 1; ++k) {
            const uint32_t q = div32(run, p.div[k]);
            const uint32_t c = run - q * p.div[k].d;
            so += (int64_t)c * p.ss[k];
            dof += (int64_t)c * p.ds[k];
            run = q;
        }
        so += (int64_t)run * p.ss[p.nd - 1];
        dof += (int64_t)run * p.ds[p.nd - 1];
        *reinterpret_cast<u32x4*>(p.dst + dof) = *reinterpret_cast<const u32x4*>(p.src + so);
    }
}

// Dense to dense, 8 elements per thread. VEC: both bases aligned to 8
// elements, so each group of 8 is one set of aligned vector accesses.
template <int SDT, int DDT, int SB, int DB, bool VEC>
__global__ __launch_bounds__(256) void cast_contig_kernel(const char* src, char* dst, int64_t n, int sdt, int ddt) {
    const Dts<SDT, DDT> t(sdt, ddt);
    const int64_t groups = (n + 7) / 8;
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < groups; g += step) {
        const int64_t e0 = g * 8;
        if (VEC && e0 + 8 <= n) {
            struct alignas(SB * 8) SV { char b[SB * 8]; };
            struct alignas(DB * 8) DV { char b[DB * 8]; };
            const SV sv = *reinterpret_cast<const SV*>(src + e0 * SB);
            DV dv;
#pragma unroll
            for (int e = 0; e < 8; ++e) convert(sv.b + e * SB, t.s, dv.b + e * DB, t.d);
            *reinterpret_cast<DV*>(dst + e0 * DB) = dv;
        } else {
            const int64_t e1 = e0 + 8 < n ? e0 + 8 : n;
            for (int64_t e = e0; e < e1; ++e) convert(src + e * SB, t.s, dst + e * DB, t.d);
        }
    }
}

// Runtime element sizes (dtypes outside the templated float set).
__global__ __launch_bounds__(256) void cast_contig_dyn_kernel(const char* src, char* dst, int64_t n, int sdt, int ddt,
                                                             int sb, int db) {
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += step)
        convert(src + e * sb, sdt, dst + e * db, ddt);
}

constexpr int TT = 64;   // transpose tile edge

struct TransposeArgs {
    const char* src;
    char* dst;
    int sdt, ddt;
    int sb, db;               // element sizes
    int64_t n0, nj;           // extents of the two tiled dimensions
    int64_t ss0, dsj;         // src stride along 0, dst stride along j (the other two are 1)
    int64_t tiles0, tilesj;
    int nb;                   // other dimensions
    int64_t bsize[kMaxDims], bss[kMaxDims], bds[kMaxDims];
};

// Writes the low `db` bytes of w (one converted element) to p.
template <typename Word>
__device__ __forceinline__ void store_elem(char* p, const Word& w, int db) {
    switch (db) {
        case 1: *reinterpret_cast<uint8_t*>(p) = (uint8_t)w; break;
        case 2: *reinterpret_cast<uint16_t*>(p) = (uint16_t)w; break;
        case 4: *reinterpret_cast<uint32_t*>(p) = (uint32_t)w; break;
        default: *reinterpret_cast<uint64_t*>(p) = (uint64_t)w; break;
    }
}

// dst is contiguous along dimension 0, src along dimension j. A 64x64 tile is
// read along j (coalesced in src), converted, parked in LDS, and written
// along 0 (coalesced in dst). Word = the LDS type holding one converted element.
template <int SDT, int DDT, typename Word>
__global__ __launch_bounds__(256) void copy_transpose_kernel(TransposeArgs p) {
    const Dts<SDT, DDT> t(p.sdt, p.ddt);
    const int db = DDT == DYN ? p.db : (int)dtype_size(DDT);
    __shared__ Word tile[TT][TT + 1];
    int64_t bid = blockIdx.x;
    const int64_t t0 = bid % p.tiles0;
    bid /= p.tiles0;
    const int64_t tj = bid % p.tilesj;
    int64_t rest = bid / p.tilesj;
    int64_t so = 0, dof = 0;
    for (int k = 0; k < p.nb; ++k) {
        const int64_t c = rest % p.bsize[k];
        rest /= p.bsize[k];
        so += c * p.bss[k];
        dof += c * p.bds[k];
    }
    const int64_t a0 = t0 * TT, b0 = tj * TT;
    const int lane = threadIdx.x % TT, row = threadIdx.x / TT;
#pragma unroll 4
    for (int r = row; r < TT; r += 256 / TT) {
        const int64_t a = a0 + r, b = b0 + lane;   // read along j
        Word w = 0;
        if (a < p.n0 && b < p.nj) convert(p.src + (so + a * p.ss0 + b) * p.sb, t.s, reinterpret_cast<char*>(&w), t.d);
        tile[r][lane] = w;
    }
    __syncthreads();
#pragma unroll 4
    for (int r = row; r < TT; r += 256 / TT) {
        const int64_t b = b0 + r, a = a0 + lane;   // write along 0
        if (a < p.n0 && b < p.nj) {
            store_elem(p.dst + (dof + a + b * p.dsj) * db, tile[lane][r], db);
        }
    }
}

// The same tile with 16-byte accesses on both sides: a thread loads
// VS = 16/sb consecutive source elements along j and stores VD = 16/db
// consecutive destination elements along 0. Chunks that cross the end of the
// matrix fall back to one element at a time. LDS holds one converted element
// per Word at [a][b] with a row pitch of TT+1 words, so both phases touch 64
// distinct banks per wave. Requires 16-byte aligned chunk starts (bases and
// the strides ss0*sb, dsj*db multiples of 16).
template <int SDT, int DDT, typename Word>
__global__ __launch_bounds__(256) void copy_transpose_vec_kernel(TransposeArgs p) {
    constexpr int SB = (int)dtype_size(SDT), DB = (int)dtype_size(DDT);
    constexpr int VS = 16 / SB, VD = 16 / DB;
    constexpr int CS = TT / VS, CD = TT / VD;   // chunks per tile row, load / store side
    __shared__ Word tile[TT][TT + 1];
    int64_t bid = blockIdx.x;
    const int64_t t0 = bid % p.tiles0;
    bid /= p.tiles0;
    const int64_t tj = bid % p.tilesj;
    int64_t rest = bid / p.tilesj;
    int64_t so = 0, dof = 0;
    for (int k = 0; k < p.nb; ++k) {
        const int64_t c = rest % p.bsize[k];
        rest /= p.bsize[k];
        so += c * p.bss[k];
        dof += c * p.bds[k];
    }
    const int64_t a0 = t0 * TT, b0 = tj * TT;
    const int tid = threadIdx.x;
    // load: thread -> (row a, chunk of VS along b); consecutive threads on consecutive chunks
#pragma unroll
    for (int q = tid; q < TT * CS; q += 256) {
        const int r = q / CS, cb = (q % CS) * VS;
        const int64_t a = a0 + r, b = b0 + cb;
        Word w[VS];
        if (a < p.n0 && b + VS <= p.nj) {
            struct alignas(16) V16 { char c[16]; };
            const V16 v = *reinterpret_cast<const V16*>(p.src + (so + a * p.ss0 + b) * SB);
#pragma unroll
            for (int e = 0; e < VS; ++e) {
                w[e] = 0;
                convert(v.c + e * SB, SDT, reinterpret_cast<char*>(&w[e]), DDT);
            }
        } else {
#pragma unroll
            for (int e = 0; e < VS; ++e) {
                w[e] = 0;
                if (a < p.n0 && b + e < p.nj) convert(p.src + (so + a * p.ss0 + b + e) * SB, SDT, reinterpret_cast<char*>(&w[e]), DDT);
            }
        }
#pragma unroll
        for (int e = 0; e < VS; ++e) tile[r][cb + e] = w[e];
    }
    __syncthreads();
    // store: thread -> (column b, chunk of VD along a); consecutive threads on consecutive chunks
#pragma unroll
    for (int q = tid; q < TT * CD; q += 256) {
        const int r = q / CD, ca = (q % CD) * VD;
        const int64_t b = b0 + r, a = a0 + ca;
        if (b >= p.nj || a >= p.n0) continue;
        char* dst = p.dst + (dof + a + b * p.dsj) * DB;
        if (a + VD <= p.n0) {
            struct alignas(16) V16 { char c[16]; };
            V16 v;
#pragma unroll
            for (int e = 0; e < VD; ++e) {
                const Word w = tile[ca + e][r];
                __builtin_memcpy(v.c + e * DB, &w, DB);
            }
            *reinterpret_cast<V16*>(dst) = v;
        } else {
            for (int e = 0; a + e < p.n0; ++e) store_elem(dst + e * DB, tile[ca + e][r], DB);
        }
    }
}

// Same-dtype 16-bit transpose without LDS (the 16-byte conditions of the
// kernel above). A wave moves 64 (along 0) x 64 (along j) elements: each lane
// loads an 8x8 block as eight 16-byte rows along j, transposes it in
// registers and stores eight 16-byte rows along 0; a quarter-wave covers 2 x 8
// blocks, so its loads and stores each touch whole 128-byte runs. Wave tiles
// are numbered j first (tilesj counts them along j), then 0, then the batch;
// a workgroup takes 4 consecutive ones (`total` of them). Blocks that cross
// the end of either dimension copy element by element.
__global__ __launch_bounds__(256) void copy_transpose_reg16_kernel(TransposeArgs p, int64_t total) {
    int64_t bid = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    if (bid >= total) return;
    const int64_t tj = bid % p.tilesj;
    bid /= p.tilesj;
    const int64_t t0 = bid % p.tiles0;
    int64_t rest = bid / p.tiles0;
    int64_t so = 0, dof = 0;
    for (int k = 0; k < p.nb; ++k) {
        const int64_t c = rest % p.bsize[k];
        rest /= p.bsize[k];
        so += c * p.bss[k];
        dof += c * p.bds[k];
    }
    const int lane = threadIdx.x % 64;
    const int l = lane % 16, q = lane / 16;
    const int64_t a = t0 * 64 + (q * 2 + l % 2) * 8;   // 8 rows along 0
    const int64_t b = tj * 64 + (l / 2) * 8;           // 8 columns along j
    if (a >= p.n0 || b >= p.nj) return;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(p.src) + so;
    uint16_t* dst = reinterpret_cast<uint16_t*>(p.dst) + dof;
    if (a + 8 <= p.n0 && b + 8 <= p.nj) {
        u32x4 r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = *reinterpret_cast<const u32x4*>(src + (a + i) * p.ss0 + b);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // column b + j: rows (2k, 2k + 1) packed low/high
            uint32_t v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = r[2 * k][j / 2], hi = r[2 * k + 1][j / 2];
                v[k] = (j % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
            }
            *reinterpret_cast<u32x4*>(dst + a + (b + j) * p.dsj) = u32x4{v[0], v[1], v[2], v[3]};
        }
    } else {
        for (int i = 0; i < 8 && a + i < p.n0; ++i)
            for (int j = 0; j < 8 && b + j < p.nj; ++j) dst[a + i + (b + j) * p.dsj] = src[(a + i) * p.ss0 + b + j];
    }
}

// ---------------------------------------------------------------------------
// host plan
// ---------------------------------------------------------------------------

enum PlanKind { PK_NONE = 0, PK_MEMCPY, PK_CAST_CONTIG, PK_TRANSPOSE, PK_STRIDED, PK_BROADCAST, PK_ROWS };

struct Plan {
    PlanKind kind;
    Shape sh;
    int64_t numel;
    int j;   // transpose: the source's contiguous dimension
};

bool valid_dtype(int dt) { return dt >= TVK_F32 && dt <= TVK_F8E5M2; }

tvk_status make_plan(const tvk_copy_desc* d, Plan& pl, const char* who) {
    if (!d) return fail(TVK_ERR_INVALID, std::string(who) + ": desc is NULL");
    if (!valid_dtype(d->src_dtype) || !valid_dtype(d->dst_dtype))
        return fail(TVK_ERR_UNSUPPORTED, std::string(who) + ": unsupported dtype");
    if (d->reserved != 0) return fail(TVK_ERR_INVALID, std::string(who) + ": nonzero reserved field");
    if (d->ndim < 0 || d->ndim > kMaxDims)
        return fail(TVK_ERR_UNSUPPORTED, std::string(who) + ": ndim " + std::to_string(d->ndim) + " is outside 0.." +
                                             std::to_string(kMaxDims));
    pl = Plan{};
    int64_t numel = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->sizes[k] < 0) return fail(TVK_ERR_INVALID, std::string(who) + ": negative size");
        if (d->src_strides[k] < 0 || d->dst_strides[k] < 0)
            return fail(TVK_ERR_UNSUPPORTED, std::string(who) + ": negative strides are not supported");
        numel *= d->sizes[k];
    }
    pl.numel = numel;
    if (numel == 0) {
        pl.kind = PK_NONE;
        return TVK_OK;
    }
    if (!d->src || !d->dst) return fail(TVK_ERR_INVALID, std::string(who) + ": src or dst is NULL");
    // dimensions of extent > 1, innermost (smallest dst stride) first; ties by src stride
    int idx[kMaxDims];
    int n = 0;
    for (int k = 0; k < d->ndim; ++k)
        if (d->sizes[k] > 1) {
            if (d->dst_strides[k] == 0)
                return fail(TVK_ERR_INVALID, std::string(who) + ": dst has a zero stride over extent " +
                                                 std::to_string(d->sizes[k]) + " (overlapping elements)");
            idx[n++] = k;
        }
    std::stable_sort(idx, idx + n, [&](int x, int y) {
        if (d->dst_strides[x] != d->dst_strides[y]) return d->dst_strides[x] < d->dst_strides[y];
        return d->src_strides[x] < d->src_strides[y];
    });
    Shape& sh = pl.sh;
    sh.nd = 0;
    for (int q = 0; q < n; ++q) {
        const int k = idx[q];
        const int64_t sz = d->sizes[k], ss = d->src_strides[k], ds = d->dst_strides[k];
        if (sh.nd > 0) {
            const int l = sh.nd - 1;
            if (ds == sh.ds[l] * sh.size[l] && ss == sh.ss[l] * sh.size[l]) {
                sh.size[l] *= sz;
                continue;
            }
        }
        sh.size[sh.nd] = sz;
        sh.ss[sh.nd] = ss;
        sh.ds[sh.nd] = ds;
        ++sh.nd;
    }
    if (sh.nd == 0) {   // one element
        sh.nd = 1;
        sh.size[0] = 1;
        sh.ss[0] = 1;
        sh.ds[0] = 1;
    }
    const bool same = d->src_dtype == d->dst_dtype && d->src_dtype != TVK_BOOL;
    if (sh.nd == 1 && sh.ss[0] == 1 && sh.ds[0] == 1) {
        pl.kind = same ? PK_MEMCPY : PK_CAST_CONTIG;
        return TVK_OK;
    }
    pl.kind = PK_STRIDED;
    // one source element repeated into a dense destination (an expanded scalar)
    if (sh.nd == 1 && sh.ss[0] == 0 && sh.ds[0] == 1 && reinterpret_cast<uintptr_t>(d->dst) % dtype_size(d->dst_dtype) == 0) {
        pl.kind = PK_BROADCAST;
        return TVK_OK;
    }
    // same dtype, the innermost dimension contiguous on both sides in whole 16-byte vectors,
    // every run start 16-byte aligned, and a vector index that fits 32 bits
    if (same && sh.nd >= 2 && sh.ss[0] == 1 && sh.ds[0] == 1) {
        const int64_t es = (int64_t)dtype_size(d->src_dtype);
        bool ok = (sh.size[0] * es) % 16 == 0 && reinterpret_cast<uintptr_t>(d->src) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(d->dst) % 16 == 0 && numel * es / 16 < (int64_t(1) << 32);
        for (int k = 1; k < sh.nd && ok; ++k) ok = (sh.ss[k] * es) % 16 == 0 && (sh.ds[k] * es) % 16 == 0;
        if (ok) {
            pl.kind = PK_ROWS;
            return TVK_OK;
        }
    }
    if (sh.ds[0] == 1 && sh.ss[0] != 1 && sh.size[0] >= 8) {
        for (int k = 1; k < sh.nd; ++k)
            if (sh.ss[k] == 1 && sh.size[k] >= 8) {
                pl.kind = PK_TRANSPOSE;
                pl.j = k;
                break;
            }
    }
    return TVK_OK;
}

const char* plan_name(PlanKind k) {
    switch (k) {
        case PK_NONE: return "none";
        case PK_MEMCPY: return "memcpy";
        case PK_CAST_CONTIG: return "cast_contig";
        case PK_TRANSPOSE: return "transpose";
        case PK_BROADCAST: return "broadcast";
        case PK_ROWS: return "rows";
        default: return "strided";
    }
}

unsigned grid_for(int64_t items) {
    const int64_t blocks = (items + 255) / 256;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks, 65536));
}

// the raw-bits stand-in of a same-dtype copy: an integer type of the element's size
int raw_dtype(int dt) {
    switch (dtype_size(dt)) {
        case 8: return TVK_I64;
        case 4: return TVK_I32;
        case 2: return TVK_I16;
        default: return TVK_U8;
    }
}

template <int S, int D>
void launch_cast_contig_t(const char* s, char* d, int64_t n, hipStream_t st) {
    constexpr int SB = S == TVK_F64 ? 8 : S == TVK_F32 ? 4 : 2;
    constexpr int DB = D == TVK_F64 ? 8 : D == TVK_F32 ? 4 : 2;
    const bool vec = reinterpret_cast<uintptr_t>(s) % (SB * 8) == 0 && reinterpret_cast<uintptr_t>(d) % (DB * 8) == 0;
    const unsigned g = grid_for((n + 7) / 8);
    if (vec) hipLaunchKernelGGL((cast_contig_kernel<S, D, SB, DB, true>), dim3(g), dim3(256), 0, st, s, d, n, S, D);
    else hipLaunchKernelGGL((cast_contig_kernel<S, D, SB, DB, false>), dim3(g), dim3(256), 0, st, s, d, n, S, D);
}

template <int S>
bool launch_cast_contig_s(int ddt, const char* s, char* d, int64_t n, hipStream_t st) {
    switch (ddt) {
        case TVK_F32: launch_cast_contig_t<S, TVK_F32>(s, d, n, st); return true;
        case TVK_F16: launch_cast_contig_t<S, TVK_F16>(s, d, n, st); return true;
        case TVK_BF16: launch_cast_contig_t<S, TVK_BF16>(s, d, n, st); return true;
        case TVK_F64: launch_cast_contig_t<S, TVK_F64>(s, d, n, st); return true;
        default: return false;
    }
}

void launch_cast_contig(int sdt, int ddt, const char* s, char* d, int64_t n, hipStream_t st) {
    bool done = false;
    switch (sdt) {
        case TVK_F32: done = launch_cast_contig_s<TVK_F32>(ddt, s, d, n, st); break;
        case TVK_F16: done = launch_cast_contig_s<TVK_F16>(ddt, s, d, n, st); break;
        case TVK_BF16: done = launch_cast_contig_s<TVK_BF16>(ddt, s, d, n, st); break;
        case TVK_F64: done = launch_cast_contig_s<TVK_F64>(ddt, s, d, n, st); break;
        default: break;
    }
    if (!done)
        hipLaunchKernelGGL(cast_contig_dyn_kernel, dim3(grid_for(n)), dim3(256), 0, st, s, d, n, sdt, ddt,
                           (int)dtype_size(sdt), (int)dtype_size(ddt));
}

void launch_strided(const Plan& pl, int sdt, int ddt, const void* src, void* dst, hipStream_t st) {
    StridedArgs a{};
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    const bool same = sdt == ddt && sdt != TVK_BOOL;
    a.sdt = same ? raw_dtype(sdt) : sdt;
    a.ddt = same ? raw_dtype(ddt) : ddt;
    a.ss_bytes = (int)dtype_size(sdt);
    a.ds_bytes = (int)dtype_size(ddt);
    a.nd = pl.sh.nd;
    a.numel = pl.numel;
    bool idx32 = pl.numel <= 0xffffffffLL;
    for (int k = 0; k < a.nd; ++k) {
        a.size[k] = pl.sh.size[k];
        a.ss[k] = pl.sh.ss[k];
        a.ds[k] = pl.sh.ds[k];
        if (idx32) a.div[k] = make_div((uint32_t)pl.sh.size[k]);
    }
    const dim3 g(grid_for(pl.numel)), b(256);
#define TVK_STRIDED(S, D)                                                                            \
    do {                                                                                            \
        if (idx32) hipLaunchKernelGGL((copy_strided_kernel<S, D, true>), g, b, 0, st, a);          \
        else hipLaunchKernelGGL((copy_strided_kernel<S, D, false>), g, b, 0, st, a);               \
    } while (0)
    if (same) {
        switch (a.sdt) {
            case TVK_I64: TVK_STRIDED(TVK_I64, TVK_I64); break;
            case TVK_I32: TVK_STRIDED(TVK_I32, TVK_I32); break;
            case TVK_I16: TVK_STRIDED(TVK_I16, TVK_I16); break;
            default: TVK_STRIDED(TVK_U8, TVK_U8); break;
        }
    } else {
        TVK_STRIDED(DYN, DYN);
    }
#undef TVK_STRIDED
}

void launch_rows(const Plan& pl, int dt, const void* src, void* dst, hipStream_t st) {
    const int64_t es = (int64_t)dtype_size(dt);
    RowsArgs a{};
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    a.nd = pl.sh.nd - 1;
    a.nvec = pl.numel * es / 16;
    a.vdiv = make_div((uint32_t)(pl.sh.size[0] * es / 16));
    for (int k = 0; k < a.nd; ++k) {
        a.size[k] = pl.sh.size[k + 1];
        a.ss[k] = pl.sh.ss[k + 1] * es;
        a.ds[k] = pl.sh.ds[k + 1] * es;
        a.div[k] = make_div((uint32_t)pl.sh.size[k + 1]);
    }
    hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(a.nvec)), dim3(256), 0, st, a);
}

void launch_transpose(const Plan& pl, int sdt, int ddt, const void* src, void* dst, hipStream_t st) {
    TransposeArgs a{};
    a.src = static_cast<const char*>(src);
    a.dst = static_cast<char*>(dst);
    const bool same = sdt == ddt && sdt != TVK_BOOL;
    a.sdt = same ? raw_dtype(sdt) : sdt;
    a.ddt = same ? raw_dtype(ddt) : ddt;
    a.sb = (int)dtype_size(sdt);
    a.db = (int)dtype_size(ddt);
    const Shape& sh = pl.sh;
    a.n0 = sh.size[0];
    a.nj = sh.size[pl.j];
    a.ss0 = sh.ss[0];
    a.dsj = sh.ds[pl.j];
    a.tiles0 = (a.n0 + TT - 1) / TT;
    a.tilesj = (a.nj + TT - 1) / TT;
    a.nb = 0;
    int64_t blocks = a.tiles0 * a.tilesj;
    for (int k = 1; k < sh.nd; ++k) {
        if (k == pl.j) continue;
        a.bsize[a.nb] = sh.size[k];
        a.bss[a.nb] = sh.ss[k];
        a.bds[a.nb] = sh.ds[k];
        ++a.nb;
        blocks *= sh.size[k];
    }
    const dim3 g((unsigned)blocks), b(256);
    // 16-byte chunk starts on both sides: aligned bases and row strides
    auto a16 = [](uintptr_t v) { return v % 16 == 0; };
    const bool vec = a16(reinterpret_cast<uintptr_t>(src)) && a16(reinterpret_cast<uintptr_t>(dst)) &&
                     (a.ss0 * a.sb) % 16 == 0 && (a.dsj * a.db) % 16 == 0 && [&]() {
                         for (int k = 0; k < a.nb; ++k)
                             if ((a.bss[k] * a.sb) % 16 != 0 || (a.bds[k] * a.db) % 16 != 0) return false;
                         return true;
                     }();
    // 16-bit: the register kernel where dimension 0 spans more than one tile
    // (W.t() of a large matrix: 297 -> 224 us on 16384^2); the LDS kernel kept
    // its edge on a 64-wide dimension 0 (NCHW -> NHWC of 64 channels: 31 vs 32 us)
    if (vec && same && a.sb == 2 && a.n0 > TT) {
        // the tile counts are the 64 x 64 ones of the LDS kernels
        hipLaunchKernelGGL(copy_transpose_reg16_kernel, dim3((unsigned)((blocks + 3) / 4)), b, 0, st, a, blocks);
        return;
    }
    if (vec) {
#define TVK_TRV(S, D, W) hipLaunchKernelGGL((copy_transpose_vec_kernel<S, D, W>), g, b, 0, st, a)
        if (same) {
            switch (a.sdt) {
                case TVK_I64: TVK_TRV(TVK_I64, TVK_I64, uint64_t); return;
                case TVK_I32: TVK_TRV(TVK_I32, TVK_I32, uint32_t); return;
                case TVK_I16: TVK_TRV(TVK_I16, TVK_I16, uint32_t); return;
                default: TVK_TRV(TVK_U8, TVK_U8, uint32_t); return;
            }
        }
        if (sdt == TVK_F32 && ddt == TVK_F16) { TVK_TRV(TVK_F32, TVK_F16, uint32_t); return; }
        if (sdt == TVK_F32 && ddt == TVK_BF16) { TVK_TRV(TVK_F32, TVK_BF16, uint32_t); return; }
        if (sdt == TVK_F16 && ddt == TVK_F32) { TVK_TRV(TVK_F16, TVK_F32, uint32_t); return; }
        if (sdt == TVK_BF16 && ddt == TVK_F32) { TVK_TRV(TVK_BF16, TVK_F32, uint32_t); return; }
#undef TVK_TRV
    }
#define TVK_TR(S, D, W) hipLaunchKernelGGL((copy_transpose_kernel<S, D, W>), g, b, 0, st, a)
    if (same) {
        switch (a.sdt) {
            case TVK_I64: TVK_TR(TVK_I64, TVK_I64, uint64_t); break;
            case TVK_I32: TVK_TR(TVK_I32, TVK_I32, uint32_t); break;
            case TVK_I16: TVK_TR(TVK_I16, TVK_I16, uint32_t); break;
            default: TVK_TR(TVK_U8, TVK_U8, uint32_t); break;
        }
    } else if (sdt == TVK_F32 && ddt == TVK_F16) TVK_TR(TVK_F32, TVK_F16, uint32_t);
    else if (sdt == TVK_F32 && ddt == TVK_BF16) TVK_TR(TVK_F32, TVK_BF16, uint32_t);
    else if (sdt == TVK_F16 && ddt == TVK_F32) TVK_TR(TVK_F16, TVK_F32, uint32_t);
    else if (sdt == TVK_BF16 && ddt == TVK_F32) TVK_TR(TVK_BF16, TVK_F32, uint32_t);
    else TVK_TR(DYN, DYN, uint64_t);
#undef TVK_TR
}

// ---------------------------------------------------------------------------
// fill
// ---------------------------------------------------------------------------

// Dense fill: 16-byte stores of the repeated pattern; the elements before the
// first 16-byte boundary and after the last are stored one by one.
template <typename E>
__device__ __forceinline__ void fill_body(E* dst, int64_t n, int64_t head, E v) {
    constexpr int PER = 16 / sizeof(E);
    const int64_t step = (int64_t)gridDim.x * 256;
    const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (tid < head && tid < n) dst[tid] = v;
    const int64_t body = (n - head) / PER;
    struct alignas(16) V16 { E e[PER]; };
    V16 vv;
#pragma unroll
    for (int i = 0; i < PER; ++i) vv.e[i] = v;
    V16* vd = reinterpret_cast<V16*>(dst + head);
    for (int64_t i = tid; i < body; i += step) vd[i] = vv;
    const int64_t tail0 = head + body * PER;
    if (tail0 + tid < n) dst[tail0 + tid] = v;
}

template <typename E>
__global__ __launch_bounds__(256) void fill_contig_kernel(E* dst, int64_t n, int64_t head, E v) {
    fill_body<E>(dst, n, head, v);
}

// A copy whose source is one element (stride 0 along every dimension, an
// expanded scalar) into a dense destination: every thread converts the
// element and stores it as the fill kernel does.
template <typename E>
__global__ __launch_bounds__(256) void broadcast_contig_kernel(const char* src, int sdt, int ddt, E* dst, int64_t n,
                                                               int64_t head) {
    alignas(8) char tmp[8];
    convert(src, sdt, tmp, ddt);
    E v;
    __builtin_memcpy(&v, tmp, sizeof(E));
    fill_body<E>(dst, n, head, v);
}

// Elements before dst's first 16-byte boundary, and the threads that cover
// the 16-byte body, the head and the tail.
template <typename E>
void dense_fill_geometry(const void* dst, int64_t numel, int64_t& head, int64_t& threads) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(dst);
    head = std::min<int64_t>((int64_t)(((16 - a % 16) % 16) / sizeof(E)), numel);
    threads = std::max<int64_t>((numel - head) / (16 / sizeof(E)), std::max<int64_t>(head, 16));
}

template <typename E>
void launch_broadcast_t(const char* src, int sdt, int ddt, void* dst, int64_t numel, hipStream_t st) {
    int64_t head, threads;
    dense_fill_geometry<E>(dst, numel, head, threads);
    hipLaunchKernelGGL(broadcast_contig_kernel<E>, dim3(grid_for(threads)), dim3(256), 0, st, src, sdt, ddt,
                       static_cast<E*>(dst), numel, head);
}

void launch_broadcast(const Plan& pl, int sdt, int ddt, const void* src, void* dst, hipStream_t st) {
    const bool same = sdt == ddt && sdt != TVK_BOOL;
    const int s = same ? raw_dtype(sdt) : sdt, d = same ? raw_dtype(ddt) : ddt;
    const char* sp = static_cast<const char*>(src);
    switch (dtype_size(ddt)) {
        case 8: launch_broadcast_t<uint64_t>(sp, s, d, dst, pl.numel, st); break;
        case 4: launch_broadcast_t<uint32_t>(sp, s, d, dst, pl.numel, st); break;
        case 2: launch_broadcast_t<uint16_t>(sp, s, d, dst, pl.numel, st); break;
        default: launch_broadcast_t<uint8_t>(sp, s, d, dst, pl.numel, st); break;
    }
}

template <typename E>
__global__ __launch_bounds__(256) void fill_strided_kernel(char* dst, int nd, int64_t numel, StridedArgs p, E v) {
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t li = (int64_t)blockIdx.x * 256 + threadIdx.x; li < numel; li += step) {
        int64_t rem = li, off = 0;
#pragma unroll 1
        for (int k = 0; k < nd - 1; ++k) {
            const int64_t q = rem / p.size[k];
            off += (rem - q * p.size[k]) * p.ds[k];
            rem = q;
        }
        off += rem * p.ds[nd - 1];
        reinterpret_cast<E*>(dst)[off] = v;
    }
}

template <typename E>
void launch_fill(const Plan& pl, void* dst, uint64_t pattern, hipStream_t st) {
    E v;
    std::memcpy(&v, &pattern, sizeof(E));
    if (pl.sh.nd == 1 && pl.sh.ds[0] == 1) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(dst);
        int64_t head = (int64_t)(((16 - a % 16) % 16) / sizeof(E));
        if (a % sizeof(E) != 0) head = pl.numel;   // misaligned elements: the head covers everything
        if (head > pl.numel) head = pl.numel;
        const int64_t threads = std::max<int64_t>((pl.numel - head) / (16 / sizeof(E)), std::max<int64_t>(head, 16));
        if (head > 256 * 65536LL) {
            // element-wise: one element per thread in a grid-stride loop
            StridedArgs p{};
            p.size[0] = pl.numel;
            p.ds[0] = 1;
            hipLaunchKernelGGL(fill_strided_kernel<E>, dim3(grid_for(pl.numel)), dim3(256), 0, st,
                               static_cast<char*>(dst), 1, pl.numel, p, v);
            return;
        }
        hipLaunchKernelGGL(fill_contig_kernel<E>, dim3(grid_for(threads)), dim3(256), 0, st, static_cast<E*>(dst), pl.numel,
                           head, v);
        return;
    }
    StridedArgs p{};
    for (int k = 0; k < pl.sh.nd; ++k) {
        p.size[k] = pl.sh.size[k];
        p.ds[k] = pl.sh.ds[k];
    }
    hipLaunchKernelGGL(fill_strided_kernel<E>, dim3(grid_for(pl.numel)), dim3(256), 0, st, static_cast<char*>(dst),
                       pl.sh.nd, pl.numel, p, v);
}

}  // namespace
}  // namespace tvk

using namespace tvk;

extern "C" tvk_status tvk_fill(const tvk_fill_desc* desc) {
    if (!desc) return fail(TVK_ERR_INVALID, "tvk_fill: desc is NULL");
    const int es = desc->elem_size;
    if (es != 1 && es != 2 && es != 4 && es != 8)
        return fail(TVK_ERR_INVALID, "tvk_fill: elem_size must be 1, 2, 4 or 8");
    // the destination's dimensions merge as a same-dtype copy's would
    tvk_copy_desc c;
    std::memset(&c, 0, sizeof(c));
    c.src_dtype = c.dst_dtype = es == 8 ? TVK_I64 : es == 4 ? TVK_I32 : es == 2 ? TVK_I16 : TVK_U8;
    c.ndim = desc->ndim;
    for (int k = 0; k < desc->ndim && k < kMaxDims; ++k) {
        c.sizes[k] = desc->sizes[k];
        c.dst_strides[k] = desc->dst_strides[k];
        c.src_strides[k] = desc->dst_strides[k];
    }
    c.src = desc->dst;
    c.dst = desc->dst;
    Plan pl;
    tvk_status st = make_plan(&c, pl, "tvk_fill");
    if (st != TVK_OK) return st;
    if (pl.kind == PK_NONE) return TVK_OK;
    const hipStream_t s = resolve_stream(desc->stream);
    switch (es) {
        case 1: launch_fill<uint8_t>(pl, desc->dst, desc->pattern, s); break;
        case 2: launch_fill<uint16_t>(pl, desc->dst, desc->pattern, s); break;
        case 4: launch_fill<uint32_t>(pl, desc->dst, desc->pattern, s); break;
        default: launch_fill<uint64_t>(pl, desc->dst, desc->pattern, s); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_fill: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

extern "C" tvk_status tvk_copy_plan(const tvk_copy_desc* desc, char* name, size_t name_len) {
    Plan pl;
    tvk_status st = make_plan(desc, pl, "tvk_copy_plan");
    if (st != TVK_OK) return st;
    if (!name || name_len == 0) return fail(TVK_ERR_INVALID, "tvk_copy_plan: name buffer is empty");
    std::strncpy(name, plan_name(pl.kind), name_len - 1);
    name[name_len - 1] = '\0';
    return TVK_OK;
}

extern "C" tvk_status tvk_copy(const tvk_copy_desc* desc) {
    Plan pl;
    tvk_status st = make_plan(desc, pl, "tvk_copy");
    if (st != TVK_OK) return st;
    if (pl.kind == PK_NONE) return TVK_OK;
    // grid x of the transpose kernel is one block per tile and batch index
    if (pl.kind == PK_TRANSPOSE) {
        const Shape& sh = pl.sh;
        int64_t blocks = ((sh.size[0] + TT - 1) / TT) * ((sh.size[pl.j] + TT - 1) / TT);
        for (int k = 1; k < sh.nd; ++k)
            if (k != pl.j) blocks *= sh.size[k];
        if (blocks > 0x7fffffffLL) pl.kind = PK_STRIDED;
    }
    const hipStream_t s = resolve_stream(desc->stream);
    const int sdt = desc->src_dtype, ddt = desc->dst_dtype;
    switch (pl.kind) {
        case PK_MEMCPY:
            TVK_HIP_CHECK(hipMemcpyAsync(desc->dst, desc->src, (size_t)pl.numel * dtype_size(sdt), hipMemcpyDeviceToDevice, s));
            return TVK_OK;
        case PK_CAST_CONTIG:
            launch_cast_contig(sdt, ddt, static_cast<const char*>(desc->src), static_cast<char*>(desc->dst), pl.numel, s);
            break;
        case PK_TRANSPOSE:
            launch_transpose(pl, sdt, ddt, desc->src, desc->dst, s);
            break;
        case PK_BROADCAST:
            launch_broadcast(pl, sdt, ddt, desc->src, desc->dst, s);
            break;
        case PK_ROWS:
            launch_rows(pl, sdt, desc->src, desc->dst, s);
            break;
        default:
            launch_strided(pl, sdt, ddt, desc->src, desc->dst, s);
            break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_copy: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}
