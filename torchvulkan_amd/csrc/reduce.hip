// Sum reduction (tvk_reduce_sum) and element-wise add/sub/mul (tvk_binary):
// the reductions and adds around the contractions (bias gradients,
// gradient accumulation, residual adds).
//
// Reference semantics:
//   sum: sum_accumulated (src/api/ops/reduce.cpp:265-273) converts the input
//     to the accumulate dtype (float32 for a float16/bfloat16 result, else the
//     result's own, src/api/ops/helpers.h:466-480), sums, and casts the total
//     to the result dtype.
//   add/sub/mul: AddOp/SubOp/MulOp (src/shaders/ops/binary.slang:39-55) in the
//     tensor dtype: T.ext_add(a, T.ext_mul(alpha, b)) when alpha != 1, with
//     float16/bfloat16 computing each operation in float32 and rounding back
//     (src/shaders/core/dtype.slang:911-913).
//
// Sum plan. The reduced dimensions and the kept ones are each sorted by
// source stride and merged where contiguous, then:
//   row mode (the source's innermost dimension is reduced): one 256-thread
//     block per output and K chunk; the threads walk the chunk in memory order,
//     then a fixed-shape tree in LDS adds their 256 partial sums (a float
//     source over one contiguous dimension: 16-byte loads, four in flight);
//   column mode (the innermost dimension is kept): one thread per output,
//     neighbouring threads on neighbouring outputs (coalesced), each adding
//     its K chunk in order.
// When the outputs alone cannot fill the device, K is cut into chunks whose
// partial sums (in the accumulate type) are added by a second pass in chunk
// order (for a few outputs of many chunks, 256 threads an output and a tree).
// A column sum of at most 1024 rows that would be chunked runs in one launch
// instead: row groups of one workgroup, then a tree over the groups.
// Every order is fixed, so a sum gives the same bits on every run.
#include "convert.h"

#include <algorithm>
#include <cstring>
#include <type_traits>

namespace tvk {
namespace {

// ---------------------------------------------------------------------------
// accumulate types
// ---------------------------------------------------------------------------

template <typename Acc> struct AccOps;
template <> struct AccOps<float> {
    __device__ static inline float from(const Wide& w, int fam) { return wide_to_f32(w, fam); }
    static constexpr int dtype = TVK_F32;
};
template <> struct AccOps<double> {
    __device__ static inline double from(const Wide& w, int fam) { return wide_to_f64(w, fam); }
    static constexpr int dtype = TVK_F64;
};
template <> struct AccOps<int64_t> {
    __device__ static inline int64_t from(const Wide& w, int fam) { return wide_to_int<int64_t>(w, fam); }
    static constexpr int dtype = TVK_I64;
};

// src element -> accumulate type, as src.to(acc_dtype) does
template <typename Acc>
__device__ __forceinline__ Acc load_acc(const char* p, int sdt) {
    Wide w = load_wide(p, sdt);
    int fam = family(sdt);
    if (sdt == TVK_BOOL) {
        w.i = w.u != 0 ? 1 : 0;
        fam = FAM_I;
    }
    return AccOps<Acc>::from(w, fam);
}

// accumulate type -> dst element (castValue from the accumulate dtype)
template <typename Acc>
__device__ __forceinline__ void store_acc(char* p, int ddt, Acc v) {
    alignas(8) char tmp[8];
    *reinterpret_cast<Acc*>(tmp) = v;
    convert(tmp, AccOps<Acc>::dtype, p, ddt);
}

struct RedArgs {
    const char* src;
    char* dst;           // final output, or the partial buffer (acc type)
    int sdt, ddt;        // ddt < 0: write partials
    int sb, db;          // element sizes (db of the final output)
    int nk, nr;          // kept / reduced dimension counts
    int64_t nout;        // kept elements
    int64_t nred;        // reduced elements
    int64_t chunk;       // reduced elements per split
    int splits;
    Div32 kdiv[kMaxDims], rdiv[kMaxDims];
    int64_t ksize[kMaxDims], kss[kMaxDims], kds[kMaxDims];
    int64_t rsize[kMaxDims], rss[kMaxDims];
    bool idx32;          // every index fits 32 bits
};

__device__ __forceinline__ void kept_offsets(const RedArgs& p, int64_t o, int64_t& so, int64_t& dof) {
    so = 0;
    dof = 0;
    if (p.idx32) {
        uint32_t rem = (uint32_t)o;
        for (int k = 0; k < p.nk - 1; ++k) {
            const uint32_t q = div32(rem, p.kdiv[k]);
            const uint32_t c = rem - q * p.kdiv[k].d;
            so += (int64_t)c * p.kss[k];
            dof += (int64_t)c * p.kds[k];
            rem = q;
        }
        if (p.nk > 0) {
            so += (int64_t)rem * p.kss[p.nk - 1];
            dof += (int64_t)rem * p.kds[p.nk - 1];
        }
    } else {
        int64_t rem = o;
        for (int k = 0; k < p.nk - 1; ++k) {
            const int64_t q = rem / p.ksize[k], c = rem - q * p.ksize[k];
            so += c * p.kss[k];
            dof += c * p.kds[k];
            rem = q;
        }
        if (p.nk > 0) {
            so += rem * p.kss[p.nk - 1];
            dof += rem * p.kds[p.nk - 1];
        }
    }
}

__device__ __forceinline__ int64_t red_offset(const RedArgs& p, int64_t r) {
    if (p.nr == 1) return r * p.rss[0];
    int64_t off = 0;
    if (p.idx32) {
        uint32_t rem = (uint32_t)r;
        for (int k = 0; k < p.nr - 1; ++k) {
            const uint32_t q = div32(rem, p.rdiv[k]);
            off += (int64_t)(rem - q * p.rdiv[k].d) * p.rss[k];
            rem = q;
        }
        return off + (int64_t)rem * p.rss[p.nr - 1];
    }
    int64_t rem = r;
    for (int k = 0; k < p.nr - 1; ++k) {
        const int64_t q = rem / p.rsize[k];
        off += (rem - q * p.rsize[k]) * p.rss[k];
        rem = q;
    }
    return off + rem * p.rss[p.nr - 1];
}

// the result of output o (chunk z of `splits`) goes to the final output or
// to the partial buffer laid out [z][o]
template <typename Acc>
__device__ __forceinline__ void put(const RedArgs& p, int64_t o, int64_t dof, int z, Acc v) {
    if (p.ddt < 0) reinterpret_cast<Acc*>(p.dst)[(int64_t)z * p.nout + o] = v;
    else store_acc<Acc>(p.dst + dof * p.db, p.ddt, v);
}

template <typename Acc, int SDT>
__global__ __launch_bounds__(256) void reduce_row_kernel(RedArgs p) {
    const int sdt = SDT == DYN ? p.sdt : SDT;
    __shared__ Acc red[256];
    const int z = blockIdx.y;
    const int64_t r0 = (int64_t)z * p.chunk;
    const int64_t r1 = r0 + p.chunk < p.nred ? r0 + p.chunk : p.nred;
    for (int64_t o = blockIdx.x; o < p.nout; o += gridDim.x) {
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        Acc acc = 0;
        for (int64_t r = r0 + threadIdx.x; r < r1; r += 256) acc += load_acc<Acc>(p.src + (so + red_offset(p, r)) * p.sb, sdt);
        red[threadIdx.x] = acc;
        __syncthreads();
#pragma unroll
        for (int w = 128; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) put<Acc>(p, o, dof, z, red[0]);
        __syncthreads();
    }
}

// Row mode over one contiguous reduced dimension, V = 16/sb elements a
// 16-byte load: thread t adds vectors t, t + 256, ... of its chunk (four
// loads in flight), each vector's elements in order; then the same tree as
// reduce_row_kernel. The chunk and nred are whole vectors.
template <typename Acc, int SDT>
__global__ __launch_bounds__(256) void reduce_rowv_kernel(RedArgs p) {
    constexpr int SB = (int)dtype_size(SDT), V = 16 / SB;
    struct alignas(16) V16 { char c[16]; };
    __shared__ Acc red[256];
    const int z = blockIdx.y;
    const int64_t r0 = (int64_t)z * p.chunk;
    const int64_t r1 = r0 + p.chunk < p.nred ? r0 + p.chunk : p.nred;
    const int64_t nv = (r1 - r0) / V;
    for (int64_t o = blockIdx.x; o < p.nout; o += gridDim.x) {
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        const V16* src = reinterpret_cast<const V16*>(p.src + (so + r0) * SB);
        Acc acc = 0;
        int64_t v = threadIdx.x;
        for (; v + 3 * 256 < nv; v += 4 * 256) {
            V16 w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) w[u] = src[v + u * 256];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc += load_acc<Acc>(w[u].c + e * SB, SDT);
        }
        {
            // the last vectors (fewer than four): every load issued before the first add
            V16 w[3];
#pragma unroll
            for (int u = 0; u < 3; ++u)
                if (v + u * 256 < nv) w[u] = src[v + u * 256];
#pragma unroll
            for (int u = 0; u < 3; ++u)
                if (v + u * 256 < nv)
#pragma unroll
                    for (int e = 0; e < V; ++e) acc += load_acc<Acc>(w[u].c + e * SB, SDT);
        }
        red[threadIdx.x] = acc;
        __syncthreads();
#pragma unroll
        for (int w = 128; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) put<Acc>(p, o, dof, z, red[0]);
        __syncthreads();
    }
}

template <typename Acc, int SDT>
__global__ __launch_bounds__(256) void reduce_col_kernel(RedArgs p) {
    const int sdt = SDT == DYN ? p.sdt : SDT;
    const int z = blockIdx.y;
    const int64_t r0 = (int64_t)z * p.chunk;
    const int64_t r1 = r0 + p.chunk < p.nred ? r0 + p.chunk : p.nred;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < p.nout; o += (int64_t)gridDim.x * 256) {
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        Acc acc = 0;
        for (int64_t r = r0; r < r1; ++r) acc += load_acc<Acc>(p.src + (so + red_offset(p, r)) * p.sb, sdt);
        put<Acc>(p, o, dof, z, acc);
    }
}

// Column mode with V = 16/sb consecutive outputs per thread along the
// source's contiguous kept dimension: one 16-byte load per row and four rows
// in flight per thread. Each output still adds its rows in order.
template <typename Acc, int SDT>
__global__ __launch_bounds__(256) void reduce_colv_kernel(RedArgs p) {
    constexpr int SB = (int)dtype_size(SDT), V = 16 / SB;
    struct alignas(16) V16 { char c[16]; };
    const int z = blockIdx.y;
    const int64_t r0 = (int64_t)z * p.chunk;
    const int64_t r1 = r0 + p.chunk < p.nred ? r0 + p.chunk : p.nred;
    const int64_t nvec = p.nout / V;
    for (int64_t ov = (int64_t)blockIdx.x * 256 + threadIdx.x; ov < nvec; ov += (int64_t)gridDim.x * 256) {
        const int64_t o = ov * V;
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        Acc acc[V];
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] = 0;
        int64_t r = r0;
        for (; r + 4 <= r1; r += 4) {
            V16 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const V16*>(p.src + (so + red_offset(p, r + u)) * SB);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += load_acc<Acc>(v[u].c + e * SB, SDT);
        }
        for (; r < r1; ++r) {
            const V16 v = *reinterpret_cast<const V16*>(p.src + (so + red_offset(p, r)) * SB);
#pragma unroll
            for (int e = 0; e < V; ++e) acc[e] += load_acc<Acc>(v.c + e * SB, SDT);
        }
#pragma unroll
        for (int e = 0; e < V; ++e) put<Acc>(p, o + e, dof + e * p.kds[0], z, acc[e]);
    }
}

// Column mode for short reductions (a bias gradient: [256, 4096] summed over
// the rows) in one launch: a workgroup takes CV = 256 / RG consecutive
// 16-byte column vectors; thread group g adds rows g, g + RG, ... of its
// vector in order (eight loads in flight), then the RG group sums are added
// in a fixed tree through LDS. (The chunked form ran a column kernel over 16
// row chunks and a second launch to fold them.)
template <typename Acc, int SDT, int RG>
__global__ __launch_bounds__(256) void reduce_colw_kernel(RedArgs p) {
    constexpr int SB = (int)dtype_size(SDT), V = 16 / SB, CV = 256 / RG;
    struct alignas(16) V16 { char c[16]; };
    __shared__ Acc red[RG][CV * V + 1];   // + 1: a row's groups on different banks
    const int v = threadIdx.x % CV, g = threadIdx.x / CV;
    const int64_t ov = (int64_t)blockIdx.x * CV + v;
    const bool live = ov < p.nout / V;
    int64_t so = 0, dof = 0;
    Acc acc[V];
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = 0;
    if (live) {
        kept_offsets(p, ov * V, so, dof);
        int64_t r = g;
        for (; r + 7 * RG < p.nred; r += 8 * RG) {
            V16 w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const V16*>(p.src + (so + red_offset(p, r + u * RG)) * SB);
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += load_acc<Acc>(w[u].c + e * SB, SDT);
        }
        {
            // the last rows (fewer than eight): every load issued before the first add
            V16 w[7];
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (r + u * RG < p.nred) w[u] = *reinterpret_cast<const V16*>(p.src + (so + red_offset(p, r + u * RG)) * SB);
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (r + u * RG < p.nred)
#pragma unroll
                    for (int e = 0; e < V; ++e) acc[e] += load_acc<Acc>(w[u].c + e * SB, SDT);
        }
    }
#pragma unroll
    for (int e = 0; e < V; ++e) red[g][v * V + e] = acc[e];
    __syncthreads();
#pragma unroll
    for (int w = RG / 2; w > 0; w >>= 1) {
        if (g < w)
#pragma unroll
            for (int e = 0; e < V; ++e) red[g][v * V + e] = red[g][v * V + e] + red[g + w][v * V + e];
        __syncthreads();
    }
    if (g == 0 && live)
#pragma unroll
        for (int e = 0; e < V; ++e) store_acc<Acc>(p.dst + (dof + e * p.kds[0]) * p.db, p.ddt, red[0][v * V + e]);
}

// dst[o] = sum over z of part[z][o], in z order; neighbouring threads read
// neighbouring partials, eight chunks in flight per thread
template <typename Acc>
__global__ __launch_bounds__(256) void reduce_fold_kernel(const Acc* part, RedArgs p) {
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < p.nout; o += (int64_t)gridDim.x * 256) {
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        Acc v = part[o];
        int z = 1;
        for (; z + 8 <= p.splits; z += 8) {
            Acc w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = part[(int64_t)(z + u) * p.nout + o];
#pragma unroll
            for (int u = 0; u < 8; ++u) v += w[u];
        }
        {
            // the last chunks (fewer than eight): every load issued before the first add
            Acc w[7];
            const int rem = p.splits - z;
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (u < rem) w[u] = part[(int64_t)(z + u) * p.nout + o];
#pragma unroll
            for (int u = 0; u < 7; ++u)
                if (u < rem) v += w[u];
        }
        store_acc<Acc>(p.dst + dof * p.db, p.ddt, v);
    }
}

// The same sum for many splits: a workgroup takes 32 consecutive outputs,
// its 8 thread groups sum the splits z = g, g + 8, ... (eight loads in flight
// a thread), and the group sums are added in group order through LDS. (One
// thread an output left a 3072-output, 256-split fold to 12 workgroups and
// 32 dependent rounds of loads.)
template <typename Acc>
__global__ __launch_bounds__(256) void reduce_fold8_kernel(const Acc* part, RedArgs p) {
    __shared__ Acc red[8][32];
    const int l = threadIdx.x % 32, g = threadIdx.x / 32;
    const int64_t o = (int64_t)blockIdx.x * 32 + l;
    Acc v = 0;
    if (o < p.nout) {
        int z = g;
        for (; z + 56 < p.splits; z += 64) {
            Acc w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = part[(int64_t)(z + 8 * u) * p.nout + o];
#pragma unroll
            for (int u = 0; u < 8; ++u) v += w[u];
        }
        // the last chunks of this group (fewer than eight): every load issued before the first add
        Acc w[7];
#pragma unroll
        for (int u = 0; u < 7; ++u)
            if (z + 8 * u < p.splits) w[u] = part[(int64_t)(z + 8 * u) * p.nout + o];
#pragma unroll
        for (int u = 0; u < 7; ++u)
            if (z + 8 * u < p.splits) v += w[u];
    }
    red[g][l] = v;
    __syncthreads();
    if (g == 0 && o < p.nout) {
        Acc t = red[0][l];
#pragma unroll
        for (int q = 1; q < 8; ++q) t += red[q][l];
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        store_acc<Acc>(p.dst + dof * p.db, p.ddt, t);
    }
}

// The same sum for few outputs and many splits (a whole tensor summed to one
// value): one workgroup an output; thread t adds splits t, t + 256, ...
// (eight loads in flight), then a tree over the 256 thread sums in a fixed
// order. (The 32-output fold left such a sum to eight threads.)
template <typename Acc>
__global__ __launch_bounds__(256) void reduce_foldw_kernel(const Acc* part, RedArgs p) {
    __shared__ Acc red[256];
    const int64_t o = blockIdx.x;
    Acc v = 0;
    int z = threadIdx.x;
    for (; z + 7 * 256 < p.splits; z += 8 * 256) {
        Acc w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = part[(int64_t)(z + u * 256) * p.nout + o];
#pragma unroll
        for (int u = 0; u < 8; ++u) v += w[u];
    }
    {
        Acc w[7];
#pragma unroll
        for (int u = 0; u < 7; ++u)
            if (z + u * 256 < p.splits) w[u] = part[(int64_t)(z + u * 256) * p.nout + o];
#pragma unroll
        for (int u = 0; u < 7; ++u)
            if (z + u * 256 < p.splits) v += w[u];
    }
    red[threadIdx.x] = v;
    __syncthreads();
#pragma unroll
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        store_acc<Acc>(p.dst + dof * p.db, p.ddt, red[0]);
    }
}

// An empty sum: every output is castValue(0), all-zero bytes in every dtype.
__global__ __launch_bounds__(256) void reduce_zero_kernel(RedArgs p) {
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < p.nout; o += (int64_t)gridDim.x * 256) {
        int64_t so, dof;
        kept_offsets(p, o, so, dof);
        for (int b = 0; b < p.db; ++b) p.dst[dof * p.db + b] = 0;
    }
}

unsigned blocks_for(int64_t n, int64_t per) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + per - 1) / per, 65535));
}

// column mode can take V = 16/sb outputs per thread: the source dtype is a
// float one, the kept dimension 0 is the source's contiguous one with a
// multiple of V elements, and every chunk start is 16-byte aligned
bool colv_applies(const RedArgs& p) {
    if (p.sdt != TVK_F32 && p.sdt != TVK_F16 && p.sdt != TVK_BF16) return false;
    const int v = 16 / p.sb;
    if (p.nk == 0 || p.kss[0] != 1 || p.ksize[0] % v != 0 || reinterpret_cast<uintptr_t>(p.src) % 16 != 0) return false;
    for (int k = 1; k < p.nk; ++k)
        if ((p.kss[k] * p.sb) % 16 != 0) return false;
    for (int k = 0; k < p.nr; ++k)
        if ((p.rss[k] * p.sb) % 16 != 0) return false;
    return true;
}

// row mode with 16-byte loads: a float source reduced over one contiguous
// dimension of whole vectors, every output's row start 16-byte aligned
bool rowv_applies(const RedArgs& p) {
    if (p.sdt != TVK_F32 && p.sdt != TVK_F16 && p.sdt != TVK_BF16) return false;
    const int v = 16 / p.sb;
    if (p.nr != 1 || p.rss[0] != 1 || p.nred % v != 0 || reinterpret_cast<uintptr_t>(p.src) % 16 != 0) return false;
    for (int k = 0; k < p.nk; ++k)
        if ((p.kss[k] * p.sb) % 16 != 0) return false;
    return true;
}

template <typename Acc>
tvk_status run_sum(RedArgs& p, bool row, int dev, hipStream_t st) {
    const bool colv = !row && colv_applies(p);
    const bool rowv = row && rowv_applies(p);
    const int64_t per_thread = colv ? 16 / p.sb : 1;
    // split K when the outputs alone would leave the device short of blocks
    const int64_t out_blocks = row ? p.nout : (p.nout / per_thread + 255) / 256;
    if (colv && out_blocks < 1024 && p.nred <= 1024) {
        // a short column sum over few outputs: one launch, row groups of a
        // workgroup (about four rows a thread: 64 groups up to 256 rows)
        p.splits = 1;
        p.chunk = p.nred;
        const int64_t nvec = p.nout / per_thread;
        auto go = [&](auto rg_c) {
            constexpr int RG = decltype(rg_c)::value;
            const dim3 grid((unsigned)((nvec + 256 / RG - 1) / (256 / RG)));
            if (p.sdt == TVK_F32) hipLaunchKernelGGL((reduce_colw_kernel<Acc, TVK_F32, RG>), grid, dim3(256), 0, st, p);
            else if (p.sdt == TVK_F16) hipLaunchKernelGGL((reduce_colw_kernel<Acc, TVK_F16, RG>), grid, dim3(256), 0, st, p);
            else hipLaunchKernelGGL((reduce_colw_kernel<Acc, TVK_BF16, RG>), grid, dim3(256), 0, st, p);
        };
        if (p.nred <= 256) go(std::integral_constant<int, 64>{});
        else go(std::integral_constant<int, 128>{});
        return TVK_OK;
    }
    int64_t splits = 1;
    if (out_blocks < 1024 && p.nred > 1) {
        const int64_t want = (1024 + out_blocks - 1) / out_blocks;
        // rowv: four 16-byte loads a thread per chunk
        const int64_t min_chunk = rowv ? 1024 * (16 / p.sb) : row ? 4096 : 256;
        splits = std::min<int64_t>(want, (p.nred + min_chunk - 1) / min_chunk);
        // a short column reduction over few outputs (a bias gradient, [256, 4096]
        // summed over dim 0: two workgroups) takes chunks of 16 rows instead, so
        // more workgroups read it; long ones keep the 256-row chunks
        if (!row && splits < 8 && p.nred >= 32) splits = std::min<int64_t>(want, p.nred / 16);
        splits = std::max<int64_t>(1, std::min<int64_t>(splits, 65535));
    }
    p.chunk = (p.nred + splits - 1) / splits;
    if (rowv) {   // whole vectors a chunk
        const int64_t v = 16 / p.sb;
        p.chunk = (p.chunk + v - 1) / v * v;
    }
    splits = (p.nred + p.chunk - 1) / p.chunk;
    p.splits = (int)splits;
    const int ddt = p.ddt;
    char* final_dst = p.dst;
    Acc* part = nullptr;
    Scratch scratch;
    if (splits > 1) {
        part = static_cast<Acc*>(scratch.get((size_t)(p.nout * splits) * sizeof(Acc), st));
        if (!part) return fail(TVK_ERR_OOM, "tvk_reduce_sum: workspace allocation failed");
        p.dst = reinterpret_cast<char*>(part);
        p.ddt = -1;
    }
    const dim3 grid(row ? blocks_for(p.nout, 1) : blocks_for(p.nout / per_thread, 256), (unsigned)splits);
#define TVK_RED(S)                                                                      \
    do {                                                                                \
        if (row) hipLaunchKernelGGL((reduce_row_kernel<Acc, S>), grid, dim3(256), 0, st, p); \
        else hipLaunchKernelGGL((reduce_col_kernel<Acc, S>), grid, dim3(256), 0, st, p);     \
    } while (0)
    if (rowv) {
        if (p.sdt == TVK_F32) hipLaunchKernelGGL((reduce_rowv_kernel<Acc, TVK_F32>), grid, dim3(256), 0, st, p);
        else if (p.sdt == TVK_F16) hipLaunchKernelGGL((reduce_rowv_kernel<Acc, TVK_F16>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((reduce_rowv_kernel<Acc, TVK_BF16>), grid, dim3(256), 0, st, p);
    } else if (colv) {
        if (p.sdt == TVK_F32) hipLaunchKernelGGL((reduce_colv_kernel<Acc, TVK_F32>), grid, dim3(256), 0, st, p);
        else if (p.sdt == TVK_F16) hipLaunchKernelGGL((reduce_colv_kernel<Acc, TVK_F16>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((reduce_colv_kernel<Acc, TVK_BF16>), grid, dim3(256), 0, st, p);
    } else switch (p.sdt) {
        case TVK_F32: TVK_RED(TVK_F32); break;
        case TVK_F16: TVK_RED(TVK_F16); break;
        case TVK_BF16: TVK_RED(TVK_BF16); break;
        default: TVK_RED(DYN); break;
    }
#undef TVK_RED
    if (splits > 1) {
        p.dst = final_dst;
        p.ddt = ddt;
        if (splits >= 256 && p.nout <= 64) hipLaunchKernelGGL(reduce_foldw_kernel<Acc>, dim3((unsigned)p.nout), dim3(256), 0, st, part, p);
        else if (splits >= 32) hipLaunchKernelGGL(reduce_fold8_kernel<Acc>, dim3((unsigned)((p.nout + 31) / 32)), dim3(256), 0, st, part, p);
        else hipLaunchKernelGGL(reduce_fold_kernel<Acc>, dim3(blocks_for(p.nout, 256)), dim3(256), 0, st, part, p);
    }
    return TVK_OK;
}

// ---------------------------------------------------------------------------
// element-wise add / sub / mul / div
// ---------------------------------------------------------------------------

template <typename T> struct BinT;   // storage type -> arithmetic
template <> struct BinT<float> {
    __device__ static inline float op(int o, float a, float b, float al, bool has_alpha) {
#pragma clang fp contract(off)
        if (o == TVK_BIN_MUL) return a * b;
        if (o == TVK_BIN_DIV) return a / b;
        const float t = has_alpha ? al * b : b;
        return o == TVK_BIN_ADD ? a + t : a - t;
    }
};
template <> struct BinT<double> {
    __device__ static inline double op(int o, double a, double b, double al, bool has_alpha) {
#pragma clang fp contract(off)
        if (o == TVK_BIN_MUL) return a * b;
        if (o == TVK_BIN_DIV) return a / b;
        const double t = has_alpha ? al * b : b;
        return o == TVK_BIN_ADD ? a + t : a - t;
    }
};

// float16 / bfloat16: each operation in float32, rounded back to the type
template <int DT>
__device__ __forceinline__ uint16_t bin16(int o, uint16_t a, uint16_t b, uint16_t al, bool has_alpha) {
#pragma clang fp contract(off)
    auto tof = [](uint16_t v) {
        return DT == TVK_F16 ? (float)__builtin_bit_cast(_Float16, v) : bf16_bits_to_f32(v);
    };
    auto fromf = [](float v) {
        return DT == TVK_F16 ? __builtin_bit_cast(uint16_t, (_Float16)v) : f32_to_bf16_bits(v);
    };
    if (o == TVK_BIN_MUL) return fromf(tof(a) * tof(b));
    if (o == TVK_BIN_DIV) return fromf(tof(a) / tof(b));
    const uint16_t t = has_alpha ? fromf(tof(al) * tof(b)) : b;
    return fromf(o == TVK_BIN_ADD ? tof(a) + tof(t) : tof(a) - tof(t));
}

// integers: two's-complement wrap in the type (computed in uint64)
template <typename I>
__device__ __forceinline__ I bin_int(int o, I a, I b, I al, bool has_alpha) {
    const uint64_t ua = (uint64_t)(int64_t)a, ub = (uint64_t)(int64_t)b, ual = (uint64_t)(int64_t)al;
    if (o == TVK_BIN_MUL) return (I)(ua * ub);
    const uint64_t t = has_alpha ? ual * ub : ub;
    return (I)(o == TVK_BIN_ADD ? ua + t : ua - t);
}

struct BinArgs {
    const char* a;
    const char* b;
    char* out;
    int op;
    int nd;
    int64_t numel;
    bool has_alpha;
    uint64_t alpha_bits;   // alpha in the element type
    Div32 div[kMaxDims];
    int64_t size[kMaxDims], as[kMaxDims], bs[kMaxDims], os[kMaxDims];
    bool idx32;
};

template <typename T, int DT>
__device__ __forceinline__ T bin_apply(int o, T a, T b, T al, bool has_alpha) {
    if constexpr (DT == TVK_F16 || DT == TVK_BF16) return (T)bin16<DT>(o, (uint16_t)a, (uint16_t)b, (uint16_t)al, has_alpha);
    else if constexpr (DT == TVK_F32) return BinT<float>::op(o, a, b, al, has_alpha);
    else if constexpr (DT == TVK_F64) return BinT<double>::op(o, a, b, al, has_alpha);
    else return bin_int<T>(o, a, b, al, has_alpha);
}

// T: storage type; DT: the tvk dtype
template <typename T, int DT>
__global__ __launch_bounds__(256) void binary_kernel(BinArgs p) {
    T al;
    __builtin_memcpy(&al, &p.alpha_bits, sizeof(T));
    const T* A = reinterpret_cast<const T*>(p.a);
    const T* B = reinterpret_cast<const T*>(p.b);
    T* O = reinterpret_cast<T*>(p.out);
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t li = (int64_t)blockIdx.x * 256 + threadIdx.x; li < p.numel; li += step) {
        int64_t ao = 0, bo = 0, oo = 0;
        if (p.idx32) {
            uint32_t rem = (uint32_t)li;
#pragma unroll 1
            for (int k = 0; k < p.nd - 1; ++k) {
                const uint32_t q = div32(rem, p.div[k]);
                const int64_t c = rem - q * p.div[k].d;
                ao += c * p.as[k];
                bo += c * p.bs[k];
                oo += c * p.os[k];
                rem = q;
            }
            ao += (int64_t)rem * p.as[p.nd - 1];
            bo += (int64_t)rem * p.bs[p.nd - 1];
            oo += (int64_t)rem * p.os[p.nd - 1];
        } else {
            int64_t rem = li;
#pragma unroll 1
            for (int k = 0; k < p.nd - 1; ++k) {
                const int64_t q = rem / p.size[k], c = rem - q * p.size[k];
                ao += c * p.as[k];
                bo += c * p.bs[k];
                oo += c * p.os[k];
                rem = q;
            }
            ao += rem * p.as[p.nd - 1];
            bo += rem * p.bs[p.nd - 1];
            oo += rem * p.os[p.nd - 1];
        }
        O[oo] = bin_apply<T, DT>(p.op, A[ao], B[bo], al, p.has_alpha);
    }
}

// every operand dense: 8 elements per thread through 16-byte (or wider) accesses
template <typename T, int DT>
__global__ __launch_bounds__(256) void binary_dense_kernel(BinArgs p) {
    T al;
    __builtin_memcpy(&al, &p.alpha_bits, sizeof(T));
    const int64_t groups = (p.numel + 7) / 8;
    const int64_t step = (int64_t)gridDim.x * 256;
    struct alignas(sizeof(T) * 8) V { T e[8]; };
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < groups; g += step) {
        const int64_t e0 = g * 8;
        if (e0 + 8 <= p.numel) {
            const V va = reinterpret_cast<const V*>(p.a)[g];
            const V vb = reinterpret_cast<const V*>(p.b)[g];
            V vo;
#pragma unroll
            for (int i = 0; i < 8; ++i) vo.e[i] = bin_apply<T, DT>(p.op, va.e[i], vb.e[i], al, p.has_alpha);
            reinterpret_cast<V*>(p.out)[g] = vo;
        } else {
            for (int64_t e = e0; e < p.numel; ++e)
                reinterpret_cast<T*>(p.out)[e] = bin_apply<T, DT>(p.op, reinterpret_cast<const T*>(p.a)[e],
                                                                   reinterpret_cast<const T*>(p.b)[e], al, p.has_alpha);
        }
    }
}

template <typename T, int DT>
void launch_binary(const BinArgs& p, bool dense, hipStream_t st) {
    if (dense)
        hipLaunchKernelGGL((binary_dense_kernel<T, DT>), dim3(blocks_for((p.numel + 7) / 8, 256)), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL((binary_kernel<T, DT>), dim3(blocks_for(p.numel, 256)), dim3(256), 0, st, p);
}

// alpha converted to the element type (the push constant in T), as raw bits
uint64_t alpha_bits_of(int dt, double alpha) {
    uint64_t bits = 0;
    switch (dt) {
        case TVK_F32: { float f = (float)alpha; std::memcpy(&bits, &f, 4); break; }
        case TVK_F64: std::memcpy(&bits, &alpha, 8); break;
        case TVK_F16: { _Float16 h = (_Float16)(float)alpha; std::memcpy(&bits, &h, 2); break; }
        case TVK_BF16: bits = f32_to_bf16_bits((float)alpha); break;
        default: { int64_t v = (int64_t)alpha; std::memcpy(&bits, &v, 8); break; }
    }
    return bits;
}

}  // namespace
}  // namespace tvk

using namespace tvk;

extern "C" tvk_status tvk_reduce_sum(const tvk_reduce_desc* d) {
    if (!d) return fail(TVK_ERR_INVALID, "tvk_reduce_sum: desc is NULL");
    auto ok_src = [](int dt) { return dt >= TVK_F32 && dt <= TVK_BOOL; };
    auto ok_dst = [](int dt) { return dt == TVK_F32 || dt == TVK_F16 || dt == TVK_BF16 || dt == TVK_F64 || dt == TVK_I64; };
    if (!ok_src(d->src_dtype) || !ok_dst(d->dst_dtype)) return fail(TVK_ERR_UNSUPPORTED, "tvk_reduce_sum: unsupported dtype");
    if (d->ndim < 0 || d->ndim > kMaxDims) return fail(TVK_ERR_UNSUPPORTED, "tvk_reduce_sum: too many dimensions");
    RedArgs p{};
    p.src = static_cast<const char*>(d->src);
    p.dst = static_cast<char*>(d->dst);
    p.sdt = d->src_dtype;
    p.ddt = d->dst_dtype;
    p.sb = (int)dtype_size(d->src_dtype);
    p.db = (int)dtype_size(d->dst_dtype);
    int kd[kMaxDims], rd[kMaxDims], nk = 0, nr = 0;
    int64_t nout = 1, nred = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->sizes[k] < 0) return fail(TVK_ERR_INVALID, "tvk_reduce_sum: negative size");
        if (d->src_strides[k] < 0 || d->dst_strides[k] < 0)
            return fail(TVK_ERR_UNSUPPORTED, "tvk_reduce_sum: negative strides are not supported");
        const bool red = (d->reduce_mask >> k) & 1u;
        if (red) nred *= d->sizes[k];
        else nout *= d->sizes[k];
        if (d->sizes[k] <= 1) continue;
        if (red) rd[nr++] = k;
        else kd[nk++] = k;
    }
    if (nout == 0) return TVK_OK;
    if (!d->dst || (nred > 0 && !d->src)) return fail(TVK_ERR_INVALID, "tvk_reduce_sum: src or dst is NULL");
    for (int i = 0; i < nk; ++i)
        if (d->dst_strides[kd[i]] == 0) return fail(TVK_ERR_INVALID, "tvk_reduce_sum: dst has a zero stride over a kept dimension");
    // kept dimensions in source memory order (merged where both src and dst allow),
    // reduced ones likewise
    std::stable_sort(kd, kd + nk, [&](int x, int y) { return d->src_strides[x] < d->src_strides[y]; });
    std::stable_sort(rd, rd + nr, [&](int x, int y) { return d->src_strides[x] < d->src_strides[y]; });
    p.nk = 0;
    for (int i = 0; i < nk; ++i) {
        const int k = kd[i];
        if (p.nk > 0) {
            const int l = p.nk - 1;
            if (d->src_strides[k] == p.kss[l] * p.ksize[l] && d->dst_strides[k] == p.kds[l] * p.ksize[l]) {
                p.ksize[l] *= d->sizes[k];
                continue;
            }
        }
        p.ksize[p.nk] = d->sizes[k];
        p.kss[p.nk] = d->src_strides[k];
        p.kds[p.nk] = d->dst_strides[k];
        ++p.nk;
    }
    p.nr = 0;
    for (int i = 0; i < nr; ++i) {
        const int k = rd[i];
        if (p.nr > 0) {
            const int l = p.nr - 1;
            if (d->src_strides[k] == p.rss[l] * p.rsize[l]) {
                p.rsize[l] *= d->sizes[k];
                continue;
            }
        }
        p.rsize[p.nr] = d->sizes[k];
        p.rss[p.nr] = d->src_strides[k];
        ++p.nr;
    }
    p.nout = nout;
    p.nred = nred;
    p.idx32 = nout <= 0xffffffffLL && nred <= 0xffffffffLL;
    for (int i = 0; i < p.nk && p.idx32; ++i) p.kdiv[i] = make_div((uint32_t)p.ksize[i]);
    for (int i = 0; i < p.nr && p.idx32; ++i) p.rdiv[i] = make_div((uint32_t)p.rsize[i]);
    const hipStream_t st = resolve_stream(d->stream);
    if (nred == 0) {
        hipLaunchKernelGGL(reduce_zero_kernel, dim3(blocks_for(nout, 256)), dim3(256), 0, st, p);
    } else {
        if (p.nr == 0) {   // nothing of extent > 1 is reduced: a sum of one element
            p.nr = 1;
            p.rsize[0] = 1;
            p.rss[0] = 0;
            p.rdiv[0] = make_div(1);
        }
        const bool row = p.nk == 0 || p.rss[0] < p.kss[0];
        int dev = 0;
        (void)hipGetDevice(&dev);
        tvk_status s;
        if (d->dst_dtype == TVK_F64) s = run_sum<double>(p, row, dev, st);
        else if (d->dst_dtype == TVK_I64) s = run_sum<int64_t>(p, row, dev, st);
        else s = run_sum<float>(p, row, dev, st);
        if (s != TVK_OK) return s;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_reduce_sum: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}

extern "C" tvk_status tvk_binary(const tvk_binary_desc* d) {
    if (!d) return fail(TVK_ERR_INVALID, "tvk_binary: desc is NULL");
    if (d->op < TVK_BIN_ADD || d->op > TVK_BIN_DIV) return fail(TVK_ERR_INVALID, "tvk_binary: unknown op");
    if (d->dtype < TVK_F32 || d->dtype > TVK_U8) return fail(TVK_ERR_UNSUPPORTED, "tvk_binary: unsupported dtype");
    if (d->op == TVK_BIN_DIV && d->dtype != TVK_F32 && d->dtype != TVK_F16 && d->dtype != TVK_BF16 && d->dtype != TVK_F64)
        return fail(TVK_ERR_UNSUPPORTED, "tvk_binary: division takes floating point dtypes only");
    if (d->reserved != 0) return fail(TVK_ERR_INVALID, "tvk_binary: nonzero reserved field");
    if (d->ndim < 0 || d->ndim > kMaxDims) return fail(TVK_ERR_UNSUPPORTED, "tvk_binary: too many dimensions");
    BinArgs p{};
    p.op = d->op;
    int idx[kMaxDims], n = 0;
    int64_t numel = 1;
    for (int k = 0; k < d->ndim; ++k) {
        if (d->sizes[k] < 0) return fail(TVK_ERR_INVALID, "tvk_binary: negative size");
        if (d->a_strides[k] < 0 || d->b_strides[k] < 0 || d->out_strides[k] < 0)
            return fail(TVK_ERR_UNSUPPORTED, "tvk_binary: negative strides are not supported");
        numel *= d->sizes[k];
        if (d->sizes[k] > 1) {
            if (d->out_strides[k] == 0) return fail(TVK_ERR_INVALID, "tvk_binary: out has a zero stride (overlapping elements)");
            idx[n++] = k;
        }
    }
    if (numel == 0) return TVK_OK;
    if (!d->a || !d->b || !d->out) return fail(TVK_ERR_INVALID, "tvk_binary: a, b or out is NULL");
    std::stable_sort(idx, idx + n, [&](int x, int y) { return d->out_strides[x] < d->out_strides[y]; });
    p.nd = 0;
    for (int i = 0; i < n; ++i) {
        const int k = idx[i];
        if (p.nd > 0) {
            const int l = p.nd - 1;
            if (d->out_strides[k] == p.os[l] * p.size[l] && d->a_strides[k] == p.as[l] * p.size[l] &&
                d->b_strides[k] == p.bs[l] * p.size[l]) {
                p.size[l] *= d->sizes[k];
                continue;
            }
        }
        p.size[p.nd] = d->sizes[k];
        p.as[p.nd] = d->a_strides[k];
        p.bs[p.nd] = d->b_strides[k];
        p.os[p.nd] = d->out_strides[k];
        ++p.nd;
    }
    if (p.nd == 0) {
        p.nd = 1;
        p.size[0] = 1;
        p.as[0] = p.bs[0] = p.os[0] = 1;
    }
    p.numel = numel;
    p.idx32 = numel <= 0xffffffffLL;
    for (int i = 0; i < p.nd && p.idx32; ++i) p.div[i] = make_div((uint32_t)p.size[i]);
    p.a = static_cast<const char*>(d->a);
    p.b = static_cast<const char*>(d->b);
    p.out = static_cast<char*>(d->out);
    p.has_alpha = (d->op == TVK_BIN_ADD || d->op == TVK_BIN_SUB) && d->alpha != 1.0;
    p.alpha_bits = alpha_bits_of(d->dtype, d->alpha);
    const size_t es = dtype_size(d->dtype);
    auto al = [&](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % (es * 8) == 0; };
    const bool dense = p.nd == 1 && p.as[0] == 1 && p.bs[0] == 1 && p.os[0] == 1 && al(d->a) && al(d->b) && al(d->out);
    const hipStream_t st = resolve_stream(d->stream);
    switch (d->dtype) {
        case TVK_F32: launch_binary<float, TVK_F32>(p, dense, st); break;
        case TVK_F64: launch_binary<double, TVK_F64>(p, dense, st); break;
        case TVK_F16: launch_binary<uint16_t, TVK_F16>(p, dense, st); break;
        case TVK_BF16: launch_binary<uint16_t, TVK_BF16>(p, dense, st); break;
        case TVK_I64: launch_binary<int64_t, TVK_I64>(p, dense, st); break;
        case TVK_I32: launch_binary<int32_t, TVK_I32>(p, dense, st); break;
        case TVK_I16: launch_binary<int16_t, TVK_I16>(p, dense, st); break;
        case TVK_I8: launch_binary<int8_t, TVK_I8>(p, dense, st); break;
        default: launch_binary<uint8_t, TVK_U8>(p, dense, st); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_binary: launch failed: ") + hipGetErrorString(e));
    return TVK_OK;
}
