/*
 * tvk_hip.h - the C ABI of the MI355X (gfx950) dense-contraction library.
 *
 * This is the thin boundary that replaces, for the dense-contraction path only,
 * the reference's Vulkan runtime layer (device/queue setup, VMA memory, shader
 * manager and autotuner under src/vulkan/) and its matmul/conv shaders
 * (src/shaders/ops/matmul_*.slang, conv_*.slang, winograd_*.slang).
 *
 * Rules of the ABI:
 *   - extern "C", plain pointers, sizes and enums; no C++ or torch types cross it.
 *   - every entry point returns a tvk_status; tvk_last_error() gives the
 *     thread-local message of the last failure.
 *   - the library never owns caller tensors: pointers are borrowed for the call.
 *   - compute and copy entry points are asynchronous on `stream` (a
 *     hipStream_t); a NULL stream is HIP's default stream. tvk_get_stream
 *     gives the library's own per-device stream, the one tvk_synchronize
 *     waits for and the caching allocator's blocks are ordered on.
 *   - strides are in ELEMENTS, not bytes, and may be zero (broadcast) or any
 *     positive value; element offsets must fit in int64.
 *   - scratch memory: tvk_gemm, tvk_conv2d_*, tvk_conv_*, tvk_reduce_sum and
 *     tvk_attention_bwd lease library scratch (split-K partials, repacked
 *     operands, convolution partials, the attention delta) from a per-device
 *     pool for the kernels they queue on their `stream`. A buffer is leased
 *     again only for the stream its first lease named, so stream order puts
 *     each call's kernels after the previous holder's; concurrent calls (other
 *     threads, other streams) get other buffers; buffers are freed only after
 *     the device has drained (on growth, allocation failure or
 *     tvk_empty_cache). Calls may therefore come from any thread and any
 *     stream; the caller orders only its own tensors.
 */
#ifndef TVK_HIP_H
#define TVK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. UNSUPPORTED means "this call cannot run on the device; the
 * caller should take its CPU fallback" - the role TORCHVULKAN_FALLBACK plays in
 * the reference (src/api/fallback.h:7-11). */
typedef enum {
    TVK_OK = 0,
    TVK_ERR_UNSUPPORTED = 1,
    TVK_ERR_OOM = 2,
    TVK_ERR_INVALID = 3,
    TVK_ERR_DEVICE = 4
} tvk_status;

/* Element types. tvk_gemm takes F32 through U8; tvk_conv2d_* and tvk_conv_*
 * take F32, F16 and BF16; tvk_copy takes every one of them. BOOL is one byte holding 0 or
 * 1. F8E4M3FN and F8E5M2 are torch's float8_e4m3fn and float8_e5m2 (OCP 8-bit
 * floats: e4m3 with no infinities and NaN = S.1111.111, e5m2 IEEE-like);
 * only tvk_copy takes them. */
typedef enum {
    TVK_F32 = 0,
    TVK_F16 = 1,
    TVK_BF16 = 2,
    TVK_F64 = 3,
    TVK_I64 = 4,
    TVK_I32 = 5,
    TVK_I16 = 6,
    TVK_I8 = 7,
    TVK_U8 = 8,
    TVK_BOOL = 9,
    TVK_F8E4M3FN = 10,
    TVK_F8E5M2 = 11
} tvk_dtype;

/* Epilogue activation, the reference's MatmulActivation
 * (src/api/ops/matmul.cpp:13-18): NONE=0, RELU=1, GELU=2 (erf form). */
typedef enum {
    TVK_ACT_NONE = 0,
    TVK_ACT_RELU = 1,
    TVK_ACT_GELU = 2
} tvk_activation;

/* ------------------------------------------------------------------------- */
/* Errors                                                                     */
/* ------------------------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). Replaces the
 * TORCH_CHECK strings the reference raises from inside its runtime. */
const char* tvk_last_error(void);

/* ------------------------------------------------------------------------- */
/* Runtime: devices and streams                                               */
/* Replaces VulkanContext::Instance()/getDeviceCount()/CurrentDevice()        */
/* (src/vulkan/vulkan_context.h:9-55, src/api/backend.cpp:11-30).             */
/* ------------------------------------------------------------------------- */

tvk_status tvk_device_count(int* count);
tvk_status tvk_set_device(int device);
tvk_status tvk_get_device(int* device);
/* The library's stream for `device` (created on first use, default priority). */
tvk_status tvk_get_stream(int device, void** stream);
/* Blocks until all work on the library stream of `device` is done.
 * Replaces DeviceContext::flush() behind torchvulkan.synchronize
 * (src/api/backend.cpp:32-35). */
tvk_status tvk_synchronize(int device);

/* Events on a stream, for the device guard's torch.Event API. They replace
 * the reference's host-timestamp VulkanEvent (src/api/guard.cpp:14-61), which
 * synchronised the whole queue on every record. `timing` != 0 makes the event
 * usable by tvk_event_elapsed. A NULL stream is HIP's default stream. */
tvk_status tvk_event_create(int device, int timing, void** event);
tvk_status tvk_event_destroy(void* event);
/* The event completes once the work queued on `stream` so far has run. */
tvk_status tvk_event_record(void* event, void* stream);
/* *done = 1 when the event's work has run (or it was never recorded). */
tvk_status tvk_event_query(void* event, int* done);
tvk_status tvk_event_synchronize(void* event);
/* Milliseconds between two recorded timing events (GPU clock). */
tvk_status tvk_event_elapsed(void* start, void* end, float* ms);
/* Work queued on `stream` from now on waits for `event`. */
tvk_status tvk_stream_wait_event(void* stream, void* event);
/* *done = 1 when every operation queued on `stream` has run. */
tvk_status tvk_stream_query(void* stream, int* done);

typedef struct {
    char name[256];
    char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    size_t total_memory;
    int compute_units;
    int clock_khz;           /* peak shader clock reported by the runtime */
    int wavefront_size;
    size_t lds_per_block;
    int pci_bus_id;
    int has_fp64, has_fp16, has_bf16;
} tvk_device_props;

/* Replaces _device_properties (src/api/backend.cpp:104-124). */
tvk_status tvk_device_properties(int device, tvk_device_props* out);

/* Measurement aid with no counterpart in the reference: the sustained float16
 * MFMA rate of `device` with random operands (v_mfma_f32_16x16x32_f16 over
 * sixteen independent accumulators, 64 a loop trip, `waves_per_simd` waves on every SIMD, 1-4),
 * timed with HIP events over one launch of `iterations` steps on a stream of
 * its own. The dense-peak figure assumes operands that barely toggle; with
 * random data the part is power-limited, and this rate is the ceiling a GEMM's
 * MFMA pipe can reach. *tflops and the launch's *ms on return. Allocates and
 * synchronises: not for hot paths. */
tvk_status tvk_calibrate_mfma(int device, int waves_per_simd, int iterations, double* tflops, double* ms);
/* The same loop with `operands` 0 (random, as tvk_calibrate_mfma) or 1 (all
 * zeros: operands that toggle nothing, which shows the pipe's issue limit
 * apart from the part's power limit); 2 and 3 are the same two operand sets
 * on v_mfma_f32_32x32x16_f16 (eight 32x32 accumulators, 32 MFMAs a trip: the
 * same flops). */
tvk_status tvk_calibrate_mfma_operands(int device, int waves_per_simd, int iterations, int operands, double* tflops,
                                       double* ms);

/* Measurement aid with no counterpart in the reference: the read bandwidth of
 * a plain streaming kernel on `device` (512 workgroups, four 16-byte loads in
 * flight a thread), the practical ceiling of a kernel that reads each byte of
 * HBM once. Three windows of `window_bytes` (a multiple of 16, 4 KiB to 8 GiB)
 * are read in rotation, one a launch; `iterations` launches are timed with HIP
 * events on a stream of its own. *gbps (window bytes / launch time, 1e9 B/s)
 * and the average launch *ms on return. Allocates 3 x window_bytes and
 * synchronises: not for hot paths. */
tvk_status tvk_calibrate_hbm(int device, size_t window_bytes, int iterations, double* gbps, double* ms);

/* ------------------------------------------------------------------------- */
/* Memory: a hipMalloc-backed caching allocator, stream-ordered on the        */
/* library stream. Replaces VulkanAllocator + DeviceContext buffer pools      */
/* (src/vulkan/allocator.cpp:59-200, src/vulkan/cache.cpp:78-89).             */
/* ------------------------------------------------------------------------- */

/* Allocates `bytes` (rounded up to a size class) on `device`. bytes==0 gives
 * *out==NULL and TVK_OK. A request past the budget set by
 * tvk_set_memory_limit, or one hipMalloc cannot serve after the cache is
 * released, follows the reference's allocateBuffer
 * (src/vulkan/allocator.cpp:171-200): with strict allocation off (the
 * default) it is served from pinned host memory, which kernels read and write
 * over the host link (slower; tvk_last_malloc_spilled then reports 1); with
 * strict allocation on it returns TVK_ERR_OOM. */
tvk_status tvk_malloc(int device, size_t bytes, void** out);
/* Returns a block to its size-class cache. NULL is a no-op. Freeing a pointer
 * the allocator did not hand out is TVK_ERR_INVALID. A block served from host
 * memory is freed at once, after the device has drained. */
tvk_status tvk_free(void* ptr);
/* Strict allocation, the reference's TORCHVULKAN_STRICT_ALLOCATION
 * (src/vulkan/vulkan_context.cpp:248, read at start-up): on when that
 * variable is set to a non-empty value other than "0" when the library loads;
 * this call changes it for the process. */
tvk_status tvk_set_strict_allocation(int strict);
tvk_status tvk_get_strict_allocation(int* strict);
/* *spilled = 1 when this thread's last successful tvk_malloc was served from
 * host memory (the caller's cue for the reference's one-time warning). */
tvk_status tvk_last_malloc_spilled(int* spilled);
/* Pinned (page-locked) host memory for tensor.pin_memory(): the reference's
 * pinned allocator with its block registry (src/api/hook.cpp:14-51). Pinned
 * blocks let host <-> device copies run as direct DMA. tvk_host_free takes
 * only pointers tvk_host_malloc returned, and the caller must not free a block
 * an asynchronous copy still reads. */
tvk_status tvk_host_malloc(size_t bytes, void** out);
tvk_status tvk_host_free(void* ptr);
/* *pinned = 1 when ptr lies inside a live tvk_host_malloc block
 * (isPinnedPtr, src/api/hook.cpp:24-31,69). */
tvk_status tvk_host_pointer_pinned(const void* ptr, int* pinned);
/* Releases every cached (unused) block of `device` back to HIP
 * (torchvulkan.empty_cache, src/api/backend.cpp:52-54). */
tvk_status tvk_empty_cache(int device);
/* Device of a pointer the allocator handed out, or -1
 * (getDeviceFromPtr, src/api/hook.cpp:58-62). */
tvk_status tvk_pointer_device(const void* ptr, int* device);
/* 0 = no limit. */
tvk_status tvk_set_memory_limit(int device, size_t bytes);

tvk_status tvk_memory_allocated(int device, size_t* bytes);
tvk_status tvk_max_memory_allocated(int device, size_t* bytes);
/* Bytes obtained from hipMalloc and held: the caching allocator's blocks and
 * the library's scratch buffers. */
tvk_status tvk_memory_reserved(int device, size_t* bytes);
tvk_status tvk_reset_peak_memory_stats(int device);
/* (free, total) as hipMemGetInfo reports them (src/api/backend.cpp:82-85). */
tvk_status tvk_mem_get_info(int device, size_t* free_bytes, size_t* total_bytes);

/* Stream-ordered copies. h2d/d2h block until done when `blocking` != 0. */
tvk_status tvk_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream, int blocking);
tvk_status tvk_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream, int blocking);
tvk_status tvk_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);

/* ------------------------------------------------------------------------- */
/* Copy and cast: one strided element-wise copy with dtype conversion         */
/* ------------------------------------------------------------------------- */

#define TVK_COPY_MAX_DIMS 16

/* dst[i] = convert(src[i]) for every index i of `sizes`, with each tensor at
 * base + sum_d i_d * stride_d (elements). src strides may be 0 (an expanded
 * source); dst must not have two indices on one element, and src and dst must
 * not partly overlap (the caller checks both, as the reference's
 * TensorIterator does with set_check_mem_overlap, transfer.cpp:18-22).
 *
 * Conversion is the reference's castValue (src/shaders/core/cast.slang:49-52,
 * src/shaders/core/dtype.slang:122-282): the source widens to int64 (signed
 * integers), uint64 (U8), float (F16, BF16, F32) or double (F64); the
 * destination is built from that wide value in one conversion:
 *   - to an integer type: C conversion (truncation toward zero from a float,
 *     two's-complement wrap from an integer; a float outside the target's
 *     range or NaN is undefined there, as in SPIR-V, and saturates here);
 *   - to F32/F64: round to nearest even;
 *   - to F16: one round to nearest even from the wide value (from F64 too);
 *   - to BF16: BFloat16(float(v)), so F64 rounds to float first.
 * With BOOL on either side the value is (src != 0) ? 1 : 0 (IS_BOOL_CAST,
 * src/shaders/ops/cast.slang:29-33).
 * The float8 types have no shader type in the reference, which converts them
 * through float32 with c10's own conversions (copy_float8_vulkan_to_vulkan,
 * src/api/tensor/transfer.cpp:129-226), so they match the CPU bit for bit:
 *   - from F8: the exact value as a float (then the float rules above);
 *   - to F8: the value converted to float first (the rules above), then
 *     rounded to nearest even onto the 8-bit grid, subnormals included.
 *     F8E4M3FN: NaN, infinities and magnitudes that round past 448 become
 *     NaN (S.1111.111, sign kept). F8E5M2: NaN becomes S.11111.11, infinities
 *     and magnitudes that round past 57344 become infinity.
 *
 * Replaces dispatch_copy_shader (src/api/tensor/transfer.cpp:16-56) and
 * dispatch_cast_shader (src/api/tensor/cast.cpp:8-56). Dimensions are merged
 * where both tensors allow it; more than TVK_COPY_MAX_DIMS dimensions left
 * after merging is TVK_ERR_UNSUPPORTED. Offsets are 64-bit: no 32-bit limit. */
typedef struct {
    int32_t src_dtype;      /* tvk_dtype */
    int32_t dst_dtype;      /* tvk_dtype */
    int32_t ndim;           /* 0 .. TVK_COPY_MAX_DIMS (0: one element) */
    int32_t reserved;       /* must be 0 */
    int64_t sizes[TVK_COPY_MAX_DIMS];
    const void* src; int64_t src_strides[TVK_COPY_MAX_DIMS];
    void* dst; int64_t dst_strides[TVK_COPY_MAX_DIMS];
    void* stream;           /* hipStream_t or NULL */
} tvk_copy_desc;

tvk_status tvk_copy(const tvk_copy_desc* desc);

/* Name of the kernel tvk_copy would launch for `desc` ("memcpy", "cast_contig",
 * "transpose", "broadcast" for one source element repeated into a dense
 * destination, "strided", or "none" for an empty copy); no launch. */
tvk_status tvk_copy_plan(const tvk_copy_desc* desc, char* name, size_t name_len);

/* Fills every element of a strided destination with one element value.
 * `pattern` holds the element's bytes (little-endian, low `elem_size` bytes):
 * the caller converts the scalar to the element type, as the reference does
 * on the host before its fill shader (src/api/ops/fill.cpp:11-131). A zero
 * stride over an extent > 1 is TVK_ERR_INVALID. Replaces the fill_ and zero_
 * dispatch (fill.cpp:131-133); fill_.Tensor reads its value on the host too. */
typedef struct {
    int32_t elem_size;      /* 1, 2, 4 or 8 */
    int32_t ndim;           /* 0 .. TVK_COPY_MAX_DIMS */
    int64_t sizes[TVK_COPY_MAX_DIMS];
    void* dst; int64_t dst_strides[TVK_COPY_MAX_DIMS];
    uint64_t pattern;
    void* stream;
} tvk_fill_desc;

tvk_status tvk_fill(const tvk_fill_desc* desc);

/* ------------------------------------------------------------------------- */
/* Reductions and element-wise arithmetic on both sides of the contractions   */
/* ------------------------------------------------------------------------- */

/* dst = sum of src over the dimensions whose bit is set in reduce_mask.
 * dst is indexed by the same dimensions as src: its strides for summed
 * dimensions are ignored (keepdim or squeezed views are both expressible).
 * Element types: src F32/F16/BF16/F64/I64/I32/I16/I8/U8/BOOL; dst F32, F16,
 * BF16, F64 or I64. The accumulator is the reference's
 * reduce_accumulate_dtype (src/api/ops/helpers.h:476-480): float32 when dst
 * is F16/BF16, else dst's own type; each source element is converted to it
 * first (sum_accumulated, src/api/ops/reduce.cpp:265-273), the total is
 * rounded once to dst. An empty sum is 0. The order of the additions is fixed
 * (the same bits on every run); it is not the reference shader's order, which
 * its driver decides. Replaces sum / sum.dim_IntList
 * (src/api/ops/reduce.cpp:276-291,750-751). */
typedef struct {
    int32_t src_dtype;
    int32_t dst_dtype;
    int32_t ndim;           /* 0 .. TVK_COPY_MAX_DIMS */
    uint32_t reduce_mask;   /* bit d: sum over dimension d */
    int64_t sizes[TVK_COPY_MAX_DIMS];
    const void* src; int64_t src_strides[TVK_COPY_MAX_DIMS];
    void* dst; int64_t dst_strides[TVK_COPY_MAX_DIMS];
    void* stream;
} tvk_reduce_desc;

tvk_status tvk_reduce_sum(const tvk_reduce_desc* desc);

typedef enum {
    TVK_BIN_ADD = 0,        /* out = a + alpha*b */
    TVK_BIN_SUB = 1,        /* out = a - alpha*b */
    TVK_BIN_MUL = 2,        /* out = a * b (alpha unused) */
    TVK_BIN_DIV = 3         /* out = a / b (alpha unused; F32, F16, BF16, F64) */
} tvk_binary_op;

/* Element-wise out = op(a, b) over `sizes`, every operand strided (zero
 * strides broadcast a and b). One dtype for all three: F32, F16, BF16, F64,
 * I64, I32, I16, I8, U8 (DIV: the float types only, IEEE division rounded to
 * nearest even, the reference's DivOp, binary.slang:57-60). As the
 * reference's binary shader (src/shaders/ops/binary.slang:39-55): alpha is
 * converted to the dtype;
 * with alpha != 1, add/sub compute T(a op T(alpha*b)), otherwise T(a op b);
 * every operation rounds to the dtype (float16/bfloat16 compute in float32
 * and round after each operation, dtype.slang:911-913), float32 products are
 * not fused into the add. out may alias a or b exactly (in-place ops), not
 * partly. Replaces add/sub/mul (.Tensor, _.Tensor, .out;
 * src/api/ops/binary.cpp:269-300,1090-1118). */
typedef struct {
    int32_t op;             /* tvk_binary_op */
    int32_t dtype;
    int32_t ndim;           /* 0 .. TVK_COPY_MAX_DIMS */
    int32_t reserved;       /* must be 0 */
    int64_t sizes[TVK_COPY_MAX_DIMS];
    const void* a; int64_t a_strides[TVK_COPY_MAX_DIMS];
    const void* b; int64_t b_strides[TVK_COPY_MAX_DIMS];
    void* out; int64_t out_strides[TVK_COPY_MAX_DIMS];
    double alpha;
    void* stream;
} tvk_binary_desc;

tvk_status tvk_binary(const tvk_binary_desc* desc);

/* ------------------------------------------------------------------------- */
/* Fused scaled dot-product attention (forward)                               */
/* ------------------------------------------------------------------------- */

/* out[b,h,i,:] = sum_j softmax_j(s[b,h,i,:]) * v[b,h/group,j,:] with
 *   s[b,h,i,j] = scale * (q[b,h,i,:] . k[b,h/group,j,:]) + bias[b,h,i,j],
 * s = -inf where `causal` and j > i (top-left aligned) or j >= len_kv;
 * group = heads_q / heads_kv (grouped-query attention). A row with every
 * key masked gives out = 0 and lse = +inf; otherwise
 * lse[b,h,i] = max_j s + log(sum_j exp(s - max_j s)) (natural log, float32).
 * Scores and the softmax are float32; the probabilities are rounded to the
 * dtype before the product with v, as the reference's cooperative-matrix
 * kernel stages them in the dtype (src/shaders/ops/attention_coop.slang;
 * row semantics from chunked_forward, src/api/ops/attention.cpp:115-139).
 * Supported: F32, F16 and BF16; head_dim and head_dim_v from 1 to 512 (they
 * may differ); any element strides for q, k, v, bias (zero strides
 * broadcast) and out; batch and heads up to 65535, sequences up to 2^30.
 * float16/bfloat16 with head_dim == head_dim_v in {64, 128}, unit stride along
 * the head dimension and 16-byte aligned rows run the MFMA kernels; every
 * other case runs general kernels (float32 dot products over LDS-staged
 * 64-column chunks of the head dims, the same staging of P in the dtype).
 * Other cases return TVK_ERR_UNSUPPORTED. Replaces fused_forward
 * (src/api/ops/attention.cpp:434-500) and, for the shapes it leaves,
 * chunked_forward (:115-139) behind
 * _scaled_dot_product_fused_attention_overrideable (:697-719). */
typedef struct {
    int32_t dtype;
    int32_t causal;
    int64_t batch, heads_q, heads_kv, len_q, len_kv, head_dim, head_dim_v;
    const void* q; int64_t q_stride[4];       /* [batch][head][row][dim], elements */
    const void* k; int64_t k_stride[4];
    const void* v; int64_t v_stride[4];
    const void* bias; int64_t bias_stride[4]; /* NULL: none */
    void* out; int64_t out_stride[4];
    float* lse; int64_t lse_stride[3];        /* [batch][head][row] */
    double scale;
    void* stream;
} tvk_attention_desc;

tvk_status tvk_attention_fwd(const tvk_attention_desc* desc);

/* Gradients of tvk_attention_fwd: dq, dk, dv (same dtype and head layouts as
 * q, k, v) from dout and the forward's out and lse (`fwd` describes q, k, v,
 * bias, out, lse, scale and causal exactly as for the forward call). With
 * P = exp(s - lse) and delta_i = sum_d dout[i,d]*out[i,d] (float32):
 *   dv[j] = sum_i P[i,j] dout[i],  dS = P * (dout.v^T - delta),
 *   dq[i] = scale * sum_j dS[i,j] k[j],  dk[j] = scale * sum_i dS[i,j] q[i],
 * summed over the query heads of each kv head (the reference's
 * chunked_backward, src/api/ops/attention.cpp:141-199; the fused passes
 * BACKWARD_Q and BACKWARD_KV, :640-665). P and dS are formed in float32 and
 * rounded to the dtype before their products, as the reference's
 * scoreGradients stages them (src/shaders/ops/attention_coop.slang:283-305);
 * accumulation is float32, and every output element
 * is written by one workgroup (no atomics: the same bits every run). When
 * `dscores` is not NULL it receives dS (float32, unrounded, [B, Hq, L, S] at
 * dscores_stride; zero where masked), the gradient of an additive bias before
 * any broadcast is summed away: the reference computes the bias gradient on
 * its chunked path (:141-199), here the caller sums dS over the bias's
 * broadcast dimensions. Same support as the forward (dout, dq, dk, dv any
 * strides; the MFMA passes need unit stride along the head dimension and
 * 16-byte aligned rows, and run only without dscores). Uses B*Hq*L floats of
 * library scratch for delta. */
typedef struct {
    tvk_attention_desc fwd;
    const void* dout; int64_t dout_stride[4];
    void* dq; int64_t dq_stride[4];
    void* dk; int64_t dk_stride[4];
    void* dv; int64_t dv_stride[4];
    float* dscores; int64_t dscores_stride[4];   /* NULL: not wanted */
} tvk_attention_bwd_desc;

tvk_status tvk_attention_bwd(const tvk_attention_bwd_desc* desc);

/* ------------------------------------------------------------------------- */
/* Compute: batched strided GEMM with fused epilogue                          */
/* ------------------------------------------------------------------------- */

/* One batched GEMM:
 *   C[b,m,n] = act( alpha * sum_k A[b,m,k] * B[b,k,n] + beta * bias[b,m,n] )
 * with every operand addressed as base + b*s[0] + row*s[1] + col*s[2]
 * (elements). The bias term is applied only when bias != NULL and beta != 0,
 * the reference's has_bias rule (src/api/ops/matmul.cpp:259,394). alpha and
 * beta are rounded to float32, the accumulate type the reference pushes them
 * in (src/vulkan/builders.h:119-140, src/api/ops/matmul.cpp:238-239).
 * F32, F16, BF16: accumulation is float32; the result is rounded once to
 * `dtype` (round to nearest even). float32 always accumulates in the
 * reference SIMD tile's order (fmaf over k in sequence per output,
 * src/shaders/helpers/gemm_simd.slang:219-239); float16/bfloat16 use MFMA
 * tiles whose order within 16 k is the hardware's, unless TVK_GEMM_EXACT. K == 0 gives act(beta*bias) or zeros
 * (src/api/ops/matmul.cpp:284-288).
 * F64 and the integer types accumulate in their own type, as the reference's
 * device does (src/shaders/core/dtype.slang:117-219): float64 by fma over k in
 * sequence per output with alpha/beta in float64; integers in two's-complement
 * with wraparound in the type's width, alpha and beta converted to integers
 * (truncated), relu = max(v, 0) and no gelu (TVK_ERR_INVALID). These run one
 * kernel ("gemm_wide_f64" / "gemm_wide_int"), use no scratch, and take any
 * strides and sizes. TVK_GEMM_EXACT changes nothing for them.
 *
 * Replaces the dispatch in dispatch_matmul_shader
 * (src/api/ops/matmul.cpp:584-597) of matmul_simd_main
 * (src/shaders/ops/matmul_simd.slang:23-44) and matmul_coop_main
 * (src/shaders/ops/matmul_coop.slang:443-452), with the same 4-stride operand
 * model as TensorStrides (src/shaders/helpers/gemm.slang:3-9).
 *
 * Scratch: split-K partials and repacked operands come from a per-device pool
 * of stream-affine buffers (freed by tvk_empty_cache after a drain). The
 * M <= 16 streaming kernel reduces its split-K partials in the same launch,
 * counting finished workgroups in a 64 KB array per stream (allocated at the
 * stream's first such product, kept until the process ends, at most 32
 * streams a device); launches under graph capture, on hipStreamPerThread and
 * on further streams use a second reduction launch instead. */
/* tvk_gemm_desc.flags */
#define TVK_GEMM_EXACT 1u   /* every dtype in the reference SIMD tile's order:
                               float32 operands, fmaf over k = 0..K-1 in
                               sequence per output (bit-identical to that
                               order); float16/bfloat16 then run at the float32
                               matrix rate instead of their own */

typedef struct {
    int32_t dtype;          /* tvk_dtype of A, B, bias and C */
    int32_t activation;     /* tvk_activation */
    uint32_t flags;         /* TVK_GEMM_* */
    int32_t reserved;       /* must be 0 */
    int64_t batch, M, N, K;
    const void* a; int64_t a_stride[3];
    const void* b; int64_t b_stride[3];
    const void* bias; int64_t bias_stride[3];   /* NULL: no bias */
    void* c; int64_t c_stride[3];
    double alpha, beta;
    void* stream;           /* hipStream_t or NULL */
    /* An optional second batch dimension. With batch_inner > 1 (it must
     * divide batch), batch index b addresses every operand at
     *   (b / batch_inner) * stride[0] + (b % batch_inner) * stride_inner,
     * so a [B, H, rows, cols] view whose B and H strides do not merge into
     * one (head-strided q, k, v: [B, L, H, D] underneath) runs as one product
     * of batch B*H without a copy; the batch dimensions of
     * prepare_matmul_operands / batched matmul (src/api/ops/matmul.cpp:27-78)
     * collapse into these two. 0 or 1: one batch dimension, stride[0]. */
    int64_t batch_inner;
    int64_t a_stride_inner, b_stride_inner, bias_stride_inner, c_stride_inner;
} tvk_gemm_desc;

tvk_status tvk_gemm(const tvk_gemm_desc* desc);

/* tvk_gemm without any allocation: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The product's scratch
 * (split-K partials, repacked operands) lives in a 32 MiB `__device__` array
 * that is part of the library's code object: every device the library is
 * loaded on holds those 32 MiB from load until the process ends, whether or
 * not this entry point is ever called. A product whose
 * shape-chosen kernel needs more is rejected with TVK_ERR_INVALID before
 * anything is queued (tvk_gemm takes it). The kernel is the shape rules'
 * choice (the kernel-choice table is not consulted). Every call on a device
 * shares that device's array: calls that overlap on one device (two streams,
 * or two threads, without ordering between them) race on it; calls ordered on
 * one stream do not. Results are those of tvk_gemm with the same kernel. */
tvk_status tvk_gemm_noalloc(const tvk_gemm_desc* desc);

/* Name of the kernel tvk_gemm would launch for `desc` (no launch). Used by
 * tests and the benchmark to state which path ran; replaces the tuner's
 * choice record (src/vulkan/autotuner.cpp:56-84). */
tvk_status tvk_gemm_plan(const tvk_gemm_desc* desc, char* name, size_t name_len);

/* ---- kernel-choice table ----------------------------------------------------
 * tvk_gemm picks its kernel from the shape (the plan above) unless the
 * kernel-choice table holds another candidate for the product's shape class:
 * dtype, flags, epilogue, operand layout and alignment, and ceil(log2) of
 * M, N, K and batch (the reference's matmul tune key,
 * src/api/ops/matmul.cpp:166-171,541). Candidates are named by their kernel
 * ("gemm16_dma_128x128"; a split-K plan adds ":<chunks>"). float32 and
 * TVK_GEMM_EXACT products have only sequential-order candidates, which give
 * identical bits. The table is read from the tuning file on first use and
 * persisted one line per result, following the reference's tuning cache
 * (Autotuner::select/load/save, src/vulkan/autotuner.cpp:56-121; file
 * location VulkanCache::cachePath, src/vulkan/cache.cpp:181-202):
 * TORCHVULKAN_PIPELINE_CACHE=0 turns persistence off, the directory is
 * $TORCHVULKAN_CACHE_DIR, else $XDG_CACHE_HOME/torchvulkan, else
 * $HOME/.cache/torchvulkan, one file per device model. */

/* Newline-separated names of every kernel that computes `desc`'s product, the
 * shape-chosen one first ("none" for an empty product). TVK_ERR_INVALID when
 * names_len is too small. */
tvk_status tvk_gemm_candidates(const tvk_gemm_desc* desc, char* names, size_t names_len);

/* Records `kernel` (one of the candidates) for `desc`'s shape class, in the
 * tuning file too when persist != 0. */
tvk_status tvk_gemm_choose(const tvk_gemm_desc* desc, const char* kernel, int persist);

/* tvk_gemm that first, when the shape class has no recorded choice, times
 * every candidate (median of five launches after a warm-up) and records and
 * persists the fastest (Autotuner::fastest, src/vulkan/autotuner.cpp:123-223).
 * The timed launches write a scratch output when c overlaps an operand. Writes
 * the kernel used to `name` (may be NULL). Synchronizes the stream when it
 * times. */
tvk_status tvk_gemm_tune(const tvk_gemm_desc* desc, char* name, size_t name_len);

/* Forgets every recorded choice; the next use reads the environment and the
 * tuning file again. */
tvk_status tvk_tune_reset(void);

/* Path of the tuning file in use ("" when persistence is off). */
tvk_status tvk_tune_path(char* path, size_t path_len);

/* ------------------------------------------------------------------------- */
/* Compute: 2-D convolution as implicit GEMM                                  */
/* ------------------------------------------------------------------------- */

/* One 2-D convolution problem. Tensors are contiguous NCHW, weights
 * [c_out][c_in/groups][kh][kw] (the reference makes every operand contiguous
 * before its conv kernels, src/api/ops/conv.cpp:1101-1103,1145-1147). The
 * same descriptor serves the three directions; which pointers are read and
 * which one is written depends on the entry point:
 *   fwd:   y = conv(x, weight) + bias        (reads x, weight, bias; writes y)
 *   dgrad: x = conv_transpose(y, weight)     (reads y, weight; writes x)
 *   wgrad: weight = correlate(x, y)          (reads x, y; writes weight)
 * h_out/w_out must equal floor((h + 2p - d(k-1) - 1)/s) + 1.
 * Accumulation is float32; float32 (and every dtype under TVK_GEMM_EXACT)
 * accumulates each output over k in order, fused multiply-add per term. */
typedef struct {
    int32_t dtype;
    uint32_t flags;          /* TVK_GEMM_EXACT */
    int64_t n, c_in, h, w;
    int64_t c_out, kh, kw;
    int64_t stride[2], padding[2], dilation[2];
    int64_t groups;
    int64_t h_out, w_out;
    void* x;
    void* weight;
    const void* bias;        /* fwd only; NULL: none */
    void* y;
    void* stream;
} tvk_conv_desc;

/* Replaces implicit_forward (src/api/ops/conv.cpp:1014-1022) and its
 * conv_simd/conv_coop/winograd kernels. */
tvk_status tvk_conv2d_fwd(const tvk_conv_desc* desc);
/* Replaces implicit_grad_input (src/api/ops/conv.cpp:1024-1032), including
 * the transposed-convolution forward that reuses it (conv.cpp:1105). */
tvk_status tvk_conv2d_dgrad(const tvk_conv_desc* desc);
/* Replaces implicit_grad_weight (src/api/ops/conv.cpp:1034-1060). */
tvk_status tvk_conv2d_wgrad(const tvk_conv_desc* desc);

/* ------------------------------------------------------------------------- */
/* Compute: convolution with 1, 2 or 3 spatial dimensions                     */
/* ------------------------------------------------------------------------- */

/* One convolution problem with `spatial_dims` spatial dimensions (1, 2 or 3),
 * the reference's ConvProblem (src/api/ops/conv.cpp:247-255), which takes up
 * to three (implicit_gemm_supported, conv.cpp:295-311). Tensors are
 * contiguous NC[D][H]W, weights [c_out][c_in/groups][kernel...]. The spatial
 * arrays list the dimensions outermost first (D, H, W); only the first
 * `spatial_dims` entries are read. out_size[i] must equal
 * floor((in_size[i] + 2 padding[i] - dilation[i] (kernel[i] - 1) - 1) / stride[i]) + 1.
 * Directions, pointers and accumulation as tvk_conv_desc. One and two spatial
 * dimensions run the 2-D kernels (one as a height of 1); three run the 3-D
 * implicit-GEMM kernels, k = (channel, kd, kh, kw). */
typedef struct {
    int32_t dtype;
    uint32_t flags;          /* TVK_GEMM_EXACT */
    int32_t spatial_dims;    /* 1, 2 or 3 */
    int32_t reserved;        /* 0 */
    int64_t n, c_in, c_out, groups;
    int64_t in_size[3];
    int64_t kernel[3];
    int64_t stride[3], padding[3], dilation[3];
    int64_t out_size[3];
    void* x;
    void* weight;
    const void* bias;        /* fwd only; NULL: none */
    void* y;
    void* stream;
} tvk_convnd_desc;

/* Replaces implicit_forward (src/api/ops/conv.cpp:1014-1022) for 1-3 spatial
 * dimensions, with the N-d gathers of src/shaders/helpers/conv.slang:93-117. */
tvk_status tvk_conv_fwd(const tvk_convnd_desc* desc);
/* Replaces implicit_grad_input (src/api/ops/conv.cpp:1024-1032) for 1-3
 * spatial dimensions (and the transposed forward that reuses it, :1105). */
tvk_status tvk_conv_dgrad(const tvk_convnd_desc* desc);
/* Replaces implicit_grad_weight (src/api/ops/conv.cpp:1034-1060) for 1-3
 * spatial dimensions. */
tvk_status tvk_conv_wgrad(const tvk_convnd_desc* desc);

/* Kernel choice for convolutions: the reference tunes its conv tilings per
 * problem through the matmul autotuner (dispatch_conv_coop_shader,
 * src/api/ops/conv.cpp:499-659, keyed by mode and the log2 problem sizes,
 * :643-644). Here a 2-D problem (one or two spatial dimensions) can run on up
 * to four kernel families, "conv_stem", "conv_halo", "conv_ring" and
 * "conv_implicit_gemm"; the shape rule takes the first that applies, unless
 * the kernel-choice table (the one tvk_gemm_* use, same tuning file) records
 * another for the problem's shape class. float32, TVK_GEMM_EXACT and three
 * spatial dimensions have one family, "conv_implicit_gemm". `mode` is one of: */
#define TVK_CONV_FWD 0
#define TVK_CONV_DGRAD 1
#define TVK_CONV_WGRAD 2
/* Newline-separated names of every family that computes the problem, the
 * shape-chosen one first. TVK_ERR_INVALID when names_len is too small. */
tvk_status tvk_conv_candidates(const tvk_convnd_desc* desc, int mode, char* names, size_t names_len);
/* Records `kernel` (one of the candidates) for the problem's shape class, in
 * the tuning file too when persist != 0. */
tvk_status tvk_conv_choose(const tvk_convnd_desc* desc, int mode, const char* kernel, int persist);
/* The convolution of `mode`, first timing every candidate (median of five
 * calls after a warm-up) and recording and persisting the fastest when the
 * shape class has no recorded choice. The timed calls write the problem's own
 * output. Writes the family used to `name` (may be NULL). Synchronizes the
 * stream when it times. */
tvk_status tvk_conv_tune(const tvk_convnd_desc* desc, int mode, char* name, size_t name_len);

#ifdef __cplusplus
}
#endif

#endif /* TVK_HIP_H */
