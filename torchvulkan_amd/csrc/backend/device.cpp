// PrivateUse1 device plumbing: allocator, device guard, hooks, the boxed CPU
// fallback, tensor creation / views / copies, and the `_C` Python module.
//
// Mirrors the reference's registration layer: allocator (src/vulkan/allocator.cpp),
// guard (src/api/guard.cpp:19-100), hooks (src/api/hook.cpp:53-83), fallback
// (src/api/fallback.cpp:5-13), tensor basics (src/api/tensor/allocation.cpp:238-247,
// transfer.cpp:392-397, views.cpp:151-158) and the pybind module
// (src/api/backend.cpp:9-130). Device memory comes from tvk_malloc; copies run
// on the library stream.
#include "common.h"

#include <ATen/EmptyTensor.h>
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/set_native.h>
#include <ATen/ops/view_as_complex_native.h>
#include <ATen/ops/view_as_real_native.h>
#include <ATen/ops/view_native.h>
#include <c10/core/Allocator.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <unordered_map>

namespace tvkb {

bool strict_mode() {
    const char* v = std::getenv("TORCHVULKAN_STRICT");
    return v && std::strcmp(v, "0") != 0 && v[0] != '\0';
}

void check_status(tvk_status st, const char* what) {
    if (st == TVK_OK) return;
    std::string msg = std::string("torchvulkan [ERROR]: ") + tvk_last_error();
    if (msg.size() == 21) msg += what;
    if (st == TVK_ERR_OOM) TORCH_CHECK_WITH(OutOfMemoryError, false, msg);
    TORCH_CHECK(false, msg);
}

void* stream_of(c10::DeviceIndex index) {
    void* s = nullptr;
    check_status(tvk_get_stream(index < 0 ? 0 : index, &s), "tvk_get_stream");
    return s;
}

int32_t tvk_dtype_of(c10::ScalarType t, bool& ok) {
    ok = true;
    switch (t) {
    case at::kFloat: return TVK_F32;
    case at::kHalf: return TVK_F16;
    case at::kBFloat16: return TVK_BF16;
    default: ok = false; return -1;
    }
}

void view_extent(const at::Tensor& t, int64_t& lo, int64_t& n) {
    lo = t.storage_offset();
    int64_t hi = lo;
    for (int64_t d = 0; d < t.dim(); ++d) {
        TORCH_CHECK(t.stride(d) >= 0, "torchvulkan [ERROR]: negative strides are not supported");
        if (t.size(d) == 0) { n = 0; return; }
        hi += (t.size(d) - 1) * t.stride(d);
    }
    n = hi - lo + 1;
}

int32_t copy_dtype_of(c10::ScalarType t, bool& ok) {
    ok = true;
    switch (t) {
    case at::kFloat: return TVK_F32;
    case at::kHalf: return TVK_F16;
    case at::kBFloat16: return TVK_BF16;
    case at::kDouble: return TVK_F64;
    case at::kLong: return TVK_I64;
    case at::kInt: return TVK_I32;
    case at::kShort: return TVK_I16;
    case at::kChar: return TVK_I8;
    case at::kByte: return TVK_U8;
    case at::kBool: return TVK_BOOL;
    case at::kFloat8_e4m3fn: return TVK_F8E4M3FN;
    case at::kFloat8_e5m2: return TVK_F8E5M2;
    default: ok = false; return -1;
    }
}

bool device_copyable(const at::Tensor& src, const at::Tensor& dst) {
    bool a = false, b = false;
    copy_dtype_of(src.scalar_type(), a);
    copy_dtype_of(dst.scalar_type(), b);
    return a && b && dst.dim() <= TVK_COPY_MAX_DIMS && !src.is_conj() && !src.is_neg() && !dst.is_conj() &&
           !dst.is_neg();
}

void device_copy(const at::Tensor& src, const at::Tensor& dst) {
    if (dst.numel() == 0) return;
    const at::Tensor s = src.sizes() == dst.sizes() ? src : src.expand(dst.sizes());
    tvk_copy_desc d;
    std::memset(&d, 0, sizeof(d));
    bool ok = false;
    d.src_dtype = copy_dtype_of(s.scalar_type(), ok);
    d.dst_dtype = copy_dtype_of(dst.scalar_type(), ok);
    d.ndim = (int32_t)dst.dim();
    for (int64_t k = 0; k < dst.dim(); ++k) {
        d.sizes[k] = dst.size(k);
        d.src_strides[k] = s.stride(k);
        d.dst_strides[k] = dst.stride(k);
    }
    d.src = s.data_ptr();
    d.dst = dst.data_ptr();
    d.stream = stream_of(dst);
    check_status(tvk_copy(&d), "tvk_copy");
}

namespace {

// The byte-extent route for dtypes the device copy does not take (complex,
// float8, unsigned 16-64 bit): the whole storage extent of the view crosses
// PCIe and the host applies the strides.
at::Tensor to_host_extent(const at::Tensor& t) {
    at::Tensor out = at::empty(t.sizes(), t.options().device(at::kCPU));
    int64_t lo = 0, n = 0;
    view_extent(t, lo, n);
    const int64_t es = t.element_size();
    at::Tensor buf = at::empty({n}, t.options().device(at::kCPU));
    const char* src = static_cast<const char*>(t.storage().data()) + lo * es;
    check_status(tvk_memcpy_d2h(buf.data_ptr(), src, (size_t)(n * es), stream_of(t), 1), "copy to host");
    std::vector<int64_t> strides(t.strides().begin(), t.strides().end());
    out.copy_(buf.as_strided(t.sizes(), strides, 0));
    return out;
}

void from_host_extent(const at::Tensor& src, const at::Tensor& dst) {
    int64_t lo = 0, n = 0;
    view_extent(dst, lo, n);
    const int64_t es = dst.element_size();
    void* s = stream_of(dst);
    at::Tensor buf = at::empty({n}, dst.options().device(at::kCPU));
    char* base = static_cast<char*>(dst.storage().mutable_data()) + lo * es;
    check_status(tvk_memcpy_d2h(buf.data_ptr(), base, (size_t)(n * es), s, 1), "copy to host");
    std::vector<int64_t> strides(dst.strides().begin(), dst.strides().end());
    buf.as_strided(dst.sizes(), strides, 0).copy_(src);
    check_status(tvk_memcpy_h2d(base, buf.data_ptr(), (size_t)(n * es), s, 1), "copy to device");
}

}  // namespace

// Device -> host, after copy_vulkan_to_host (src/api/tensor/transfer.cpp:78-127):
// expanded dimensions are narrowed to their one distinct slice first; a
// strided view is gathered on the device into a dense buffer, which is the
// only thing that crosses PCIe.
at::Tensor to_host(const at::Tensor& t) {
    at::Tensor out = at::empty(t.sizes(), t.options().device(at::kCPU));
    if (t.numel() == 0) return out;
    bool ok = false;
    copy_dtype_of(t.scalar_type(), ok);
    if (!ok || t.dim() > TVK_COPY_MAX_DIMS) return to_host_extent(t);
    at::Tensor distinct = t;
    bool expanded = false;
    for (int64_t d = 0; d < t.dim(); ++d)
        if (t.stride(d) == 0 && t.size(d) > 1) {
            distinct = distinct.narrow(d, 0, 1);
            expanded = true;
        }
    at::Tensor dense = distinct;
    if (!distinct.is_contiguous()) {
        dense = at::empty(distinct.sizes(), distinct.options().memory_format(at::MemoryFormat::Contiguous));
        device_copy(distinct, dense);
    }
    at::Tensor host = expanded ? at::empty(distinct.sizes(), out.options()) : out;
    check_status(tvk_memcpy_d2h(host.data_ptr(), dense.data_ptr(), (size_t)(dense.numel() * dense.element_size()),
                                stream_of(t), 1),
                 "copy to host");
    if (expanded) out.copy_(host.expand(t.sizes()));
    return out;
}

// Host -> device, after copy_host_to_vulkan (src/api/tensor/transfer.cpp:58-76):
// the host converts to the destination dtype and packs densely; a strided
// destination is written from a dense device staging buffer by tvk_copy.
void from_host(const at::Tensor& host, const at::Tensor& dst) {
    if (dst.numel() == 0) return;
    at::Tensor src = host.to(dst.scalar_type());
    if (src.sizes() != dst.sizes()) src = src.expand(dst.sizes());
    src = src.contiguous();
    void* s = stream_of(dst);
    if (dst.is_contiguous()) {
        check_status(tvk_memcpy_h2d(dst.data_ptr(), src.data_ptr(), (size_t)(src.numel() * src.element_size()), s, 1),
                     "copy to device");
        return;
    }
    if (!device_copyable(dst, dst)) {
        from_host_extent(src, dst);
        return;
    }
    at::Tensor staging = at::empty(dst.sizes(), dst.options().memory_format(at::MemoryFormat::Contiguous));
    check_status(tvk_memcpy_h2d(staging.data_ptr(), src.data_ptr(), (size_t)(src.numel() * src.element_size()), s, 1),
                 "copy to device");
    device_copy(staging, dst);
}

namespace {

// ---------------------------------------------------------------------------
// allocator
// ---------------------------------------------------------------------------

thread_local c10::DeviceIndex g_current = 0;

void free_fn(void* p) {
    if (p) (void)tvk_free(p);
}

struct TvkAllocator final : c10::Allocator {
    c10::DataPtr allocate(size_t nbytes) override {
        const c10::DeviceIndex dev = g_current;
        void* p = nullptr;
        if (nbytes) {
            check_status(tvk_malloc(dev, nbytes, &p), "tvk_malloc");
            int spilled = 0;
            (void)tvk_last_malloc_spilled(&spilled);
            // the reference's warning (src/vulkan/allocator.cpp:189-195)
            if (spilled) {
                TORCH_WARN_ONCE("torchvulkan [WARNING]: Vulkan memory may be allocated using host memory, which may cause "
                                "performance degradation. Set TORCHVULKAN_STRICT_ALLOCATION=1 to raise an out-of-memory "
                                "error instead.");
            }
        }
        return {p, p, &free_fn, c10::Device(c10::DeviceType::PrivateUse1, dev)};
    }
    c10::DeleterFnPtr raw_deleter() const override { return &free_fn; }
    void copy_data(void* dest, const void* src, std::size_t count) const override {
        check_status(tvk_memcpy_d2d(dest, src, count, stream_of(g_current)), "tvk_memcpy_d2d");
    }
};

TvkAllocator g_allocator;

// Pinned host memory for tensor.pin_memory() (src/api/hook.cpp:14-51): page-
// locked blocks from tvk_host_malloc, which the device's copies reach by DMA.
void pinned_free_fn(void* p) {
    if (p) (void)tvk_host_free(p);
}

struct TvkPinnedAllocator final : c10::Allocator {
    c10::DataPtr allocate(size_t nbytes) override {
        void* p = nullptr;
        if (nbytes) check_status(tvk_host_malloc(nbytes, &p), "tvk_host_malloc");
        return {p, p, &pinned_free_fn, c10::Device(c10::DeviceType::CPU)};
    }
    c10::DeleterFnPtr raw_deleter() const override { return &pinned_free_fn; }
    void copy_data(void* dest, const void* src, std::size_t count) const override { std::memcpy(dest, src, count); }
};

TvkPinnedAllocator g_pinned_allocator;

// ---------------------------------------------------------------------------
// device guard. Every stream id of a device names the device's one library
// stream (the reference's guard likewise hands out stream ids over one queue,
// src/api/guard.cpp:24-33); the current id is kept per thread and device.
// Events are HIP events recorded on that stream, so torch.Event record, wait,
// query and elapsed_time are stream-ordered and timed on the GPU clock
// (the reference stamps host time after draining the queue, guard.cpp:44-61).
// ---------------------------------------------------------------------------

struct TvkGuardImpl final : c10::impl::DeviceGuardImplInterface {
    c10::DeviceType type() const override { return c10::DeviceType::PrivateUse1; }
    c10::Device exchangeDevice(c10::Device d) const override {
        c10::Device old = getDevice();
        setDevice(d);
        return old;
    }
    c10::Device getDevice() const override { return c10::Device(c10::DeviceType::PrivateUse1, g_current); }
    void setDevice(c10::Device d) const override {
        TORCH_CHECK(d.type() == c10::DeviceType::PrivateUse1, "torchvulkan [ERROR]: expected a vulkan device");
        if (d.index() >= 0) {
            check_status(tvk_set_device(d.index()), "tvk_set_device");
            g_current = d.index();
        }
    }
    void uncheckedSetDevice(c10::Device d) const noexcept override {
        if (d.index() >= 0 && tvk_set_device(d.index()) == TVK_OK) g_current = d.index();
    }
    c10::Stream getStream(c10::Device d) const noexcept override {
        d = indexed(d);
        return c10::Stream(c10::Stream::UNSAFE, d, current_ids()[d.index()]);
    }
    c10::Stream getDefaultStream(c10::Device d) const override { return c10::Stream(c10::Stream::UNSAFE, indexed(d), 0); }
    c10::Stream getStreamFromGlobalPool(c10::Device d, bool) const override { return getNewStream(d, 0); }
    c10::Stream getNewStream(c10::Device d, int) const override {
        static std::atomic<c10::StreamId> next{0};
        return c10::Stream(c10::Stream::UNSAFE, indexed(d), ++next);
    }
    c10::Stream exchangeStream(c10::Stream s) const noexcept override {
        const c10::Device d = indexed(s.device());
        c10::StreamId& cur = current_ids()[d.index()];
        c10::Stream prev(c10::Stream::UNSAFE, d, cur);
        cur = s.id();
        return prev;
    }
    c10::DeviceIndex deviceCount() const noexcept override {
        int n = 0;
        (void)tvk_device_count(&n);
        return static_cast<c10::DeviceIndex>(n);
    }
    bool queryStream(const c10::Stream& s) const override {
        int done = 0;
        check_status(tvk_stream_query(stream_of(s.device_index()), &done), "tvk_stream_query");
        return done != 0;
    }
    void synchronizeStream(const c10::Stream& s) const override { synchronizeDevice(s.device_index()); }
    void synchronizeDevice(const c10::DeviceIndex index) const override {
        check_status(tvk_synchronize(index < 0 ? g_current : index), "tvk_synchronize");
    }
    void destroyEvent(void* event, const c10::DeviceIndex) const noexcept override { (void)tvk_event_destroy(event); }
    void record(void** event, const c10::Stream& stream, const c10::DeviceIndex device_index,
                const c10::EventFlag flag) const override {
        TORCH_CHECK(device_index == -1 || device_index == stream.device_index(), "Event device index ", device_index,
                    " does not match recording stream's device index ", stream.device_index(), ".");
        if (*event == nullptr) {
            // torch's default events do not time (as on CUDA); enable_timing asks for the backend default
            const int timing = flag == c10::EventFlag::BACKEND_DEFAULT ? 1 : 0;
            check_status(tvk_event_create(stream.device_index(), timing, event), "tvk_event_create");
        }
        check_status(tvk_event_record(*event, stream_of(stream.device_index())), "tvk_event_record");
    }
    void block(void* event, const c10::Stream& stream) const override {
        if (event) check_status(tvk_stream_wait_event(stream_of(stream.device_index()), event), "tvk_stream_wait_event");
    }
    bool queryEvent(void* event) const override {
        if (!event) return true;
        int done = 0;
        check_status(tvk_event_query(event, &done), "tvk_event_query");
        return done != 0;
    }
    void synchronizeEvent(void* event) const override {
        if (event) check_status(tvk_event_synchronize(event), "tvk_event_synchronize");
    }
    double elapsedTime(void* a, void* b, const c10::DeviceIndex) const override {
        TORCH_CHECK(a && b, "Both events must be recorded before calculating elapsed time.");
        float ms = 0.0f;
        check_status(tvk_event_elapsed(a, b, &ms), "tvk_event_elapsed");
        return ms;
    }

private:
    c10::Device indexed(c10::Device d) const { return d.has_index() ? d : getDevice(); }
    static std::unordered_map<c10::DeviceIndex, c10::StreamId>& current_ids() {
        thread_local std::unordered_map<c10::DeviceIndex, c10::StreamId> ids;
        return ids;
    }
};

C10_REGISTER_GUARD_IMPL(PrivateUse1, TvkGuardImpl);

// ---------------------------------------------------------------------------
// hooks
// ---------------------------------------------------------------------------

struct TvkHooks final : at::PrivateUse1HooksInterface {
    bool isBuilt() const override { return true; }
    bool isAvailable() const override {
        int n = 0;
        return tvk_device_count(&n) == TVK_OK && n > 0;
    }
    const at::Generator& getDefaultGenerator(c10::DeviceIndex) const override {
        // random numbers on this path are drawn on the host (the CPU fallback)
        return at::detail::getDefaultCPUGenerator();
    }
    at::Device getDeviceFromPtr(void* data) const override {
        int dev = -1;
        (void)tvk_pointer_device(data, &dev);
        TORCH_CHECK(dev >= 0, "torchvulkan [ERROR]: pointer was not allocated by the vulkan allocator");
        return at::Device(at::DeviceType::PrivateUse1, static_cast<c10::DeviceIndex>(dev));
    }
    bool isPinnedPtr(const void* p) const override {
        int pinned = 0;
        return tvk_host_pointer_pinned(p, &pinned) == TVK_OK && pinned != 0;
    }
    at::Allocator* getPinnedMemoryAllocator() const override { return &g_pinned_allocator; }
    bool hasPrimaryContext(c10::DeviceIndex) const override { return true; }
    void resizePrivateUse1Bytes(const c10::Storage& storage, size_t newsize) const override {
        c10::StorageImpl* impl = storage.unsafeGetStorageImpl();
        const size_t old = impl->nbytes();
        if (newsize == old) return;
        c10::DataPtr fresh = g_allocator.allocate(newsize);
        const size_t keep = std::min(old, newsize);
        if (keep) check_status(tvk_memcpy_d2d(fresh.get(), impl->data(), keep, stream_of(g_current)), "resize copy");
        impl->set_data_ptr_noswap(std::move(fresh));
        impl->set_nbytes(newsize);
    }
};

struct HooksRegistrar {
    HooksRegistrar() {
        at::RegisterPrivateUse1HooksInterface(new TvkHooks());
        c10::SetAllocator(c10::DeviceType::PrivateUse1, &g_allocator);
    }
} g_hooks_registrar;

// ---------------------------------------------------------------------------
// boxed CPU fallback (src/api/fallback.cpp:5-13)
// ---------------------------------------------------------------------------

void cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
    TVKB_FALLBACK("Silent fallback detected for operation: ", op.schema().operator_name(), ".");
    at::native::cpu_fallback(op, stack);
}

// ---------------------------------------------------------------------------
// tensor basics
// ---------------------------------------------------------------------------

at::Tensor empty_memory_format(c10::IntArrayRef size, std::optional<at::ScalarType> dtype, std::optional<at::Layout> layout,
                               std::optional<at::Device> device, std::optional<bool> pin_memory,
                               std::optional<at::MemoryFormat> memory_format) {
    const c10::DeviceGuard guard(device.value_or(c10::Device(c10::DeviceType::PrivateUse1, g_current)));
    constexpr c10::DispatchKeySet ks(c10::DispatchKey::PrivateUse1);
    return at::detail::empty_generic(size, &g_allocator, ks, c10::dtype_or_default(dtype), memory_format);
}

at::Tensor empty_strided(c10::IntArrayRef size, c10::IntArrayRef stride, std::optional<at::ScalarType> dtype,
                         std::optional<at::Layout> layout, std::optional<at::Device> device, std::optional<bool> pin_memory) {
    const c10::DeviceGuard guard(device.value_or(c10::Device(c10::DeviceType::PrivateUse1, g_current)));
    constexpr c10::DispatchKeySet ks(c10::DispatchKey::PrivateUse1);
    return at::detail::empty_strided_generic(size, stride, &g_allocator, ks, c10::dtype_or_default(dtype));
}

// Copies with a complex side, on one device, as copies of the (real,
// imaginary) pairs (copy_complex_vulkan_to_vulkan,
// src/api/tensor/transfer.cpp:228-244): complex to complex casts the pairs;
// real to complex writes the real parts and zeroes the imaginary ones;
// complex to real keeps the real parts (the caller warned). False when not
// applicable (the caller resolves conjugate and negative views first).
bool complex_copy(const at::Tensor& src, const at::Tensor& dst) {
    if (!src.is_complex() && !dst.is_complex()) return false;
    if (src.device() != dst.device() || src.is_conj() || src.is_neg() || dst.is_conj() || dst.is_neg()) return false;
    if (dst.dim() + 1 > TVK_COPY_MAX_DIMS) return false;
    bool ok_s = false, ok_d = false;
    copy_dtype_of(c10::toRealValueType(src.scalar_type()), ok_s);
    copy_dtype_of(c10::toRealValueType(dst.scalar_type()), ok_d);
    if (!ok_s || !ok_d) return false;
    if (src.is_complex() && dst.is_complex()) {
        at::Tensor d = at::view_as_real(dst);
        d.copy_(at::view_as_real(src));
    } else if (dst.is_complex()) {
        at::Tensor pairs = at::view_as_real(dst);
        pairs.select(-1, 0).copy_(src);
        pairs.select(-1, 1).zero_();
    } else {
        at::Tensor d = dst;
        d.copy_(at::view_as_real(src).select(-1, 0));
    }
    return true;
}

// A copy with a pending conjugation or negation on either side
// (copy_vulkan's lazily conjugated / negated cases, transfer.cpp:306-331).
// A tensor's values are (neg ? -1 : 1) * (conj ? conj(stored) : stored), so
// dst's stored values become the source's stored values, negated where
// exactly one side is negative and with the imaginary parts negated where
// exactly one side is conjugate: a plain copy of the stored values, then
// those sign flips on dst's side (on the device for a vulkan dst).
at::Tensor copy_math_bits(const at::Tensor& self, const at::Tensor& dst) {
    at::Tensor s = self, d = dst;
    if (s.is_conj()) s = at::_conj(s);        // the same storage without the pending conjugation
    if (s.is_neg()) s = at::_neg_view(s);
    if (d.is_conj()) d = at::_conj(d);
    if (d.is_neg()) d = at::_neg_view(d);
    d.copy_(s);
    const bool flip_all = self.is_neg() != dst.is_neg();
    const bool flip_im = self.is_conj() != dst.is_conj() && d.is_complex();
    if (flip_all || flip_im) {
        at::Tensor pairs = d.is_complex() ? at::view_as_real(d) : d;
        if (flip_all) pairs.mul_(-1);
        if (flip_im) pairs.select(-1, 1).mul_(-1);
    }
    return dst;
}

// _copy_from: torch routes copy_ here whenever one side is a vulkan tensor
// (torchvulkan::copy_vulkan, src/api/tensor/transfer.cpp:292-397). Device to
// device copies, casts and layout changes run on the device (tvk_copy);
// crossing to or from the host moves only dense bytes.
at::Tensor copy_from(const at::Tensor& self, const at::Tensor& dst, bool non_blocking) {
    if (dst.numel() == 0) return dst;
    // as at::native::copy_, a copy onto its own memory is a no-op
    if (self.is_alias_of(dst) && self.storage_offset() == dst.storage_offset() && self.sizes().equals(dst.sizes()) &&
        self.strides().equals(dst.strides()) && self.scalar_type() == dst.scalar_type() &&
        self.is_conj() == dst.is_conj() && self.is_neg() == dst.is_neg())
        return dst;
    if (self.is_conj() || self.is_neg() || dst.is_conj() || dst.is_neg()) return copy_math_bits(self, dst);
    at::Tensor src = self;
    if (src.sizes() != dst.sizes()) {
        if (at::is_expandable_to(src.sizes(), dst.sizes())) src = src.expand(dst.sizes());
        else {
            TORCH_CHECK(src.numel() == dst.numel(), "torchvulkan [ERROR]: _copy_from size mismatch");
            src = src.reshape(dst.sizes());
        }
    }
    if (src.is_privateuseone() && dst.is_privateuseone()) {
        if (device_copyable(src, dst)) {
            at::assert_no_internal_overlap(dst);
            at::assert_no_partial_overlap(dst, src);
            if (src.device() != dst.device()) {
                // another device's memory: stage through a dense buffer on the destination
                at::Tensor dense = src.contiguous();
                at::Tensor staged = at::empty(dense.sizes(), dense.options().device(dst.device()));
                check_status(tvk_synchronize(src.device().index()), "tvk_synchronize");
                check_status(tvk_memcpy_d2d(staged.data_ptr(), dense.data_ptr(),
                                            (size_t)(dense.numel() * dense.element_size()), stream_of(dst)),
                             "tvk_memcpy_d2d");
                device_copy(staged, dst);
            } else {
                device_copy(src, dst);
            }
            return dst;
        }
        if (complex_copy(src, dst)) return dst;
        TVKB_FALLBACK("A copy from ", src.scalar_type(), " to ", dst.scalar_type(), " can't run on the device. Falling back to CPU.");
        from_host(to_host(src), dst);
        return dst;
    }
    if (dst.is_privateuseone()) {
        from_host(src, dst);
        return dst;
    }
    // device -> host: a cast the device can do is done before the transfer
    if (src.scalar_type() != dst.scalar_type() && device_copyable(src, dst)) {
        at::Tensor cast = at::empty(src.sizes(), src.options().dtype(dst.scalar_type()).memory_format(at::MemoryFormat::Contiguous));
        device_copy(src, cast);
        src = cast;
    }
    dst.copy_(to_host(src));
    return dst;
}

// fill_.Scalar / zero_ / fill_.Tensor (src/api/ops/fill.cpp:11-133): the host
// converts the scalar to the element type, the device writes its bytes. The
// conversion is a CPU fill of one element (for a one-element tensor) or of two
// (otherwise), so the value and the overflow error are those of the CPU's fill
// of the same tensor: CPU fill_ converts a lone element without the overflow
// check it applies to larger tensors.
at::Tensor& fill_scalar(at::Tensor& self, const at::Scalar& value) {
    if (self.numel() == 0) return self;
    bool ok = false;
    copy_dtype_of(self.scalar_type(), ok);
    at::Tensor one = at::empty({self.numel() == 1 ? 1 : 2}, self.options().device(at::kCPU)).fill_(value);
    if (!ok || self.dim() > TVK_COPY_MAX_DIMS || self.is_conj() || self.is_neg()) {
        TVKB_FALLBACK("Can't fill a ", self.scalar_type(), " tensor of this shape on the device. Falling back to CPU.");
        from_host(one.narrow(0, 0, 1).expand(self.sizes()), self);
        return self;
    }
    at::Tensor t = self;
    for (int64_t d = 0; d < t.dim(); ++d)
        if (t.stride(d) == 0 && t.size(d) > 1) t = t.narrow(d, 0, 1);   // one write per distinct element
    tvk_fill_desc fd;
    std::memset(&fd, 0, sizeof(fd));
    fd.elem_size = (int32_t)t.element_size();
    fd.ndim = (int32_t)t.dim();
    for (int64_t k = 0; k < t.dim(); ++k) {
        fd.sizes[k] = t.size(k);
        fd.dst_strides[k] = t.stride(k);
    }
    fd.dst = t.data_ptr();
    std::memcpy(&fd.pattern, one.data_ptr(), (size_t)one.element_size());   // element 0
    fd.stream = stream_of(t);
    check_status(tvk_fill(&fd), "tvk_fill");
    return self;
}

at::Tensor& zero_(at::Tensor& self) { return fill_scalar(self, 0); }

at::Tensor& fill_tensor(at::Tensor& self, const at::Tensor& value) {
    TORCH_CHECK(value.dim() == 0, "fill_ only supports 0-dimension value tensor but got tensor with ", value.dim(),
                " dimensions.");
    return fill_scalar(self, value.item());
}

at::Tensor copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
    at::native::resize_output(dst, self.sizes());
    return copy_from(self, dst, false);
}

at::Scalar local_scalar_dense(const at::Tensor& self) { return to_host(self).item(); }

const at::Tensor& resize_(const at::Tensor& self, c10::IntArrayRef size, std::optional<at::MemoryFormat> memory_format) {
    at::TensorImpl* impl = self.unsafeGetTensorImpl();
    impl->set_sizes_contiguous(size);
    const size_t itemsize = impl->dtype().itemsize();
    const size_t need = at::detail::computeStorageNbytesContiguous(size, itemsize, impl->storage_offset());
    if (need > impl->storage().nbytes()) {
        at::detail::getPrivateUse1Hooks().resizePrivateUse1Bytes(impl->storage(), need);
    }
    if (memory_format.has_value() && *memory_format != at::MemoryFormat::Preserve) {
        impl->empty_tensor_restride(*memory_format);
    }
    return self;
}

}  // namespace
}  // namespace tvkb

// _copy_from sees conjugate and negative views itself (copy_math_bits): the
// generic math-bit fallback would resolve them by a clone, which is a copy_
// and so another _copy_from of the same view, without end.
TORCH_LIBRARY_IMPL(aten, Conjugate, m) {
    m.impl("_copy_from", torch::CppFunction::makeFallthrough());
    m.impl("_copy_from_and_resize", torch::CppFunction::makeFallthrough());
}

TORCH_LIBRARY_IMPL(aten, Negative, m) {
    m.impl("_copy_from", torch::CppFunction::makeFallthrough());
    m.impl("_copy_from_and_resize", torch::CppFunction::makeFallthrough());
}

TORCH_LIBRARY_IMPL(_, PrivateUse1, m) {
    m.fallback(torch::CppFunction::makeFromBoxedFunction<&tvkb::cpu_fallback>());
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
    m.impl("empty.memory_format", &tvkb::empty_memory_format);
    m.impl("empty_strided", &tvkb::empty_strided);
    m.impl("as_strided", &at::native::as_strided_tensorimpl);
    m.impl("view_as_real", &at::native::view_as_real);
    m.impl("view_as_complex", &at::native::view_as_complex);
    m.impl("view", &at::native::view);
    m.impl("_reshape_alias", &at::native::_reshape_alias);
    m.impl("resize_", &tvkb::resize_);
    m.impl("set_.source_Storage", &at::native::set_);
    m.impl("set_.source_Storage_storage_offset", &at::native::set_storage_cpu_);
    m.impl("_copy_from", &tvkb::copy_from);
    m.impl("_copy_from_and_resize", &tvkb::copy_from_and_resize);
    m.impl("fill_.Scalar", &tvkb::fill_scalar);
    m.impl("fill_.Tensor", &tvkb::fill_tensor);
    m.impl("zero_", &tvkb::zero_);
    m.impl("_local_scalar_dense", &tvkb::local_scalar_dense);
}

// ---------------------------------------------------------------------------
// Python module (the reference's _C, src/api/backend.cpp:9-130)
// ---------------------------------------------------------------------------

namespace {
size_t stat(tvk_status (*fn)(int, size_t*), int64_t dev) {
    size_t v = 0;
    tvkb::check_status(fn((int)dev, &v), "memory statistics");
    return v;
}
}  // namespace

PYBIND11_MODULE(_C, m) {
    m.doc() = "torchvulkan_amd backend: the vulkan (PrivateUse1) device on MI355X";
    m.def("is_available", []() {
        int n = 0;
        return tvk_device_count(&n) == TVK_OK && n > 0;
    });
    m.def("device_count", []() -> int64_t {
        int n = 0;
        (void)tvk_device_count(&n);
        return n;
    });
    m.def("current_device", []() -> int64_t { return tvkb::g_current; });
    m.def("set_device", [](int64_t d) {
        tvkb::check_status(tvk_set_device((int)d), "set_device");
        tvkb::g_current = static_cast<c10::DeviceIndex>(d);
    });
    m.def("synchronize", [](int64_t d) { tvkb::check_status(tvk_synchronize((int)d), "synchronize"); },
          py::call_guard<py::gil_scoped_release>());
    m.def("empty_cache", [](int64_t d) { tvkb::check_status(tvk_empty_cache((int)d), "empty_cache"); },
          py::call_guard<py::gil_scoped_release>());
    m.def("_memory_allocated", [](int64_t d) { return stat(tvk_memory_allocated, d); });
    m.def("_max_memory_allocated", [](int64_t d) { return stat(tvk_max_memory_allocated, d); });
    m.def("_memory_reserved", [](int64_t d) { return stat(tvk_memory_reserved, d); });
    m.def("_reset_peak_memory_stats", [](int64_t d) { tvkb::check_status(tvk_reset_peak_memory_stats((int)d), "reset_peak"); });
    m.def("_set_memory_limit", [](int64_t d, size_t bytes) { tvkb::check_status(tvk_set_memory_limit((int)d, bytes), "limit"); });
    m.def("_set_strict_allocation", [](bool on) { tvkb::check_status(tvk_set_strict_allocation(on ? 1 : 0), "strict allocation"); });
    m.def("_strict_allocation", []() {
        int on = 0;
        tvkb::check_status(tvk_get_strict_allocation(&on), "strict allocation");
        return on != 0;
    });
    m.def("_mem_get_info", [](int64_t d) {
        size_t f = 0, t = 0;
        tvkb::check_status(tvk_mem_get_info((int)d, &f, &t), "mem_get_info");
        return std::make_pair(f, t);
    });
    m.def("_device_properties", [](int64_t d) {
        tvk_device_props p;
        tvkb::check_status(tvk_device_properties((int)d, &p), "device_properties");
        py::dict info;
        info["name"] = std::string(p.name);
        info["arch"] = std::string(p.arch);
        info["total_memory"] = p.total_memory;
        info["compute_units"] = p.compute_units;
        info["clock_khz"] = p.clock_khz;
        info["subgroup_size"] = p.wavefront_size;
        info["has_fp64"] = (bool)p.has_fp64;
        info["has_fp16"] = (bool)p.has_fp16;
        info["has_bf16"] = (bool)p.has_bf16;
        return info;
    });
    m.def("_strict", []() { return tvkb::strict_mode(); });
}
