// Shared helpers of the PrivateUse1 ("vulkan") backend extension. The backend
// is the reference's operator surface (src/api/**) kept as-is; everything it
// does on the device goes through the C ABI of libtvk_hip.so.
#pragma once

#include <torch/extension.h>
#include <c10/core/Device.h>

#include <string>

#include "../../../include/tvk_hip.h"

namespace tvkb {

// TORCHVULKAN_STRICT=1 turns every CPU fallback into an error
// (src/api/fallback.h:7-11).
bool strict_mode();

// The reference's TORCHVULKAN_FALLBACK: warn once, or raise under strict mode.
#define TVKB_FALLBACK(...)                                                                                         \
    do {                                                                                                            \
        if (::tvkb::strict_mode())                                                                                  \
            TORCH_CHECK(false, "torchvulkan [NOT IMPLEMENTED]: ", __VA_ARGS__,                                      \
                        " Set TORCHVULKAN_STRICT=0 to disable strict mode.");                                       \
        TORCH_WARN_ONCE("torchvulkan [WARNING]: ", __VA_ARGS__, " Set TORCHVULKAN_STRICT=1 to enable strict mode."); \
    } while (0)

// Raises a RuntimeError (or OutOfMemoryError) carrying tvk_last_error().
void check_status(tvk_status st, const char* what);

// The library stream of a device: every kernel and copy of the backend is
// ordered on it, so allocator reuse and data hazards follow stream order.
void* stream_of(c10::DeviceIndex index);
inline void* stream_of(const at::Tensor& t) { return stream_of(t.device().index()); }

// Byte extent [lo, hi) of a strided view inside its storage.
void view_extent(const at::Tensor& t, int64_t& lo_elems, int64_t& n_elems);

// Values of a device tensor (any strides) as a new contiguous CPU tensor.
at::Tensor to_host(const at::Tensor& t);
// Writes a CPU tensor's values into a device tensor (any strides, same shape).
void from_host(const at::Tensor& host, const at::Tensor& dst);

int32_t tvk_dtype_of(c10::ScalarType t, bool& ok);
// tvk_dtype of every dtype tvk_copy handles.
int32_t copy_dtype_of(c10::ScalarType t, bool& ok);
// Both dtypes have a device copy, the dimension count fits, and neither side is
// a lazily conjugated or negated view.
bool device_copyable(const at::Tensor& src, const at::Tensor& dst);
// dst.copy_(src) on the device (both device tensors on dst's device; src
// broadcast to dst's shape), ordered on dst's stream.
void device_copy(const at::Tensor& src, const at::Tensor& dst);

}  // namespace tvkb
