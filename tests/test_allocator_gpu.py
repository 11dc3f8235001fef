"""The caching allocator's policy past the device's memory and the pinned host
allocator, on the vulkan device.

- TORCHVULKAN_STRICT_ALLOCATION (src/vulkan/allocator.cpp:171-200,
  src/vulkan/vulkan_context.cpp:248): past the budget (tvk_set_memory_limit),
  strict allocation raises torch.OutOfMemoryError; otherwise the block comes
  from pinned host memory, kernels still compute on it, and the values match.
- pin_memory on the vulkan device (src/api/hook.cpp:14-69): blocks from
  tvk_host_malloc, reported by is_pinned, usable as copy sources and targets.
"""
from __future__ import annotations

import ctypes as C
import warnings

import pytest
import torch

pytestmark = pytest.mark.gpu

V = "vulkan"


def test_budget_strict_and_spilled(gpu):
    import torchvulkan_amd as tv

    tv.synchronize()
    tv.empty_cache()
    lib = gpu.load()
    base = tv.memory_allocated()
    old_strict = tv._C._strict_allocation()
    tv._C._set_memory_limit(0, base + (1 << 20))   # 1 MiB of headroom
    try:
        tv._C._set_strict_allocation(True)
        with pytest.raises(torch.OutOfMemoryError):
            torch.empty((4 << 20,), dtype=torch.uint8, device=V)
        assert tv.memory_allocated() == base
        tv._C._set_strict_allocation(False)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            x = torch.empty((1 << 20,), dtype=torch.float32, device=V)    # 4 MiB: served from host memory
            spilled = C.c_int(0)
            assert lib.tvk_last_malloc_spilled(C.byref(spilled)) == gpu.TVK_OK and spilled.value == 1
            assert tv.memory_allocated() >= base + (4 << 20)
            src = torch.arange(1 << 20, dtype=torch.float32)
            x.copy_(src)                               # host -> spilled block
            y = torch.add(x, x, alpha=0.5)             # a kernel reading a spilled block, writing another
            z = y.cpu()
        assert torch.equal(z, src + 0.5 * src)
        del x, y
        tv.synchronize()
        assert tv.memory_allocated() == base
    finally:
        tv._C._set_memory_limit(0, 0)
        tv._C._set_strict_allocation(old_strict)
    # with the limit gone, allocations come from the device again
    w = torch.empty((1 << 20,), dtype=torch.float32, device=V)
    spilled = C.c_int(1)
    assert lib.tvk_last_malloc_spilled(C.byref(spilled)) == gpu.TVK_OK and spilled.value == 0
    del w


def test_pinned_host_memory(gpu):
    import torchvulkan_amd  # noqa: F401

    dev = torch.device(V)
    t = torch.randn((512, 1024))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")   # the device argument of pin_memory is deprecated upstream
        p = t.pin_memory(dev)
        assert p.is_pinned(dev)
        assert not t.is_pinned(dev)
        assert torch.equal(p, t)
        v = p.to(V)
        back = torch.empty_like(p).pin_memory(dev)
    back.copy_(v * 2)
    assert torch.equal(back, t * 2)
    lib = gpu.load()
    pinned = C.c_int(0)
    assert lib.tvk_host_pointer_pinned(C.c_void_p(p.data_ptr() + 4096), C.byref(pinned)) == gpu.TVK_OK and pinned.value == 1
    addr = p.data_ptr()
    del p
    assert lib.tvk_host_pointer_pinned(C.c_void_p(addr), C.byref(pinned)) == gpu.TVK_OK and pinned.value == 0
