"""torchvulkan_amd: the vulkan (PrivateUse1) device of torchvulkan on MI355X.

Importing the package registers PyTorch's PrivateUse1 backend under the name
"vulkan" (as the reference does, torchvulkan/__init__.py:168-175): the dense
contraction ops (mm, addmm, bmm, baddbmm, _addmm_activation, addbmm and their
.out forms; convolution and its backward) run hand-written gfx950 kernels from
libtvk_hip.so; every other op runs on the CPU through the boxed fallback, with
the reference's warn-once message (TORCHVULKAN_STRICT=1 makes it an error).

The module also provides the reference's device API subset: is_available,
device_count, current_device, set_device, synchronize, empty_cache,
memory_allocated, max_memory_allocated, memory_reserved, mem_get_info,
reset_peak_memory_stats, memory_stats, get_device_properties, get_device_name,
manual_seed (torchvulkan/__init__.py:32-166).
"""
from __future__ import annotations

import sys
from collections import namedtuple

import torch

from . import _abi  # noqa: F401  (the C ABI binding)
from . import _C

__version__ = "0.1.0"

# ---------------------------------------------------------------------------
# device API (torchvulkan/__init__.py:32-166)
# ---------------------------------------------------------------------------


def _device_index(dev) -> int:
    if isinstance(dev, int):
        return dev
    index = None if dev is None else torch.device(dev).index
    return current_device() if index is None else index


def is_available() -> bool:
    return _C.is_available()


def device_count() -> int:
    return _C.device_count()


def current_device() -> int:
    return _C.current_device()


def set_device(device) -> None:
    index = _device_index(device)
    if index >= 0:
        _C.set_device(index)


def is_initialized() -> bool:
    return True


def _lazy_init() -> None:
    return None


def synchronize(device=None) -> None:
    """Waits for every kernel and copy queued on the device's stream."""
    _C.synchronize(_device_index(device))


def current_stream(device=None) -> torch.Stream:
    """The device's one stream (every kernel and copy of the backend is queued on it)."""
    return torch.accelerator.current_stream(torch.device("vulkan", _device_index(device)))


def empty_cache() -> None:
    for d in range(device_count()):
        _C.empty_cache(d)


def memory_allocated(device=None) -> int:
    return _C._memory_allocated(_device_index(device))


def max_memory_allocated(device=None) -> int:
    return _C._max_memory_allocated(_device_index(device))


def memory_reserved(device=None) -> int:
    return _C._memory_reserved(_device_index(device))


def mem_get_info(device=None) -> tuple:
    return _C._mem_get_info(_device_index(device))


def reset_peak_memory_stats(device=None) -> None:
    _C._reset_peak_memory_stats(_device_index(device))


def memory_stats(device=None) -> dict:
    index = _device_index(device)
    allocated = _C._memory_allocated(index)
    peak = _C._max_memory_allocated(index)
    return {
        "active_bytes.all.current": allocated,
        "active_bytes.all.peak": peak,
        "allocated_bytes.all.current": allocated,
        "allocated_bytes.all.peak": peak,
        "reserved_bytes.all.current": _C._memory_reserved(index),
    }


DeviceProperties = namedtuple("DeviceProperties", ["name", "arch", "total_memory", "compute_units", "clock_khz",
                                                   "subgroup_size", "has_fp64", "has_fp16", "has_bf16"])


def get_device_properties(device=None) -> DeviceProperties:
    return DeviceProperties(**_C._device_properties(_device_index(device)))


def get_device_name(device=None) -> str:
    return get_device_properties(device).name


def get_amp_supported_dtype() -> list:
    return [torch.float16, torch.bfloat16]


def is_bf16_supported() -> bool:
    return True


def manual_seed(seed) -> None:
    """Random numbers for vulkan tensors are drawn on the host (the CPU fallback
    runs the random ops), so seeding seeds the host generator. torch.manual_seed
    calls manual_seed_all of this module in turn, so neither calls back into it."""
    torch.default_generator.manual_seed(int(seed))


def manual_seed_all(seed) -> None:
    torch.default_generator.manual_seed(int(seed))


def _is_in_bad_fork() -> bool:
    """torch.manual_seed asks every device module this before seeding it; the
    host generator this device draws from has no fork state of its own."""
    return False


def seed() -> None:
    torch.seed()


def initial_seed() -> int:
    return torch.initial_seed()


# ---------------------------------------------------------------------------
# registration (torchvulkan/__init__.py:168-175)
# ---------------------------------------------------------------------------

torch.utils.rename_privateuse1_backend("vulkan")
torch._register_device_module("vulkan", sys.modules[__name__])


def _tensor_to_vulkan(self, device=None, non_blocking=False, **kwargs) -> torch.Tensor:
    if isinstance(device, (str, torch.device)) and torch.device(device).type != "vulkan":
        raise RuntimeError("Invalid device, must be vulkan device")
    return self.to(torch.device("vulkan", _device_index(device)), non_blocking=non_blocking, **kwargs)


# torch's own (legacy) Vulkan backend owns these names; the reference overrides them the same way
torch.Tensor.vulkan = _tensor_to_vulkan
torch.Tensor.is_vulkan = property(lambda self: self.device.type == "vulkan")
torch.utils.generate_methods_for_privateuse1_backend(for_tensor=False)
