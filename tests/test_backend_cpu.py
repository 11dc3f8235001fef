"""CPU checks of the vulkan (PrivateUse1) registration: the extension loads,
the backend is named "vulkan" as in the reference, the device API exists and
reports no device here, and nn.Module gains .vulkan()."""
import torch

import torchvulkan_amd as tv


def test_backend_is_named_vulkan():
    assert torch._C._get_privateuse1_backend_name() == "vulkan"
    assert torch.device("vulkan", 0).type == "vulkan"
    assert torch.vulkan is tv


def test_device_api_surface():
    for name in ("is_available", "device_count", "current_device", "set_device", "synchronize", "empty_cache",
                 "memory_allocated", "max_memory_allocated", "memory_reserved", "mem_get_info",
                 "reset_peak_memory_stats", "memory_stats", "get_device_properties", "get_device_name",
                 "manual_seed", "is_bf16_supported", "current_stream"):
        assert callable(getattr(tv, name)), name


def test_no_device_without_gpu():
    if torch.cuda.is_available():
        return
    assert tv.is_available() is False
    assert tv.device_count() == 0


def test_module_and_tensor_methods():
    assert hasattr(torch.nn.Linear(2, 2), "vulkan")
    assert torch.zeros(1).is_vulkan is False


def test_import_alias():
    import torchvulkan

    assert torchvulkan.is_available is tv.is_available


def test_autocast_registered():
    # the AutocastPrivateUse1 kernels of the reference (src/api/registration.cpp:4-21)
    for op in ("aten::mm", "aten::addmm", "aten::bmm", "aten::baddbmm", "aten::linear", "aten::conv2d",
               "aten::conv3d", "aten::matmul"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op, "AutocastPrivateUse1"), op
    assert torch.amp.is_autocast_available("vulkan")
    assert torch.get_autocast_dtype("vulkan") == torch.float16
