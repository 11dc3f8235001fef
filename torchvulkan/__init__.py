"""Import alias: `import torchvulkan` loads torchvulkan_amd, the MI355X build of
the vulkan device, so code written against the reference keeps its imports."""
import sys as _sys

import torchvulkan_amd as _impl
from torchvulkan_amd import *  # noqa: F401,F403
from torchvulkan_amd import (_device_index, current_stream, device_count, empty_cache, get_device_name,  # noqa: F401
                             get_device_properties, is_available, manual_seed, max_memory_allocated, mem_get_info,
                             memory_allocated, memory_reserved, memory_stats, reset_peak_memory_stats, synchronize)

__version__ = _impl.__version__
