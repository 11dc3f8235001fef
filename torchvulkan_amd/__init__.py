"""torchvulkan_amd: MI355X (gfx950) dense-contraction path of torchvulkan.

The C ABI lives in libtvk_hip.so (include/tvk_hip.h); `_abi` binds it.
"""
from . import _abi  # noqa: F401

__version__ = "0.1.0"
