"""vkflame_amd — MI355X (gfx950) quantized-linear hot path of vkflame.

The product is the native library ``libvkflame_amd.so`` (C ABI in
``include/vkflame_amd.h``, plus hipBLAS / hipBLASLt entry points) and the
``libvkflame_preload.so`` hipLaunchKernel interposer.  This package builds
them (``vkflame_amd.build``) and exposes a ctypes binding (``vkflame_amd.ops``
wraps it for torch device tensors).
"""
from ._lib import (LIB_PATH, PRELOAD_PATH, VkflameError, check, lib)  # noqa: F401

__all__ = ["lib", "check", "VkflameError", "LIB_PATH", "PRELOAD_PATH"]
