"""tensors_amd — MI355X (gfx950) backend for tensorforge's training hot path.

The product is native: ``lib/libtf_hip.so`` (HIP kernels + C ABI,
``include/tf_hip.h``) and ``lib/libtensorforge.so`` (the C++20 tensorforge
API on top of it).  This package only loads them; importing it fails when the
HIP library has not been built.
"""
from . import _lib  # noqa: F401  (raises ImportError when libtf_hip.so is missing)
from ._lib import TFError, device_count
from .device import BF16, Context, DeviceArray, bf16_bits_to_f32, f32_to_bf16_bits

__all__ = ["TFError", "device_count", "Context", "DeviceArray", "BF16", "f32_to_bf16_bits", "bf16_bits_to_f32"]
