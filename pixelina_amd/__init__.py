"""pixelina_amd: MI355X (gfx950) HIP backend for Pixelina's quantized linear
layer.  The product is libpixhip.so (include/pixhip.h); this package holds its
sources (csrc/, host/), the build script and a ctypes handle for callers that
drive it from Python."""
from ._lib import Q5_K, Q6_K, Q8_0, PixhipError, load  # noqa: F401
from .session import DeviceBuffer, Session  # noqa: F401

__all__ = ["Q5_K", "Q6_K", "Q8_0", "PixhipError", "load", "Session", "DeviceBuffer"]
