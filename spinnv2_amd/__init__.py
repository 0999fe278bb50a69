"""MI355X-native backend for the SPINNV2 inference runtime.

The product is the C-ABI library `lib/libspkv2_mi355x.so` (runtime + HIP
kernels for gfx950, headers in include/).  This package holds its sources
(`csrc/`), the build driver (`build.py`), a ctypes binding (`runtime.py`) and
the SPK package toolchain used to produce models for it (`spk/`).
"""

from .runtime import LIB_PATH, DeviceBuffer, Model, load_library  # noqa: F401

__all__ = ["LIB_PATH", "DeviceBuffer", "Model", "load_library"]
