"""MI355X-native DeviceBackend for Pulsatrix's causal-LM forward + AttnLRP path.

The product is native: gfx950 HIP kernels (libpxk_gfx950.so, include/pxk.h) and the C++17 host
framework over them (libpulsatrix_amd.so, include/pulsatrix_amd.h). `native` holds their ctypes
bindings; `models` a thin Python handle over the host framework's C ABI.
"""
from . import native  # noqa: F401
