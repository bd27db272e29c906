"""nerf_amd — MI355X-native (gfx950) backend of the NeRF hot path.

The product is libnerf.so (nerf_amd/csrc/*.hip), a C-ABI shared library that
implements include/nerf.h (the reference's ABI, unchanged) and
include/nerf_ext.h (kernel-level extension entry points).  This package is the
Python host side: ctypes bindings of both headers (_lib), device buffers,
streams and events (device), extension helpers (ext), the build recipe
(build) and the host harness (harness/: dataset loader, PNG, PSNR, the
nerf_bench program).  The library is loaded on
first use and loading fails loudly if it is not built or lacks a symbol; there
is no CPU fallback.
"""
from ._lib import NerfError, load

__all__ = ["NerfError", "load"]
