"""naylis_amd — the Mixture-of-Memory read of OpenRootdev/Naylis, MI355X-native.

Layout:
  csrc/          HIP kernels for gfx950 and the C ABI (include/naylis_mom.h)
  _lib.py        ctypes loader of the in-tree libnaylis_mom.so
  mom_kernels/   drop-in for the reference's ``mom_kernels`` package
  layer.py       ``MoMLayer`` with the reference's parameter names
  build.py       hipcc build of the library
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"
