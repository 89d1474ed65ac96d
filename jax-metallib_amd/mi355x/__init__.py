"""Python side of the MI355X PJRT plugin.

  mi355x._lib   ctypes loader of the kernel C-ABI (include/mk_kernels.h); it
                raises when the built library is missing -- there is no CPU
                fallback anywhere in this package.
  mi355x.ops    thin torch-tensor wrappers over the C-ABI (device memory and
                streams come from torch; the kernels are the product).
"""

from . import _lib  # noqa: F401
