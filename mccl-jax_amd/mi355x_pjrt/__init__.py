"""Host side of the MI355X PJRT plugin (Python part).

  _lib      locate / dlopen the in-tree native libraries (no fallback)
  kernels   torch-tensor wrappers over the C-ABI of include/mk_kernels.h
  pjrt      ctypes driver of libpjrt_mi355x.so through the PJRT C API
            (the counterpart of the reference's pjrt_e2e harness)
  modules   StableHLO text of the benchmark config functions
"""

import os as _os

PKG_ROOT = _os.path.dirname(_os.path.dirname(_os.path.abspath(__file__)))
PJRT_LIBRARY = _os.path.join(PKG_ROOT, "lib", "libpjrt_mi355x.so")
KERNELS_LIBRARY = _os.path.join(PKG_ROOT, "lib", "libmk_kernels.so")
