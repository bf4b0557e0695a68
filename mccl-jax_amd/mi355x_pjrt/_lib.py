"""Loader for the in-tree native libraries (ctypes, no torch types at the ABI).

The libraries live in ``mccl-jax_amd/lib`` and are built by
``__graft_entry__.build()`` (``make -C mccl-jax_amd``).  There is no fallback:
a missing library raises, so nothing can silently run a non-HIP path.

torch ships its own libamdhip64.so (same SONAME, libamdhip64.so.7).  When
torch is imported first, the dynamic loader resolves our libraries' HIP
dependency to torch's copy, so tensors, streams and our kernels share one
HIP runtime.  Loading our library first would instead pull in a second
runtime; ``load_kernels`` therefore imports torch before dlopen.
"""

from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_ROOT, "lib")
KERNELS_SO = os.path.join(LIB_DIR, "libmk_kernels.so")
PJRT_SO = os.path.join(LIB_DIR, "libpjrt_mi355x.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/mk_kernels.h
SIGNATURES = {
    "mk_last_error": (ctypes.c_char_p, []),
    "mk_abi_version": (_I, []),
    "mk_device_count": (_I, []),
    "mk_gemm": (_I, [_P, _I, _I, _I64, _I64, _I64, _I64,
                     _P, _I64, _I64, _I64,
                     _P, _I64, _I64, _I64,
                     _P, _I64, _I64, _P, _I]),
    "mk_gemm_blas": (_I, [_P, _I, _I, _I64, _I64, _I64, _I64,
                          _P, _I64, _I64, _I64,
                          _P, _I64, _I64, _I64,
                          _P, _I64, _I64, _F, _F]),
    "mk_sdpa_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64,
                         _P, _I64, _I64, _I64,
                         _P, _I64, _I64, _I64,
                         _P, _I64, _I64, _I64,
                         _P, _I64, _I64, _I64,
                         _F, _I, _P]),
    "mk_row_reduce": (_I, [_P, _I, _I, _I, _I64, _I64, _P, _F, _P]),
    "mk_row_argmax": (_I, [_P, _I, _I, _I64, _I64, _P, _P, _I, _P]),
    "mk_layernorm": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _F, _P]),
    "mk_layernorm_typed": (_I, [_P, _I, _I, _I64, _I64, _P, _P, _P, _F, _P]),
    "mk_gemm_bias_gelu": (_I, [_P, _I, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I, _P,
                               _I64]),
    "mk_gemm_gelu_bwd_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "mk_gemm_gelu_bwd": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _P]),
    "mk_add_layernorm_typed": (_I, [_P, _I, _I, _I64, _I64, _P, _P, _P, _P, _P, _F, _P, _P]),
    "mk_gelu_tanh": (_I, [_P, _I, _I64, _P, _P]),
    "mk_ew_program": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P, _P, _I, _I, _I, _P]),
    "mk_ew_program_multi": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P, _P, _I, _I, _P, _P, _P]),
    "mk_gather_rows": (_I, [_P, _I64, _I64, _P, _I, _I64, _P, _P]),
    "mk_scatter_add_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "mk_scatter_add_rows": (_I, [_P, _I, _I64, _I64, _P, _I, _I64, _P, _P, _P, _P]),
    "mk_scatter_add_rows_noalloc": (_I, [_P, _I, _I64, _I64, _P, _I, _I64, _P, _P, _P]),
    "mk_iota": (_I, [_P, _I, _I, _P, _I, _P]),
    "mk_copy_strided": (_I, [_P, _I, _I, _P, _P, _P, _P]),
    "mk_softmax_rows": (_I, [_P, _I, _I64, _I64, _P, _P]),
    "mk_convert": (_I, [_P, _I, _I, _I64, _P, _P]),
    "mk_fill": (_I, [_P, _I, _I64, ctypes.c_uint64, _P]),
    "mk_gelu_tanh_bwd": (_I, [_P, _I, _I64, _P, _P, _P]),
    "mk_add_rows": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _P]),
    "mk_add_layernorm": (_I, [_P, _I64, _I64, _P, _P, _P, _P, _P, _F, _P, _P]),
    "mk_bias_gelu": (_I, [_P, _I64, _I64, _P, _P, _P, _P]),
    "mk_col_sum_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "mk_col_sum": (_I, [_P, _I, _I64, _I64, _P, _P, _P]),
    "mk_layernorm_bwd_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "mk_layernorm_bwd": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P]),
    "mk_layernorm_bwd_typed": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P]),
    "mk_gelu_tanh_bwd_colsum": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _P, _P]),
    "mk_gemm_splitk_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "mk_gemm_splitk": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P]),
    "mk_gemm_splitk_typed": (_I, [_P, _I, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                  _P, _P, _I]),
    "mk_gemm_blas_splitk_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "mk_gemm_blas_splitk": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P]),
    "mk_adam_update_dev": (_I, [_P, _I64, _I, _P, _P, _I, _P, _P, _P, _P, ctypes.c_double, ctypes.c_double,
                                ctypes.c_double]),
    "mk_softmax_xent": (_I, [_P, _I, _I64, _I64, _P, _I, _P, _F, _P, _P]),
    "mk_softmax_xent_typed": (_I, [_P, _I, _I, _I64, _I64, _P, _I, _P, _F, _P, _P]),
    "mk_softmax_xent_strided": (_I, [_P, _I, _I, _I64, _I64, _P, _I64, _I, _P, _F, _P, _P, _I64]),
    "mk_adam_update": (_I, [_P, _I64, _I, _P, _P, _I, _P, _P, _P] + [ctypes.c_double] * 6),
    "mk_sdpa_bwd_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, _I64, _I64]),
    "mk_sdpa_bwd": (_I, [_P, _I64, _I64, _I64, _I64, _I64]
                    + [_P, _I64, _I64, _I64] * 5 + [_P]
                    + [_P, _I64, _I64, _I64] * 3 + [_F, _I, _P]),
}

_kernels = None


class NativeLibraryMissing(RuntimeError):
    pass


def load_kernels(path: str = KERNELS_SO):
    """dlopen libmk_kernels.so and attach the C signatures."""
    global _kernels
    if _kernels is not None:
        return _kernels
    if not os.path.exists(path):
        raise NativeLibraryMissing(
            f"{path} is not built; run __graft_entry__.build() (make -C mccl-jax_amd)")
    import torch  # noqa: F401  (share torch's HIP runtime, see module docstring)
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _kernels = lib
    return lib


class KernelError(RuntimeError):
    pass


def check(rc: int, what: str):
    if rc != 0:
        msg = _kernels.mk_last_error().decode() if _kernels is not None else ""
        raise KernelError(f"{what} failed (code {rc}): {msg}")
