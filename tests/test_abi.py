"""The C-ABI libraries load and export exactly what include/*.h declares
(no GPU needed: nothing here launches a kernel)."""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "mccl-jax_amd", "lib")


def _declared(header: str, prefix: str):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w*)\s*\(", text)))


def _exported(so: str):
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True)
    return sorted(line.split()[-1] for line in out.stdout.splitlines() if " T " in line)


def test_kernel_library_exports_every_declared_symbol():
    so = os.path.join(LIB, "libmk_kernels.so")
    assert os.path.exists(so), "build first: __graft_entry__.build()"
    declared = _declared("mk_kernels.h", "mk_")
    assert len(declared) >= 18
    exported = _exported(so)
    assert exported == declared, (set(declared) ^ set(exported))


def test_kernel_library_loads_and_answers_without_gpu():
    import torch  # noqa: F401  (same HIP runtime as on the GPU box)
    from mi355x_pjrt import _lib

    lib = _lib.load_kernels()
    assert lib.mk_abi_version() == 1
    assert lib.mk_device_count() >= 0
    # argument validation happens before any launch
    rc = lib.mk_gemm(None, 11, 11, 1, 4, 4, 4, None, 0, 4, 1, None, 0, 4, 1, None, 0, 4, None, 7)
    assert rc == 1 and b"epilogue" in lib.mk_last_error()
    rc = lib.mk_sdpa_fwd(None, 1, 1, 8, 8, 96, *([None, 0, 0, 0] * 4), ctypes.c_float(1.0), 1, None)
    assert rc == 2 and b"head_dim" in lib.mk_last_error()
    assert lib.mk_scatter_add_workspace_bytes(50257, 65536) > 4 * 65536 * 4


def test_pjrt_plugin_exports_only_GetPjrtApi():
    so = os.path.join(LIB, "libpjrt_mi355x.so")
    if not os.path.exists(so):
        pytest.skip("PJRT plugin not built yet")
    assert _declared("pjrt_mi355x.h", "GetPjrtApi") == ["GetPjrtApi"]
    assert _exported(so) == ["GetPjrtApi"]
