"""ctypes bridge to oracle/c/oracle.c (oracle; test infrastructure only).

The C restatement is built by oracle/Makefile into oracle/_build/liboracle.so
(``__graft_entry__.build()`` runs it); load() builds it on first use if the
library is missing and a C compiler is available.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int64


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "_build/liboracle.so"], check=True)
    return _LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.oracle_scatter_add_f32.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.oracle_scatter_add_bf16.argtypes = [_P, _I, _I, _P, _I, _P]
    lib.oracle_argmax_rows_bf16.argtypes = [_P, _I, _I, ctypes.c_int, _P, _P]
    lib.oracle_row_sum_bf16.argtypes = [_P, _I, _I, _P]
    lib.oracle_gather_rows.argtypes = [_P, _I, _I, _P, _I, _P]
    for f in (lib.oracle_scatter_add_f32, lib.oracle_scatter_add_bf16,
              lib.oracle_argmax_rows_bf16, lib.oracle_row_sum_bf16, lib.oracle_gather_rows):
        f.restype = None
    _lib = lib
    return lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def scatter_add_f32(table, ids, updates) -> np.ndarray:
    out = np.array(table, dtype=np.float32, order="C", copy=True)
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    upd = np.ascontiguousarray(updates, dtype=np.float32).reshape(ids.size, out.shape[1])
    load().oracle_scatter_add_f32(_ptr(out), out.shape[0], out.shape[1], _ptr(ids), ids.size, _ptr(upd))
    return out


def scatter_add_bf16(table_bits, ids, updates_bits) -> np.ndarray:
    out = np.array(table_bits, dtype=np.uint16, order="C", copy=True)
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    upd = np.ascontiguousarray(updates_bits, dtype=np.uint16).reshape(ids.size, out.shape[1])
    load().oracle_scatter_add_bf16(_ptr(out), out.shape[0], out.shape[1], _ptr(ids), ids.size, _ptr(upd))
    return out


def argmax_rows_bf16(x_bits, is_min=False):
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, cols = x.shape
    idx = np.empty(rows, dtype=np.int64)
    vals = np.empty(rows, dtype=np.uint16)
    load().oracle_argmax_rows_bf16(_ptr(x), rows, cols, int(is_min), _ptr(idx), _ptr(vals))
    return idx, vals


def row_sum_bf16(x_bits) -> np.ndarray:
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    out = np.empty(x.shape[0], dtype=np.float64)
    load().oracle_row_sum_bf16(_ptr(x), x.shape[0], x.shape[1], _ptr(out))
    return out


def gather_rows(table, ids) -> np.ndarray:
    t = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    row_bytes = t.strides[0]
    out = np.empty((ids.size,) + t.shape[1:], dtype=t.dtype)
    load().oracle_gather_rows(_ptr(t), t.shape[0], row_bytes, _ptr(ids), ids.size, _ptr(out))
    return out
