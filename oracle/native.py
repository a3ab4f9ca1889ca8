"""ctypes bindings of the compiled CPU checkers -- TEST INFRASTRUCTURE ONLY.

* ``oracle/_build/libcl3_oracle.so`` -- the C restatement
  (``oracle/csrc/cl3_oracle.c``), single-threaded and OpenMP geometric matmul.
* ``oracle/_ref/libmjolnir_cpu.so`` -- the reference's own CPU library,
  compiled from ``/root/reference/mjolnir/src/cpu/*.c`` by ``oracle/Makefile``;
  entry point ``cl3_geom_matmul_flat`` (``mjolnir/src/cpu/batch_ops.c:165-172``,
  declared ``mjolnir/include/cl3_ops.h:210``, bound by the reference at
  ``rune/bindings/mjolnir_ffi.py:208-209,442-460``).

Both are optional at import; the loaders return ``None`` when a library is
not built.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# YGG_ORACLE_LIB names another build of the C restatement (e.g. one with sanitizers)
ORACLE_LIB = os.environ.get("YGG_ORACLE_LIB") or os.path.join(HERE, "_build", "libcl3_oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libmjolnir_cpu.so")

_F = ctypes.POINTER(ctypes.c_float)
_SZ = ctypes.c_size_t

_cache: dict[str, ctypes.CDLL | None] = {}


def _load(path: str):
    if path not in _cache:
        _cache[path] = ctypes.CDLL(path) if os.path.exists(path) else None
    return _cache[path]


def oracle_lib():
    lib = _load(ORACLE_LIB)
    if lib is not None and not hasattr(lib, "_typed"):
        lib.oracle_geom_matmul.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ]
        lib.oracle_geom_matmul_omp.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ, ctypes.c_int]
        lib.oracle_geom_prod.argtypes = [_F, _F, _F, _SZ]
        lib.oracle_tables.argtypes = [ctypes.POINTER(ctypes.c_int32), _F]
        lib._typed = True
    return lib


def ref_lib():
    lib = _load(REF_LIB)
    if lib is not None and not hasattr(lib, "_typed"):
        lib.cl3_geom_matmul_flat.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ]
        lib.cl3_geom_matmul_flat.restype = None
        lib.cl3_batch_gp_flat.argtypes = [_F, _F, _F, _SZ]
        lib.cl3_batch_gp_flat.restype = None
        lib._typed = True
    return lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _prep(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    assert a.ndim == 3 and b.ndim == 3 and a.shape[1] == b.shape[0] and a.shape[2] == b.shape[2] == 8
    out = np.empty((a.shape[0], b.shape[1], 8), dtype=np.float32)
    return a, b, out


def c_geom_matmul(a, b, threads: int = 1):
    """C restatement; ``threads > 1`` uses the OpenMP variant (same bits)."""
    lib = oracle_lib()
    if lib is None:
        raise FileNotFoundError(ORACLE_LIB)
    a, b, out = _prep(a, b)
    M, K, N = a.shape[0], a.shape[1], b.shape[1]
    if threads > 1:
        lib.oracle_geom_matmul_omp(_p(a), _p(b), _p(out), M, K, N, threads)
    else:
        lib.oracle_geom_matmul(_p(a), _p(b), _p(out), M, K, N)
    return out


def c_geom_prod(a, b):
    """C restatement of the element-wise geometric product over rows of 8."""
    lib = oracle_lib()
    if lib is None:
        raise FileNotFoundError(ORACLE_LIB)
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1, 8)
    b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1, 8)
    out = np.empty_like(a)
    lib.oracle_geom_prod(_p(a), _p(b), _p(out), a.shape[0])
    return out


def ref_geom_matmul(a, b):
    """The reference's compiled ``cl3_geom_matmul_flat``."""
    lib = ref_lib()
    if lib is None:
        raise FileNotFoundError(REF_LIB)
    a, b, out = _prep(a, b)
    lib.cl3_geom_matmul_flat(_p(a), _p(b), _p(out), a.shape[0], a.shape[1], b.shape[1])
    return out


def ref_geom_prod(a, b):
    lib = ref_lib()
    if lib is None:
        raise FileNotFoundError(REF_LIB)
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1, 8)
    b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1, 8)
    out = np.empty_like(a)
    lib.cl3_batch_gp_flat(_p(a), _p(b), _p(out), a.shape[0])
    return out


def c_tables():
    lib = oracle_lib()
    idx = np.zeros(64, dtype=np.int32)
    sign = np.zeros(64, dtype=np.float32)
    lib.oracle_tables(idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), _p(sign))
    return idx.reshape(8, 8), sign.reshape(8, 8)
