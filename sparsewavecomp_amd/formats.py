"""Sparse matrix files of the reference's benchmark harness, read and written
by the native code of libsparsewave_amd.so (csrc/sw_io.cpp).

Mirrors benchmark/benchmark_utils.py:56-379 -- ``read_matrix_market``,
``write_csr_binary``, ``write_coo_binary``, ``convert_to_bsr``,
``write_bsr_binary`` return and take dicts with the same keys (arrays are
numpy arrays instead of lists) and raise ``ValueError`` where it does -- plus
the readers of benchmark/SparseBenchmarkUtils.cpp:83-185
(``read_csr_binary``, ``read_coo_binary``, ``read_bsr_binary``) and the
harness's deterministic operands (``benchmark_vector``, ``benchmark_rhs``).
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

from . import load_library

CSR_BINARY_MAGIC = b"SWCSR001"
COO_BINARY_MAGIC = b"SWCOO001"
BSR_BINARY_MAGIC = b"SWBSR001"

_I32P = ctypes.POINTER(ctypes.c_int32)
_F64P = ctypes.POINTER(ctypes.c_double)


class _CHostMatrix(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64), ("columns", ctypes.c_int64),
        ("nnz", ctypes.c_int64), ("row_offsets", _I32P),
        ("row_indices", _I32P), ("column_indices", _I32P),
        ("values", _F64P), ("has_row_offsets", ctypes.c_int32),
        ("field", ctypes.c_char * 16), ("symmetry", ctypes.c_char * 16),
        ("min_row_nnz", ctypes.c_int64), ("max_row_nnz", ctypes.c_int64),
        ("mean_row_nnz", ctypes.c_double),
    ]


class _CHostBsr(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64), ("columns", ctypes.c_int64),
        ("nnzb", ctypes.c_int64), ("block_size", ctypes.c_int64),
        ("original_rows", ctypes.c_int64),
        ("original_columns", ctypes.c_int64), ("nnz", ctypes.c_int64),
        ("block_row_offsets", _I32P), ("block_column_indices", _I32P),
        ("block_values", _F64P), ("input_row_indices", _I32P),
        ("input_column_indices", _I32P), ("input_values", _F64P),
        ("block_density", ctypes.c_double),
        ("internal_zero_fraction", ctypes.c_double),
        ("storage_overhead", ctypes.c_double),
    ]


_MP = ctypes.POINTER(_CHostMatrix)
_BP = ctypes.POINTER(_CHostBsr)
_configured = None


def _lib():
    global _configured
    lib = load_library()
    if _configured is lib:
        return lib
    C, I = ctypes.c_char_p, ctypes.c_int
    sig = {
        "sw_host_matrix_free": (None, [_MP]),
        "sw_host_bsr_free": (None, [_BP]),
        "sw_matrix_market_read": (I, [C, ctypes.POINTER(_MP)]),
        "sw_csr_binary_write": (I, [C, _MP]),
        "sw_coo_binary_write": (I, [C, _MP]),
        "sw_csr_binary_read": (I, [C, ctypes.POINTER(_MP)]),
        "sw_coo_binary_read": (I, [C, ctypes.POINTER(_MP)]),
        "sw_convert_to_bsr": (I, [_MP, ctypes.c_int64, ctypes.POINTER(_BP)]),
        "sw_bsr_binary_write": (I, [C, _BP]),
        "sw_bsr_binary_read": (I, [C, ctypes.POINTER(_BP)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _configured = lib
    return lib


def _ok(rc):
    if rc != 0:
        raise ValueError(_lib().sw_last_error().decode())


def _copy(ptr, n, dtype):
    if n == 0 or not ptr:
        return np.zeros(0, dtype)
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)


def _matrix_dict(m: _CHostMatrix, path=None) -> dict:
    rows, nnz = m.rows, m.nnz
    d = {
        "rows": rows, "columns": m.columns, "nnz": nnz,
        "field": m.field.decode(), "symmetry": m.symmetry.decode(),
        "min_row_nnz": m.min_row_nnz, "max_row_nnz": m.max_row_nnz,
        "mean_row_nnz": m.mean_row_nnz,
        "row_offsets": (_copy(m.row_offsets, rows + 1, np.int32)
                        if m.has_row_offsets else None),
        "row_indices": _copy(m.row_indices, nnz, np.int32),
        "column_indices": _copy(m.column_indices, nnz, np.int32),
        "values": _copy(m.values, nnz, np.float64),
    }
    if path is not None:
        d["path"] = pathlib.Path(path)
        d["name"] = pathlib.Path(path).stem
    return d


def _bsr_dict(b: _CHostBsr) -> dict:
    bb = b.block_size * b.block_size
    return {
        "rows": b.rows, "columns": b.columns,
        "original_rows": b.original_rows,
        "original_columns": b.original_columns, "nnz": b.nnz,
        "block_size": b.block_size, "nnzb": b.nnzb,
        "block_row_offsets": _copy(b.block_row_offsets,
                                   b.rows // b.block_size + 1, np.int32),
        "block_column_indices": _copy(b.block_column_indices, b.nnzb,
                                      np.int32),
        "block_values": _copy(b.block_values, b.nnzb * bb, np.float64),
        "input_row_indices": _copy(b.input_row_indices, b.nnz, np.int32),
        "input_column_indices": _copy(b.input_column_indices, b.nnz,
                                      np.int32),
        "input_values": _copy(b.input_values, b.nnz, np.float64),
        "block_density": b.block_density,
        "internal_zero_fraction": b.internal_zero_fraction,
        "storage_overhead": b.storage_overhead,
    }


def _arr(a, dtype, n, name):
    a = np.ascontiguousarray(np.asarray(a if a is not None else [], dtype))
    if a.size != n:
        raise ValueError(f"{name} has {a.size} entries, expected {n}")
    return a


def _c_matrix(matrix: dict, need_offsets: bool):
    """A _CHostMatrix view of a matrix dict (arrays kept alive in `keep`)."""
    rows, nnz = int(matrix["rows"]), int(matrix["nnz"])
    keep = []
    m = _CHostMatrix(rows=rows, columns=int(matrix["columns"]), nnz=nnz)
    for key, dtype, n in (("row_indices", np.int32, nnz),
                          ("column_indices", np.int32, nnz),
                          ("values", np.float64, nnz)):
        a = _arr(matrix.get(key), dtype, n, key)
        keep.append(a)
        setattr(m, key, a.ctypes.data_as(_F64P if dtype is np.float64
                                         else _I32P))
    ro = matrix.get("row_offsets")
    if ro is not None:
        a = _arr(ro, np.int32, rows + 1, "row_offsets")
        keep.append(a)
        m.row_offsets = a.ctypes.data_as(_I32P)
        m.has_row_offsets = 1
    elif need_offsets:
        raise ValueError("a CSR file needs row_offsets")
    return m, keep


def read_matrix_market(path) -> dict:
    """benchmark/benchmark_utils.py:56-177."""
    out = _MP()
    _ok(_lib().sw_matrix_market_read(str(path).encode(), ctypes.byref(out)))
    try:
        return _matrix_dict(out.contents, path)
    finally:
        _lib().sw_host_matrix_free(out)


def write_csr_binary(path, matrix: dict) -> None:
    """benchmark/benchmark_utils.py:192-211."""
    m, _keep = _c_matrix(matrix, need_offsets=True)
    _ok(_lib().sw_csr_binary_write(str(path).encode(), ctypes.byref(m)))


def write_coo_binary(path, matrix: dict) -> None:
    """benchmark/benchmark_utils.py:214-237."""
    m, _keep = _c_matrix(matrix, need_offsets=False)
    _ok(_lib().sw_coo_binary_write(str(path).encode(), ctypes.byref(m)))


def read_csr_binary(path) -> dict:
    """benchmark/SparseBenchmarkUtils.cpp:83-121 (plus structure checks)."""
    out = _MP()
    _ok(_lib().sw_csr_binary_read(str(path).encode(), ctypes.byref(out)))
    try:
        return _matrix_dict(out.contents)
    finally:
        _lib().sw_host_matrix_free(out)


def read_coo_binary(path) -> dict:
    """benchmark/SparseBenchmarkUtils.cpp:123-141 (plus bounds checks);
    ``row_offsets`` is None unless the entries are stored by (row, column)."""
    out = _MP()
    _ok(_lib().sw_coo_binary_read(str(path).encode(), ctypes.byref(out)))
    try:
        return _matrix_dict(out.contents)
    finally:
        _lib().sw_host_matrix_free(out)


def convert_to_bsr(matrix: dict, block_size: int) -> dict:
    """benchmark/benchmark_utils.py:240-312."""
    m, _keep = _c_matrix(matrix, need_offsets=False)
    out = _BP()
    _ok(_lib().sw_convert_to_bsr(ctypes.byref(m), int(block_size),
                                 ctypes.byref(out)))
    try:
        return _bsr_dict(out.contents)
    finally:
        _lib().sw_host_bsr_free(out)


def write_bsr_binary(path, bsr: dict) -> None:
    """benchmark/benchmark_utils.py:315-379."""
    b = _CHostBsr()
    for k in ("rows", "columns", "nnzb", "block_size", "original_rows",
              "original_columns", "nnz"):
        setattr(b, k, int(bsr[k]))
    if b.block_size <= 0 or b.rows % b.block_size:
        raise ValueError("BSR rows must be a multiple of a positive block size")
    keep = []
    bb = b.block_size * b.block_size
    for key, dtype, n in (
            ("block_row_offsets", np.int32, b.rows // b.block_size + 1),
            ("block_column_indices", np.int32, b.nnzb),
            ("block_values", np.float64, b.nnzb * bb),
            ("input_row_indices", np.int32, b.nnz),
            ("input_column_indices", np.int32, b.nnz),
            ("input_values", np.float64, b.nnz)):
        a = _arr(bsr[key], dtype, n, key)
        keep.append(a)
        setattr(b, key, a.ctypes.data_as(_F64P if dtype is np.float64
                                         else _I32P))
    _ok(_lib().sw_bsr_binary_write(str(path).encode(), ctypes.byref(b)))


def read_bsr_binary(path) -> dict:
    """benchmark/SparseBenchmarkUtils.cpp:143-185 (plus structure checks)."""
    out = _BP()
    _ok(_lib().sw_bsr_binary_read(str(path).encode(), ctypes.byref(out)))
    try:
        return _bsr_dict(out.contents)
    finally:
        _lib().sw_host_bsr_free(out)


def read_matrix(path) -> dict:
    """Any of the harness's files, chosen by the binary magic (Matrix Market
    otherwise)."""
    with open(path, "rb") as f:
        magic = f.read(8)
    if magic == CSR_BINARY_MAGIC:
        return read_csr_binary(path)
    if magic == COO_BINARY_MAGIC:
        return read_coo_binary(path)
    return read_matrix_market(path)


def benchmark_vector(columns: int) -> np.ndarray:
    """The harness's SpMV vector: all ones
    (benchmark/SparseBenchmarkUtils.cpp:187-193)."""
    return np.ones(columns, np.float32)


def benchmark_rhs(rows: int, k: int) -> np.ndarray:
    """The harness's SpMM / BSR right-hand side,
    1 + ((row + column) mod 7) / 8 (SparseBenchmarkUtils.cpp:270-273)."""
    r = np.arange(rows, dtype=np.int64)[:, None]
    c = np.arange(k, dtype=np.int64)[None, :]
    return (1.0 + ((r + c) % 7).astype(np.float32) * 0.125).astype(
        np.float32)
