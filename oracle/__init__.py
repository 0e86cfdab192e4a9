"""ctypes bindings of the CPU oracle (oracle/sw_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, always as the checker or the timed CPU
baseline, never by the product path.  Each wrapper names the reference
function it restates in sw_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsw_oracle.so")
_lib = None

SDDMM_MUL, SDDMM_AFFINE, SDDMM_DOT = 0, 1, 2
REDUCE_SUM, REDUCE_MAX = 0, 1
MAP_EXP_SUB, MAP_DIV, MAP_SUB, MAP_MUL = 0, 1, 2, 3


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc only, a few seconds)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def _declare(l):
    l.oracle_spmv_csr_f32.argtypes = [_I64, _P, _P, _P, _P, _P]
    l.oracle_spmv_csr_f32_mt.argtypes = [_I64, _P, _P, _P, _P, _P]
    l.oracle_num_threads.restype = ctypes.c_int
    l.oracle_spmv_abs_bound.argtypes = [_I64, _P, _P, _P, _P, _P]
    l.oracle_spmv_coo_f32.argtypes = [_I64, _I64, _P, _P, _P, _P, _P, _P]
    l.oracle_spmm_csr_f32.argtypes = [_I64, _I64, _P, _P, _P, _P, _P]
    l.oracle_spmm_abs_bound.argtypes = [_I64, _I64, _P, _P, _P, _P, _P]
    l.oracle_bsr_spmm_f32.argtypes = [_I64, _I64, _I64, _P, _P, _P, _P, _P]
    l.oracle_bsr_abs_bound.argtypes = [_I64, _I64, _I64, _P, _P, _P, _P, _P]
    l.oracle_sddmm_csr_f32.argtypes = [_I64, _I64, _I64, _P, _P, _P, _P, _P,
                                       _P, ctypes.c_int, ctypes.c_float,
                                       ctypes.c_float]
    l.oracle_csr_row_reduce_f32.argtypes = [_I64, _P, _P, _P, ctypes.c_int]
    l.oracle_csr_rowwise_map_f32.argtypes = [_I64, _P, _P, _P, _P,
                                             ctypes.c_int]
    l.oracle_sparse_attention_f32.argtypes = [_I64, _I64, _I64, _I64, _P, _P,
                                              _P, _P, _P, _P, _P, _P, _P, _P,
                                              ctypes.c_float, ctypes.c_float]
    l.oracle_sparse_attention_bf16.argtypes = [_I64, _I64, _I64, _I64, _P, _P,
                                               _P, _P, _P, _P, _P, _P, _P, _P,
                                               ctypes.c_float, ctypes.c_float]
    l.oracle_round_bf16.argtypes = [_I64, _P, _P]
    l.oracle_bf16_to_f32.argtypes = [_I64, _P, _P]
    l.oracle_csr_row_at_position.argtypes = [_I64, _P, _I64]
    l.oracle_csr_row_at_position.restype = _I64
    l.oracle_csr_rows_at_positions.argtypes = [_I64, _P, _I64, _P, _P]
    l.oracle_position_space.argtypes = [_I64, _I64, _I64, _I64,
                                        ctypes.POINTER(_I64),
                                        ctypes.POINTER(_I64)]
    l.oracle_wave_segmented_scan.argtypes = [ctypes.c_int, _P, _P, _P, _P, _P]
    l.oracle_spmv_wave_position_f32.argtypes = [_I64, _I64, _P, _P, _P, _P,
                                                _P, _I64, ctypes.c_int]


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def spmv(ro, col, val, x, threads: bool = False):
    """SparseBenchmarkUtils.cpp:211-229 / SparseWaveToGPU.cpp:216-274."""
    ro, col, val, x = (_c(ro, np.int32), _c(col, np.int32),
                       _c(val, np.float32), _c(x, np.float32))
    rows = ro.size - 1
    y = np.empty(rows, np.float32)
    fn = lib().oracle_spmv_csr_f32_mt if threads else lib().oracle_spmv_csr_f32
    fn(rows, _ptr(ro), _ptr(col), _ptr(val), _ptr(x), _ptr(y))
    return y


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def spmv_abs_bound(ro, col, val, x):
    ro, col, val, x = (_c(ro, np.int32), _c(col, np.int32),
                       _c(val, np.float32), _c(x, np.float32))
    rows = ro.size - 1
    b = np.empty(rows, np.float64)
    lib().oracle_spmv_abs_bound(rows, _ptr(ro), _ptr(col), _ptr(val), _ptr(x),
                                _ptr(b))
    return b


def spmv_coo(rows, ri, ci, val, x):
    """COO SpMV in storage order; returns (y, per-row bound sum |val*x|).
    SparseWaveToGPU.cpp:154-214 / SparseBenchmarkUtils.cpp:231-251."""
    ri, ci, val, x = (_c(ri, np.int32), _c(ci, np.int32),
                      _c(val, np.float32), _c(x, np.float32))
    y = np.empty(rows, np.float32)
    b = np.empty(rows, np.float64)
    lib().oracle_spmv_coo_f32(rows, ri.size, _ptr(ri), _ptr(ci), _ptr(val),
                              _ptr(x), _ptr(y), _ptr(b))
    return y, b


def spmm(ro, col, val, rhs):
    """SparseBenchmarkUtils.cpp:277-288 / SparseWaveToGPU.cpp:489-558."""
    ro, col, val = _c(ro, np.int32), _c(col, np.int32), _c(val, np.float32)
    rhs = _c(rhs, np.float32)
    rows, k = ro.size - 1, rhs.shape[1]
    out = np.empty((rows, k), np.float32)
    lib().oracle_spmm_csr_f32(rows, k, _ptr(ro), _ptr(col), _ptr(val),
                              _ptr(rhs), _ptr(out))
    return out


def spmm_abs_bound(ro, col, val, rhs):
    ro, col, val = _c(ro, np.int32), _c(col, np.int32), _c(val, np.float32)
    rhs = _c(rhs, np.float32)
    rows, k = ro.size - 1, rhs.shape[1]
    out = np.empty((rows, k), np.float64)
    lib().oracle_spmm_abs_bound(rows, k, _ptr(ro), _ptr(col), _ptr(val),
                                _ptr(rhs), _ptr(out))
    return out


def bsr_spmm(bro, bcol, bval, rhs, block_size):
    """SparseWaveToGPU.cpp:560-665 (blocks row-major [nnzb][b][b])."""
    bro, bcol = _c(bro, np.int32), _c(bcol, np.int32)
    bval, rhs = _c(bval, np.float32), _c(rhs, np.float32)
    rows = (bro.size - 1) * block_size
    k = rhs.shape[1]
    out = np.empty((rows, k), np.float32)
    lib().oracle_bsr_spmm_f32(rows, k, block_size, _ptr(bro), _ptr(bcol),
                              _ptr(bval), _ptr(rhs), _ptr(out))
    return out


def bsr_abs_bound(bro, bcol, bval, rhs, block_size):
    bro, bcol = _c(bro, np.int32), _c(bcol, np.int32)
    bval, rhs = _c(bval, np.float32), _c(rhs, np.float32)
    rows = (bro.size - 1) * block_size
    k = rhs.shape[1]
    out = np.empty((rows, k), np.float64)
    lib().oracle_bsr_abs_bound(rows, k, block_size, _ptr(bro), _ptr(bcol),
                               _ptr(bval), _ptr(rhs), _ptr(out))
    return out


def sddmm(ro, col, val, lhs, rhs, kind=SDDMM_MUL, alpha=1.0, beta=0.0):
    """SparseWaveToGPU.cpp:667-750; affine form from
    SparseAttentionToSparseWave.cpp:270-283."""
    ro, col, val = _c(ro, np.int32), _c(col, np.int32), _c(val, np.float32)
    lhs, rhs = _c(lhs, np.float32), _c(rhs, np.float32)
    rows, kdim = lhs.shape
    cols = rhs.shape[1]
    out = np.empty(col.size, np.float32)
    lib().oracle_sddmm_csr_f32(rows, kdim, cols, _ptr(ro), _ptr(col),
                               _ptr(val), _ptr(lhs), _ptr(rhs), _ptr(out),
                               kind, alpha, beta)
    return out


def row_reduce(ro, val, kind=REDUCE_SUM):
    """SparseWaveToGPU.cpp:752-818."""
    ro, val = _c(ro, np.int32), _c(val, np.float32)
    rows = ro.size - 1
    out = np.empty(rows, np.float32)
    lib().oracle_csr_row_reduce_f32(rows, _ptr(ro), _ptr(val), _ptr(out), kind)
    return out


def rowwise_map(ro, val, row_values, kind=MAP_EXP_SUB):
    """SparseWaveToGPU.cpp:820-878."""
    ro, val = _c(ro, np.int32), _c(val, np.float32)
    rv = _c(row_values, np.float32)
    rows = ro.size - 1
    out = np.empty(val.size, np.float32)
    lib().oracle_csr_rowwise_map_f32(rows, _ptr(ro), _ptr(val), _ptr(rv),
                                     _ptr(out), kind)
    return out


def sparse_attention(ro, col, mask_values, query, transposed_key, value,
                     alpha, beta=0.0):
    """SparseAttentionToSparseWave.cpp:230-315 (six ops in order).
    Returns (scores, row_max, row_sum, output)."""
    ro, col = _c(ro, np.int32), _c(col, np.int32)
    mv = _c(mask_values, np.float32)
    q, kt, v = (_c(query, np.float32), _c(transposed_key, np.float32),
                _c(value, np.float32))
    rows, d = q.shape
    cols = kt.shape[1]
    dv = v.shape[1]
    scores = np.empty(col.size, np.float32)
    rmax = np.empty(rows, np.float32)
    rsum = np.empty(rows, np.float32)
    out = np.empty((rows, dv), np.float32)
    lib().oracle_sparse_attention_f32(rows, cols, d, dv, _ptr(ro), _ptr(col),
                                      _ptr(mv), _ptr(q), _ptr(kt), _ptr(v),
                                      _ptr(scores), _ptr(rmax), _ptr(rsum),
                                      _ptr(out), alpha, beta)
    return scores, rmax, rsum, out


def round_bf16(a):
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    a = _c(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().oracle_round_bf16(a.size, _ptr(a), _ptr(out))
    return out


def bf16_to_f32(h):
    """bf16 bit patterns (uint16) -> their exact fp32 values."""
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_bf16_to_f32(h.size, _ptr(h), _ptr(out))
    return out


def as_bf16(a):
    """The fp32 values of a rounded to bf16 (what a bf16 buffer holds)."""
    return bf16_to_f32(round_bf16(a))


def sparse_attention_bf16(ro, col, mask_values, query, transposed_key, value,
                          alpha, beta=0.0):
    """The six ops on bf16 buffers, each op's result rounded to bf16
    (SparseAttentionToSparseWave.cpp:270-312 with a bf16 element type).
    Inputs are rounded to bf16 first.  Returns the fp32 values of the bf16
    (scores, row_max, row_sum, output)."""
    ro, col = _c(ro, np.int32), _c(col, np.int32)
    mv = as_bf16(mask_values)
    q, kt, v = as_bf16(query), as_bf16(transposed_key), as_bf16(value)
    rows, d = q.shape
    cols = kt.shape[1]
    dv = v.shape[1]
    scores = np.empty(col.size, np.float32)
    rmax = np.empty(rows, np.float32)
    rsum = np.empty(rows, np.float32)
    out = np.empty((rows, dv), np.float32)
    lib().oracle_sparse_attention_bf16(rows, cols, d, dv, _ptr(ro), _ptr(col),
                                       _ptr(mv), _ptr(q), _ptr(kt), _ptr(v),
                                       _ptr(scores), _ptr(rmax), _ptr(rsum),
                                       _ptr(out), alpha, beta)
    return scores, rmax, rsum, out


def rows_at_positions(ro, positions):
    """SparsePositionToSCF.cpp:225-271."""
    ro = _c(ro, np.int32)
    pos = _c(positions, np.int64)
    out = np.empty(pos.size, np.int32)
    lib().oracle_csr_rows_at_positions(ro.size - 1, _ptr(ro), pos.size,
                                       _ptr(pos), _ptr(out))
    return out


def position_space(lower, upper, worker, worker_count):
    """SparsePositionToSCF.cpp:190-223."""
    b, e = _I64(), _I64()
    lib().oracle_position_space(lower, upper, worker, worker_count,
                                ctypes.byref(b), ctypes.byref(e))
    return b.value, e.value


def wave_segmented_scan(keys, values, active):
    """SparseGPUUtils.cpp:247-292 emulated for one wave."""
    keys = _c(keys, np.int64)
    values = _c(values, np.float32)
    active = _c(active, np.uint8)
    w = keys.size
    out = np.empty(w, np.float32)
    seg = np.empty(w, np.uint8)
    lib().oracle_wave_segmented_scan(w, _ptr(keys), _ptr(values),
                                     _ptr(active), _ptr(out), _ptr(seg))
    return out, seg.astype(bool)


def spmv_wave_position(ro, col, val, x, block=256, wave=64):
    """SparsePositionScheduling.cpp:318-403 schedule, emulated serially."""
    ro, col, val, x = (_c(ro, np.int32), _c(col, np.int32),
                       _c(val, np.float32), _c(x, np.float32))
    rows = ro.size - 1
    y = np.empty(rows, np.float32)
    lib().oracle_spmv_wave_position_f32(rows, col.size, _ptr(ro), _ptr(col),
                                        _ptr(val), _ptr(x), _ptr(y), block,
                                        wave)
    return y
