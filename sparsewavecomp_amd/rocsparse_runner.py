"""rocSPARSE comparison runner: the vendor library's CSR SpMV / SpMM on the
same device buffers, as a second GPU baseline beside the CPU one (the
reference does the same in benchmark/SparseRocSparseBenchmark.cpp:205-387,
timing rocSPARSE's default SpMV/SpMM with HIP events).

Uses the generic API (rocsparse_spmv / rocsparse_spmm) through ctypes on
the installed librocsparse; the buffer-size and preprocess stages run once
at set-up, the returned callable runs only the compute stage.  Nothing in
the product path imports this module.
"""
from __future__ import annotations

import ctypes

_OP_NONE = 111
_INDEX_I32 = 2
_F32 = 151
_BASE_ZERO = 0
_ORDER_ROW = 0
_STAGE_BUFFER, _STAGE_PRE, _STAGE_COMPUTE = 1, 2, 3

SPMV_ALGS = {"default": 0, "csr_adaptive": 2, "csr_rowsplit": 3,
             "csr_lrb": 7, "csr_nnzsplit": 8}
SPMM_ALGS = {"default": 0, "csr": 1, "csr_row_split": 4, "csr_merge": 5,
             "csr_merge_path": 9}


class RocSparseError(RuntimeError):
    pass


class RocSparse:
    def __init__(self, stream=None):
        import torch
        torch.cuda.init()
        self.lib = ctypes.CDLL("librocsparse.so.1")
        self.handle = ctypes.c_void_p()
        self._ok(self.lib.rocsparse_create_handle(ctypes.byref(self.handle)),
                 "create_handle")
        st = (stream or torch.cuda.current_stream()).cuda_stream
        self._ok(self.lib.rocsparse_set_stream(self.handle,
                                               ctypes.c_void_p(st)),
                 "set_stream")
        self._keep = []

    @staticmethod
    def _ok(rc, what):
        if rc != 0:
            raise RocSparseError(f"rocsparse_{what} failed with status {rc}")

    def _csr(self, ro, col, val, rows, cols):
        d = ctypes.c_void_p()
        f = self.lib.rocsparse_create_csr_descr
        f.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64,
                      ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                      ctypes.c_int, ctypes.c_int, ctypes.c_int]
        self._ok(f(ctypes.byref(d), rows, cols, val.numel(), ro.data_ptr(),
                   col.data_ptr(), val.data_ptr(), _INDEX_I32, _INDEX_I32,
                   _BASE_ZERO, _F32), "create_csr_descr")
        return d

    def _vec(self, t):
        d = ctypes.c_void_p()
        f = self.lib.rocsparse_create_dnvec_descr
        f.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64,
                      ctypes.c_void_p, ctypes.c_int]
        self._ok(f(ctypes.byref(d), t.numel(), t.data_ptr(), _F32),
                 "create_dnvec_descr")
        return d

    def _mat(self, t):
        d = ctypes.c_void_p()
        f = self.lib.rocsparse_create_dnmat_descr
        f.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int64,
                      ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                      ctypes.c_int, ctypes.c_int]
        r, c = t.shape
        self._ok(f(ctypes.byref(d), r, c, c, t.data_ptr(), _F32, _ORDER_ROW),
                 "create_dnmat_descr")
        return d

    def spmv(self, ro, col, val, x, y, alg="default"):
        """Set up y = A x; returns the compute-stage callable."""
        import torch
        mat = self._csr(ro, col, val, ro.numel() - 1, x.numel())
        vx, vy = self._vec(x), self._vec(y)
        alpha, beta = ctypes.c_float(1.0), ctypes.c_float(0.0)
        size = ctypes.c_size_t(0)
        f = self.lib.rocsparse_spmv
        f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                      ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                      ctypes.c_int, ctypes.POINTER(ctypes.c_size_t),
                      ctypes.c_void_p]
        a = SPMV_ALGS[alg]

        def call(stage, buf):
            self._ok(f(self.handle, _OP_NONE, ctypes.byref(alpha), mat, vx,
                       ctypes.byref(beta), vy, _F32, a, stage,
                       ctypes.byref(size), buf), "spmv")

        call(_STAGE_BUFFER, None)
        tmp = torch.empty(max(size.value, 1), dtype=torch.uint8,
                          device=x.device)
        call(_STAGE_PRE, ctypes.c_void_p(tmp.data_ptr()))
        self._keep.append((mat, vx, vy, alpha, beta, size, tmp))
        buf = ctypes.c_void_p(tmp.data_ptr())
        return lambda: call(_STAGE_COMPUTE, buf)

    def spmm(self, ro, col, val, rhs, out, alg="default"):
        """Set up out = A rhs (row-major dense); returns the compute call."""
        import torch
        mat = self._csr(ro, col, val, ro.numel() - 1, rhs.shape[0])
        mb, mc = self._mat(rhs), self._mat(out)
        alpha, beta = ctypes.c_float(1.0), ctypes.c_float(0.0)
        size = ctypes.c_size_t(0)
        f = self.lib.rocsparse_spmm
        f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                      ctypes.c_int, ctypes.c_int,
                      ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p]
        a = SPMM_ALGS[alg]

        def call(stage, buf):
            self._ok(f(self.handle, _OP_NONE, _OP_NONE, ctypes.byref(alpha),
                       mat, mb, ctypes.byref(beta), mc, _F32, a, stage,
                       ctypes.byref(size), buf), "spmm")

        call(_STAGE_BUFFER, None)
        tmp = torch.empty(max(size.value, 1), dtype=torch.uint8,
                          device=rhs.device)
        call(_STAGE_PRE, ctypes.c_void_p(tmp.data_ptr()))
        self._keep.append((mat, mb, mc, alpha, beta, size, tmp))
        buf = ctypes.c_void_p(tmp.data_ptr())
        return lambda: call(_STAGE_COMPUTE, buf)
