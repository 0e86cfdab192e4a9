"""sparsewavecomp_amd: the SparseWave sparse hot path on MI355X (gfx950).

Python mirror of the op-level interface: each function takes the operands of
the matching ``sparsewave`` op in the op's operand order
(include/sparsewave/Dialect/SparseWave/IR/SparseWaveOps.td) as device
tensors, plus lowering options under the reference's option names, and
enqueues the hand-written HIP kernels of ``libsparsewave_amd.so`` through its
C ABI (include/sparsewave_amd.h) on the current torch stream.

Errors raise :class:`SparseWaveError` carrying the library's diagnostic.
There is no CPU fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import os

__all__ = [
    "Options", "SparseWaveError", "ShapeError", "library_path",
    "load_library", "spmv",
    "coo_spmv", "spmv_gather_floor", "bsr_slab_floor", "attention_tile_floor",
    "spmm", "bsr_spmm", "sddmm", "csr_row_reduce", "csr_rowwise_map",
    "sparse_attention", "csr_row_at_position", "SDDMM_MUL", "SDDMM_AFFINE",
    "SDDMM_DOT", "MAP_EXP_SUB", "MAP_DIV", "MAP_SUB", "MAP_MUL",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_NAME = "libsparsewave_amd.so"

SW_OK = 0
SDDMM_MUL, SDDMM_AFFINE, SDDMM_DOT = 0, 1, 2
MAP_EXP_SUB, MAP_DIV, MAP_SUB, MAP_MUL = 0, 1, 2, 3

EXPORTED_SYMBOLS = (
    "sw_options_init", "sw_options_set", "sw_options_parse",
    "sw_validate_options", "sw_last_error", "sw_version", "sw_spmv_csr_f32",
    "sw_spmv_coo_f32", "sw_spmv_gather_floor_f32",
    "sw_spmm_csr_f32", "sw_spmm_csr_bf16", "sw_bsr_spmm_f32",
    "sw_bsr_spmm_bf16", "sw_bsr_spmm_bf16_f32out", "sw_bsr_slab_floor",
    "sw_sddmm_csr_f32",
    "sw_sddmm_csr_bf16", "sw_csr_row_reduce_f32", "sw_csr_row_reduce_bf16",
    "sw_csr_rowwise_map_f32", "sw_csr_rowwise_map_bf16",
    "sw_sparse_attention_f32", "sw_sparse_attention_bf16",
    "sw_csr_row_at_position", "sw_attention_tile_floor",
    "sw_host_matrix_free", "sw_host_bsr_free", "sw_matrix_market_read",
    "sw_csr_binary_write", "sw_coo_binary_write", "sw_csr_binary_read",
    "sw_coo_binary_read", "sw_convert_to_bsr", "sw_bsr_binary_write",
    "sw_bsr_binary_read",
)


class SparseWaveError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class _COptions(ctypes.Structure):
    _fields_ = [
        ("spmv_mapping", ctypes.c_char * 32),
        ("spmv_block_size", ctypes.c_int64),
        ("spmv_position_chunk_size", ctypes.c_int64),
        ("spmv_position_reduction", ctypes.c_char * 16),
        ("position_block_size", ctypes.c_int64),
        ("spmm_mapping", ctypes.c_char * 32),
        ("spmm_block_size", ctypes.c_int64),
        ("spmm_tile_size", ctypes.c_int64),
        ("spmm_position_chunk_size", ctypes.c_int64),
        ("sddmm_block_size", ctypes.c_int64),
        ("row_reduction_block_size", ctypes.c_int64),
        ("rowwise_map_block_size", ctypes.c_int64),
        ("elementwise_block_size", ctypes.c_int64),
        ("wavefront_size", ctypes.c_int64),
        ("spmv_lanes_per_row", ctypes.c_int64),
        ("spmv_positions_per_lane", ctypes.c_int64),
        ("spmm_lanes_per_row", ctypes.c_int64),
        ("bsr_use_mfma", ctypes.c_int64),
        ("sddmm_lanes_per_row", ctypes.c_int64),
        ("spmm_positions_per_lane", ctypes.c_int64),
        ("sddmm_mapping", ctypes.c_char * 32),
    ]


_lib = None


def library_path() -> str:
    return os.path.join(_HERE, _LIB_NAME)


def load_library():
    """Load the in-tree HIP library (built by sparsewavecomp_amd.build)."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it with `python -m "
            f"sparsewavecomp_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(path)
    P, I64, C = ctypes.c_void_p, ctypes.c_int64, ctypes.c_char_p
    OP = ctypes.POINTER(_COptions)
    F = ctypes.c_float
    sig = {
        "sw_options_init": (None, [OP]),
        "sw_options_set": (ctypes.c_int, [OP, C, C]),
        "sw_options_parse": (ctypes.c_int, [OP, C]),
        "sw_validate_options": (ctypes.c_int, [OP]),
        "sw_last_error": (C, []),
        "sw_version": (C, []),
        "sw_spmv_csr_f32": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64, OP,
                                           P]),
        "sw_spmv_coo_f32": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64, OP,
                                           P]),
        "sw_spmv_gather_floor_f32": (ctypes.c_int, [P, P, P, P, I64, P]),
        "sw_bsr_slab_floor": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64,
                                             I64, ctypes.c_int, ctypes.c_int,
                                             P]),
        "sw_attention_tile_floor": (ctypes.c_int, [P] * 10 + [I64] * 5 + [
            ctypes.c_int, P]),
        "sw_spmm_csr_f32": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64, I64,
                                           OP, P]),
        "sw_spmm_csr_bf16": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64, I64,
                                            OP, P]),
        "sw_bsr_spmm_f32": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64, I64,
                                           I64, OP, P]),
        "sw_bsr_spmm_bf16": (ctypes.c_int, [P, P, P, P, P, I64, I64, I64, I64,
                                            I64, OP, P]),
        "sw_bsr_spmm_bf16_f32out": (ctypes.c_int, [P, P, P, P, P, I64, I64,
                                                   I64, I64, I64, OP, P]),
        "sw_sddmm_csr_f32": (ctypes.c_int, [P, P, P, P, P, P, I64, I64, I64,
                                            I64, ctypes.c_int, F, F, OP, P]),
        "sw_sddmm_csr_bf16": (ctypes.c_int, [P, P, P, P, P, P, I64, I64, I64,
                                             I64, ctypes.c_int, F, F, OP, P]),
        "sw_csr_row_reduce_f32": (ctypes.c_int, [P, P, P, P, I64, I64, C, OP,
                                                 P]),
        "sw_csr_row_reduce_bf16": (ctypes.c_int, [P, P, P, P, I64, I64, C, OP,
                                                  P]),
        "sw_csr_rowwise_map_f32": (ctypes.c_int, [P, P, P, P, P, I64, I64,
                                                  ctypes.c_int, OP, P]),
        "sw_csr_rowwise_map_bf16": (ctypes.c_int, [P, P, P, P, P, I64, I64,
                                                   ctypes.c_int, OP, P]),
        "sw_sparse_attention_f32": (ctypes.c_int, [P, P, P, P, P, P, P, P, P,
                                                   P, I64, I64, I64, I64, I64,
                                                   F, F, OP, P]),
        "sw_sparse_attention_bf16": (ctypes.c_int, [P, P, P, P, P, P, P, P, P,
                                                    P, I64, I64, I64, I64,
                                                    I64, F, F, OP, P]),
        "sw_csr_row_at_position": (ctypes.c_int, [P, I64, P, P, I64, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc: int):
    if rc != SW_OK:
        msg = load_library().sw_last_error().decode()
        raise SparseWaveError(rc, msg)


class Options:
    """Lowering options under the reference's names.

    ``Options(spmv_mapping="wave-per-row", spmv_block_size=128)`` or
    ``Options.parse("spmv-mapping=wave-per-row spmv-block-size=128")``.
    Keyword names are the option names with '-' replaced by '_'.
    """

    def __init__(self, **kwargs):
        self._c = _COptions()
        load_library().sw_options_init(ctypes.byref(self._c))
        for key, value in kwargs.items():
            self.set(key.replace("_", "-"), value)

    @classmethod
    def parse(cls, text: str) -> "Options":
        o = cls()
        _check(load_library().sw_options_parse(ctypes.byref(o._c),
                                               text.encode()))
        return o

    def set(self, name: str, value) -> "Options":
        _check(load_library().sw_options_set(ctypes.byref(self._c),
                                             name.encode(),
                                             str(value).encode()))
        return self

    def validate(self) -> "Options":
        _check(load_library().sw_validate_options(ctypes.byref(self._c)))
        return self

    def __getattr__(self, item):
        if item.startswith("_"):
            raise AttributeError(item)
        v = getattr(self._c, item)
        return v.decode() if isinstance(v, bytes) else v

    @property
    def ref(self):
        return ctypes.byref(self._c)

    def __repr__(self):
        fields = ", ".join(f"{n}={getattr(self, n)!r}"
                           for n, _ in _COptions._fields_)
        return f"Options({fields})"


def _opts(options):
    if options is None:
        return None
    if isinstance(options, str):
        options = Options.parse(options)
    return options.ref


def _dev(t, dtype, name):
    import torch
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:  # cheaper than building t.device on every call
        raise ValueError(f"{name} must be a device tensor, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch
    if stream is None:
        # the current stream's handle without building a Stream object
        # (about 0.1 us against 2.8 us per call on the MI355X host)
        raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if raw is not None:
            return ctypes.c_void_p(raw(torch.cuda.current_device()))
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class ShapeError(SparseWaveError, ValueError):
    """Operand shapes that do not fit the op, caught before the C ABI is
    called (SW_ERR_INVALID_SHAPE)."""

    def __init__(self, message: str):
        super().__init__(-2, message)


def _need(cond, message):
    if not cond:
        raise ShapeError(message)


def _rows_of(row_offsets, name="row_offsets"):
    _need(row_offsets.dim() == 1 and row_offsets.numel() >= 1,
          f"{name} must be a 1-D tensor of rows + 1 offsets")
    return row_offsets.numel() - 1


def _value_dtype(t, name):
    """fp32 or bf16: the element type shared by an op's value operands."""
    import torch
    if t.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"{name} must be float32 or bfloat16, got {t.dtype}")
    return t.dtype


def _fn(base, dtype):
    import torch
    return getattr(load_library(),
                   base + ("_bf16" if dtype == torch.bfloat16 else "_f32"))


def spmv(row_offsets, column_indices, values, vector, output, options=None,
         stream=None):
    """sparsewave.spmv (SparseWaveOps.td:17-52): output = A @ vector."""
    import torch
    rows = _rows_of(row_offsets)
    _need(column_indices.numel() == values.numel(),
          "column indices and values must have the same length")
    _need(vector.dim() == 1, "vector must be 1-D")
    _need(output.dim() == 1 and output.numel() == rows,
          f"output must hold rows = {rows} values")
    _check(load_library().sw_spmv_csr_f32(
        _dev(row_offsets, torch.int32, "row_offsets"),
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(values, torch.float32, "values"),
        _dev(vector, torch.float32, "vector"),
        _dev(output, torch.float32, "output"), rows, vector.numel(),
        values.numel(), _opts(options), _stream(stream)))
    return output


def coo_spmv(row_indices, column_indices, values, vector, output,
             options=None, stream=None):
    """sparsewave.coo_spmv (SparseWaveOps.td:54-88): output = A @ vector with
    A as COO entries (any order, repeated coordinates add up)."""
    import torch
    _need(row_indices.numel() == column_indices.numel() == values.numel(),
          "COO row indices, column indices and values must have the same "
          "length")
    _need(vector.dim() == 1 and output.dim() == 1,
          "vector and output must be 1-D")
    _check(load_library().sw_spmv_coo_f32(
        _dev(row_indices, torch.int32, "row_indices"),
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(values, torch.float32, "values"),
        _dev(vector, torch.float32, "vector"),
        _dev(output, torch.float32, "output"), output.numel(), vector.numel(),
        values.numel(), _opts(options), _stream(stream)))
    return output


def spmv_gather_floor(column_indices, values, vector, partial, stream=None):
    """Diagnostic (no reference counterpart): partial[w] = sum of
    values[p] * vector[column_indices[p]] over p in [512 w, 512 w + 512),
    i.e. a CSR SpMV's column/value reads and x gathers without its rows."""
    import torch
    nnz = values.numel()
    _need(column_indices.numel() == nnz,
          "column indices and values must have the same length")
    _need(partial.numel() >= (nnz + 511) // 512,
          "partial needs ceil(nnz / 512) entries")
    _check(load_library().sw_spmv_gather_floor_f32(
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(values, torch.float32, "values"),
        _dev(vector, torch.float32, "vector"),
        _dev(partial, torch.float32, "partial"), nnz, _stream(stream)))
    return partial


def spmm(row_offsets, column_indices, values, rhs, output, options=None,
         stream=None):
    """sparsewave.spmm (SparseWaveOps.td:91-124): output = A @ rhs.  values,
    rhs and output share one element type, float32 or bfloat16."""
    import torch
    rows = _rows_of(row_offsets)
    dt = _value_dtype(values, "values")
    _need(column_indices.numel() == values.numel(),
          "column indices and values must have the same length")
    _need(rhs.dim() == 2 and output.dim() == 2 and
          tuple(output.shape) == (rows, rhs.shape[1]),
          "expected rhs [cols, k] and output [rows, k]")
    _check(_fn("sw_spmm_csr", dt)(
        _dev(row_offsets, torch.int32, "row_offsets"),
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(values, dt, "values"), _dev(rhs, dt, "rhs"),
        _dev(output, dt, "output"), rows, rhs.shape[0], values.numel(),
        rhs.shape[1], _opts(options), _stream(stream)))
    return output


def bsr_spmm(block_row_offsets, block_column_indices, block_values, rhs,
             output, block_size, options=None, stream=None):
    """sparsewave.bsr_spmm (SparseWaveOps.td:126-169).  float32 operands, or
    bfloat16 block values and rhs with a bfloat16 output (the op's
    same-element-type rule) or, as an extension, a float32 output."""
    import torch
    _need(block_size >= 1, "block size must be positive")
    rows = _rows_of(block_row_offsets, "block_row_offsets") * block_size
    nnzb = block_column_indices.numel()
    dt = _value_dtype(block_values, "block_values")
    _need(block_values.numel() == nnzb * block_size * block_size,
          "block values must hold nnzb * block_size^2 entries")
    _need(rhs.dim() == 2 and output.dim() == 2 and
          tuple(output.shape) == (rows, rhs.shape[1]),
          "expected rhs [cols, k] and output [rows, k]")
    lib = load_library()
    if dt == torch.float32:
        fn, odt = lib.sw_bsr_spmm_f32, torch.float32
    elif output.dtype == torch.float32:
        fn, odt = lib.sw_bsr_spmm_bf16_f32out, torch.float32
    else:
        fn, odt = lib.sw_bsr_spmm_bf16, torch.bfloat16
    _check(fn(_dev(block_row_offsets, torch.int32, "block_row_offsets"),
              _dev(block_column_indices, torch.int32, "block_column_indices"),
              _dev(block_values, dt, "block_values"), _dev(rhs, dt, "rhs"),
              _dev(output, odt, "output"), rows, rhs.shape[0], nnzb,
              rhs.shape[1], block_size, _opts(options), _stream(stream)))
    return output


def bsr_slab_floor(block_row_offsets, block_column_indices, block_values,
                   rhs, output, stream=None):
    """Diagnostic (no reference counterpart): the matrix-core BSR SpMM
    launch for these operands (16 x 16 blocks) with its loads, reduction and
    stores as they are and the block products replaced by an XOR of the
    words each lane loads (sw_bsr_slab_floor); the output holds those XORs
    as bit patterns.  float32 operands, or bfloat16 block values and rhs with
    a bfloat16 or float32 output."""
    import torch
    rows = _rows_of(block_row_offsets, "block_row_offsets") * 16
    nnzb = block_column_indices.numel()
    dt = _value_dtype(block_values, "block_values")
    _need(block_values.numel() == nnzb * 256,
          "block values must hold nnzb * 16 * 16 entries")
    _need(rhs.dim() == 2 and output.dim() == 2 and
          tuple(output.shape) == (rows, rhs.shape[1]),
          "expected rhs [cols, k] and output [rows, k]")
    _need(output.dtype in (torch.float32, torch.bfloat16) and
          (dt == torch.bfloat16 or output.dtype == torch.float32),
          "fp32 operands take a float32 output; bf16 a bf16 or float32 one")
    vb = 4 if dt == torch.float32 else 2
    ob = 4 if output.dtype == torch.float32 else 2
    _check(load_library().sw_bsr_slab_floor(
        _dev(block_row_offsets, torch.int32, "block_row_offsets"),
        _dev(block_column_indices, torch.int32, "block_column_indices"),
        _dev(block_values, dt, "block_values"), _dev(rhs, dt, "rhs"),
        _dev(output, output.dtype, "output"), rows, rhs.shape[0], nnzb,
        rhs.shape[1], vb, ob, _stream(stream)))
    return output


def attention_tile_floor(row_offsets, column_indices, mask_values, query,
                         transposed_key, value, scores, row_maximum, row_sum,
                         output, stream=None):
    """Diagnostic (no reference counterpart): the fused attention tile
    kernel for these buffers with its loads, structure check, stores and
    output reduction as they are and every product, exponential and
    division replaced by an XOR of the loaded words
    (sw_attention_tile_floor).  float32 or bfloat16 buffers."""
    import torch
    rows = _rows_of(row_offsets)
    nnz = column_indices.numel()
    dt = _value_dtype(query, "query")
    _need(query.dim() == 2 and transposed_key.dim() == 2 and
          value.dim() == 2 and output.dim() == 2 and
          query.shape[1] == transposed_key.shape[0] and
          transposed_key.shape[1] == value.shape[0] and
          tuple(output.shape) == (rows, value.shape[1]),
          "expected query [rows, d], transposed_key [d, cols], "
          "value [cols, dv] and output [rows, dv]")
    _need(mask_values.numel() == nnz and scores.numel() == nnz and
          row_maximum.numel() == rows and row_sum.numel() == rows,
          "mask values and scores hold nnz entries, row buffers rows")
    _check(load_library().sw_attention_tile_floor(
        _dev(row_offsets, torch.int32, "row_offsets"),
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(mask_values, dt, "mask_values"), _dev(query, dt, "query"),
        _dev(transposed_key, dt, "transposed_key"), _dev(value, dt, "value"),
        _dev(scores, dt, "scores"), _dev(row_maximum, dt, "row_maximum"),
        _dev(row_sum, dt, "row_sum"), _dev(output, dt, "output"), rows,
        transposed_key.shape[1], nnz, query.shape[1], value.shape[1],
        4 if dt == torch.float32 else 2, _stream(stream)))
    return output


def sddmm(row_offsets, column_indices, values, lhs, rhs, output_values,
          combine=SDDMM_MUL, alpha=1.0, beta=0.0, options=None, stream=None):
    """sparsewave.sddmm (SparseWaveOps.td:171-223); float32 or bfloat16."""
    import torch
    rows = _rows_of(row_offsets)
    nnz = column_indices.numel()
    dt = _value_dtype(output_values, "output_values")
    _need(lhs.dim() == 2 and rhs.dim() == 2 and lhs.shape[1] == rhs.shape[0],
          "expected lhs [rows, k] and rhs [k, cols]")
    _need(lhs.shape[0] == rows, f"lhs must have rows = {rows} rows")
    _need(output_values.numel() == nnz,
          "output values must hold one value per stored entry")
    if combine != SDDMM_DOT:
        _need(values.numel() == nnz,
              "values must hold one value per stored entry")
    vals = values if combine != SDDMM_DOT else output_values
    _check(_fn("sw_sddmm_csr", dt)(
        _dev(row_offsets, torch.int32, "row_offsets"),
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(vals, dt, "values"), _dev(lhs, dt, "lhs"), _dev(rhs, dt, "rhs"),
        _dev(output_values, dt, "output_values"), rows, rhs.shape[1], nnz,
        lhs.shape[1], combine, alpha, beta, _opts(options), _stream(stream)))
    return output_values


def csr_row_reduce(row_offsets, column_indices, values, output, kind="sum",
                   options=None, stream=None):
    """sparsewave.csr_row_reduce (SparseWaveOps.td:225-257)."""
    import torch
    rows = _rows_of(row_offsets)
    dt = _value_dtype(values, "values")
    _need(output.numel() == rows, f"output must hold rows = {rows} values")
    if column_indices is not None:
        _need(column_indices.numel() == values.numel(),
              "column indices and values must have the same length")
    ci = (None if column_indices is None else
          _dev(column_indices, torch.int32, "column_indices"))
    _check(_fn("sw_csr_row_reduce", dt)(
        _dev(row_offsets, torch.int32, "row_offsets"), ci,
        _dev(values, dt, "values"), _dev(output, dt, "output"), rows,
        values.numel(), kind.encode(), _opts(options), _stream(stream)))
    return output


def csr_rowwise_map(row_offsets, column_indices, values, row_values,
                    output_values, kind=MAP_EXP_SUB, options=None,
                    stream=None):
    """sparsewave.csr_rowwise_map (SparseWaveOps.td:259-299)."""
    import torch
    rows = _rows_of(row_offsets)
    dt = _value_dtype(values, "values")
    _need(row_values.numel() == rows,
          f"row values must hold rows = {rows} values")
    _need(output_values.numel() == values.numel(),
          "output values and values must have the same length")
    if column_indices is not None:
        _need(column_indices.numel() == values.numel(),
              "column indices and values must have the same length")
    ci = (None if column_indices is None else
          _dev(column_indices, torch.int32, "column_indices"))
    _check(_fn("sw_csr_rowwise_map", dt)(
        _dev(row_offsets, torch.int32, "row_offsets"), ci,
        _dev(values, dt, "values"), _dev(row_values, dt, "row_values"),
        _dev(output_values, dt, "output_values"), rows, values.numel(), kind,
        _opts(options), _stream(stream)))
    return output_values


def sparse_attention(row_offsets, column_indices, mask_values, query,
                     transposed_key, value, scores, row_maximum, row_sum,
                     output, alpha, beta=0.0, options=None, stream=None):
    """The six-op sparse attention chain
    (SparseAttentionToSparseWave.cpp:230-315), ten-buffer ABI; all value
    buffers float32, or all bfloat16 (the bf16 option)."""
    import torch
    rows = _rows_of(row_offsets)
    nnz = column_indices.numel()
    dt = _value_dtype(query, "query")
    _need(query.dim() == 2 and transposed_key.dim() == 2 and
          value.dim() == 2 and output.dim() == 2,
          "query, transposed_key, value and output must be 2-D")
    d, cols, dv = query.shape[1], transposed_key.shape[1], value.shape[1]
    _need(query.shape[0] == rows, f"query must have rows = {rows} rows")
    _need(transposed_key.shape[0] == d,
          "transposed key must have head-dim rows")
    _need(value.shape[0] == cols,
          "value must have one row per key (transposed key column)")
    _need(mask_values.numel() == nnz and scores.numel() == nnz,
          "mask values and scores must hold one value per stored entry")
    _need(row_maximum.numel() == rows and row_sum.numel() == rows,
          f"row maximum and row sum must hold rows = {rows} values")
    _need(tuple(output.shape) == (rows, dv), "expected output [rows, dv]")
    _check(_fn("sw_sparse_attention", dt)(
        _dev(row_offsets, torch.int32, "row_offsets"),
        _dev(column_indices, torch.int32, "column_indices"),
        _dev(mask_values, dt, "mask_values"), _dev(query, dt, "query"),
        _dev(transposed_key, dt, "transposed_key"), _dev(value, dt, "value"),
        _dev(scores, dt, "scores"), _dev(row_maximum, dt, "row_maximum"),
        _dev(row_sum, dt, "row_sum"), _dev(output, dt, "output"), rows, cols,
        nnz, d, dv, alpha, beta, _opts(options), _stream(stream)))
    return output


def csr_row_at_position(row_offsets, positions, out_rows, stream=None):
    """sparsewave.csr_row_at_position for a batch (SparsePositionToSCF.cpp:225-271)."""
    import torch
    _check(load_library().sw_csr_row_at_position(
        _dev(row_offsets, torch.int32, "row_offsets"),
        row_offsets.numel() - 1, _dev(positions, torch.int64, "positions"),
        _dev(out_rows, torch.int32, "out_rows"), positions.numel(),
        _stream(stream)))
    return out_rows
