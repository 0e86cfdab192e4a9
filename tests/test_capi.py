"""Host-side tests of the C ABI: the library loads, exports every function
the header declares, and validates options and shapes the way the
reference's passes do -- all without touching a GPU (each call here returns
before any HIP call)."""
import ctypes
import os
import re

import pytest

import sparsewavecomp_amd as sw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    text = open(os.path.join(ROOT, "include", "sparsewave_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sw_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    lib = sw.load_library()
    declared = _declared_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), f"{name} declared but not exported"
    assert set(declared) == set(sw.EXPORTED_SYMBOLS)


def test_version():
    assert b"gfx950" in sw.load_library().sw_version()


def test_defaults_match_reference():
    o = sw.Options()
    # Pipelines.h:114-178 / Passes.td:207-241 defaults
    assert o.spmv_mapping == "thread-per-row"
    assert o.spmv_block_size == 256
    assert o.spmm_mapping == "thread-per-output"
    assert o.spmm_block_size == 256
    assert o.spmm_tile_size == 4
    assert o.spmv_position_chunk_size == 1
    assert o.spmv_position_reduction == "atomic"
    assert o.position_block_size == 256
    assert o.sddmm_block_size == 256
    assert o.row_reduction_block_size == 256
    assert o.rowwise_map_block_size == 256
    assert o.wavefront_size == 64
    o.validate()


def test_parse_pipeline_string():
    o = sw.Options.parse(
        "sparsewave-to-amdgpu-pipeline{chip=gfx950 wavefront-size=64 "
        "spmv-mapping=wave-per-row spmv-block-size=128 spmm-mapping="
        "wave-per-row-tile spmm-tile-size=8 rocm-path=/opt/rocm}")
    assert o.spmv_mapping == "wave-per-row"
    assert o.spmv_block_size == 128
    assert o.spmm_mapping == "wave-per-row-tile"
    assert o.spmm_tile_size == 8
    o.validate()
    # pass-level names map onto the same fields
    o2 = sw.Options.parse("mapping=block-per-row block-size=512 wave-size=64")
    assert o2.spmv_mapping == "block-per-row" and o2.spmv_block_size == 512


@pytest.mark.parametrize("text,needle", [
    ("spmv-mapping=diagonal", "unsupported SpMV mapping strategy 'diagonal'"),
    ("spmm-mapping=row", "unsupported SpMM mapping strategy 'row'"),
    ("spmm-mapping=wave-per-position spmm-block-size=96", "wave-per-position requires the SpMM block size to be a multiple of 64, but got 96"),
    ("spmm-positions-per-lane=3", "spmm-positions-per-lane must be 1, 2, 4, 8 or 16"),
    ("spmv-block-size=0", "SpMV block size must be between 1 and 1024, but got 0"),
    ("spmv-block-size=1025", "SpMV block size must be between 1 and 1024, but got 1025"),
    ("position-block-size=0", "position-parallel block size must be between 1 and 1024"),
    ("spmm-block-size=2000", "SpMM block size must be between 1 and 1024"),
    ("spmm-tile-size=0", "SpMM tile size must be between 1 and 32, but got 0"),
    ("spmm-tile-size=33", "SpMM tile size must be between 1 and 32, but got 33"),
    ("sddmm-block-size=0", "SDDMM block size must be between 1 and 1024"),
    ("row-reduction-block-size=0", "CSR row-reduction block size must be between"),
    ("rowwise-map-block-size=0", "CSR row-wise map block size must be between"),
    ("elementwise-block-size=0", "elementwise block size must be between"),
    ("spmv-mapping=wave-per-row wavefront-size=32", "wave-per-row currently requires Wave64"),
    ("spmm-mapping=wave-per-row-tile wavefront-size=32", "wave-per-row-tile currently requires Wave64"),
    ("wavefront-size=32", "gfx950 executes Wave64 only"),
    ("spmv-mapping=wave-per-row spmv-block-size=96", "wave-per-row requires the SpMV block size to be a multiple of 64, but got 96"),
    ("spmv-mapping=block-per-row spmv-block-size=32", "block-per-row requires the SpMV block size to be a multiple of 64"),
    ("spmm-mapping=wave-per-row-tile spmm-block-size=100", "wave-per-row-tile requires the SpMM block size to be a multiple of 64, but got 100"),
    ("spmv-mapping=wave-per-position spmv-block-size=100", "wave position mapping requires the block size to be a multiple of 64"),
    ("spmv-position-chunk-size=0", "thread position chunk size must be positive, but got 0"),
    ("spmv-position-reduction=tree", "unsupported thread position reduction 'tree'"),
    ("spmv-mapping=wave-per-position spmv-position-chunk-size=4", "thread position chunk size applies only to thread mapping"),
    ("spmv-mapping=wave-per-position spmv-position-reduction=segmented", "thread position reduction applies only to thread mapping"),
    ("spmv-lanes-per-row=3", "spmv-lanes-per-row must be a power of two"),
    ("spmv-positions-per-lane=3", "spmv-positions-per-lane must be 1, 2, 4, 8 or 16"),
])
def test_invalid_options(text, needle):
    o = sw.Options.parse(text)
    with pytest.raises(sw.SparseWaveError) as e:
        o.validate()
    assert e.value.code == -1
    assert needle in e.value.message


def test_unknown_option_and_chip():
    with pytest.raises(sw.SparseWaveError, match="unknown option 'bogus'"):
        sw.Options.parse("bogus=1")
    with pytest.raises(sw.SparseWaveError, match="chip=gfx1101"):
        sw.Options.parse("chip=gfx1101")
    with pytest.raises(sw.SparseWaveError, match="expects an integer"):
        sw.Options.parse("spmv-block-size=abc")


def test_entry_points_reject_before_launch():
    """Invalid options / shapes / kinds fail before any device work."""
    lib = sw.load_library()
    bad = sw.Options(spmv_block_size=0)
    P = ctypes.c_void_p
    fake = P(16)  # never dereferenced: validation fails first
    rc = lib.sw_spmv_csr_f32(fake, fake, fake, fake, fake, 4, 4, 4, bad.ref,
                             None)
    assert rc == -1
    assert b"SpMV block size" in lib.sw_last_error()
    rc = lib.sw_spmv_csr_f32(fake, fake, fake, fake, fake, -1, 4, 4, None,
                             None)
    assert rc == -2
    rc = lib.sw_spmv_csr_f32(None, fake, fake, fake, fake, 4, 4, 4, None, None)
    assert rc == -3
    rc = lib.sw_bsr_spmm_f32(fake, fake, fake, fake, fake, 10, 10, 1, 2, 4,
                             None, None)
    assert rc == -2 and b"divisible" in lib.sw_last_error()
    rc = lib.sw_csr_row_reduce_f32(fake, None, fake, fake, 4, 4, b"min", None,
                                   None)
    assert rc == -3 and b"'sum' or 'max'" in lib.sw_last_error()
    rc = lib.sw_csr_rowwise_map_f32(fake, None, fake, fake, fake, 4, 4, 9,
                                    None, None)
    assert rc == -3
    rc = lib.sw_sddmm_csr_f32(fake, fake, fake, fake, fake, fake, 4, 4, 4, 4,
                              7, 1.0, 0.0, None, None)
    assert rc == -3
    # empty problems are no-ops that never launch
    assert lib.sw_spmv_csr_f32(fake, None, None, None, None, 0, 0, 0, None,
                               None) == 0


def test_bf16_entry_points_reject_before_launch():
    """The bf16 entry points validate like the fp32 ones, and the bf16 SpMM
    refuses the mappings that add partial sums into the output."""
    lib = sw.load_library()
    P = ctypes.c_void_p
    fake = P(16)  # never dereferenced: every call below fails validation
    for mapping in ("wave-per-position", "thread-per-position"):
        o = sw.Options(spmm_mapping=mapping, spmm_block_size=64)
        rc = lib.sw_spmm_csr_bf16(fake, fake, fake, fake, fake, 4, 4, 4, 8,
                                  o.ref, None)
        assert rc == -1
        assert b"bf16 output cannot hold" in lib.sw_last_error()
    rc = lib.sw_bsr_spmm_bf16(fake, fake, fake, fake, fake, 10, 10, 1, 2, 4,
                              None, None)
    assert rc == -2 and b"divisible" in lib.sw_last_error()
    rc = lib.sw_bsr_spmm_bf16_f32out(fake, fake, fake, fake, fake, 10, 10, 1,
                                     2, 4, None, None)
    assert rc == -2 and b"divisible" in lib.sw_last_error()
    rc = lib.sw_csr_row_reduce_bf16(fake, None, fake, fake, 4, 4, b"min",
                                    None, None)
    assert rc == -3 and b"'sum' or 'max'" in lib.sw_last_error()
    rc = lib.sw_csr_rowwise_map_bf16(fake, None, fake, fake, fake, 4, 4, 9,
                                     None, None)
    assert rc == -3
    rc = lib.sw_sddmm_csr_bf16(fake, fake, fake, fake, fake, fake, 4, 4, 4, 4,
                               7, 1.0, 0.0, None, None)
    assert rc == -3
    rc = lib.sw_sparse_attention_bf16(fake, fake, fake, fake, fake, fake, fake,
                                      fake, fake, fake, -1, 4, 4, 4, 4, 1.0,
                                      0.0, None, None)
    assert rc == -2
    # empty problems never launch
    assert lib.sw_sparse_attention_bf16(fake, None, None, None, None, None,
                                        None, None, None, None, 0, 0, 0, 4, 4,
                                        1.0, 0.0, None, None) == 0


def test_bf16_attention_rejects_position_spmm_before_any_launch():
    """The bf16 chain ends in a bf16 SpMM, which refuses the position
    mappings: the attention entry point rejects them before its first
    kernel (the SDDMM), so the scores, row maxima and row sums keep what
    they held.  Host buffers stand in for device memory: the call must
    return before it reads or writes any of them."""
    import numpy as np
    lib = sw.load_library()
    rows, nnz, d, dv = 4, 8, 64, 64
    ro = np.array([0, 2, 4, 6, 8], np.int32)
    col = np.array([0, 1] * 4, np.int32)
    ins = [np.zeros(n, np.uint16) for n in (nnz, rows * d, d * 2, 2 * dv)]
    scores = np.full(nnz, 0x7fc1, np.uint16)
    rmax = np.full(rows, 0x7fc2, np.uint16)
    rsum = np.full(rows, 0x7fc3, np.uint16)
    out = np.full(rows * dv, 0x7fc4, np.uint16)
    before = [a.copy() for a in (scores, rmax, rsum, out)]
    P = ctypes.c_void_p
    for mapping in ("wave-per-position", "thread-per-position"):
        o = sw.Options(spmm_mapping=mapping)
        rc = lib.sw_sparse_attention_bf16(
            P(ro.ctypes.data), P(col.ctypes.data),
            *(P(a.ctypes.data) for a in ins),
            *(P(a.ctypes.data) for a in (scores, rmax, rsum, out)),
            rows, 2, nnz, d, dv, 0.125, 0.0, o.ref, None)
        assert rc == -1
        assert b"bf16 output cannot hold" in lib.sw_last_error()
        for a, b in zip((scores, rmax, rsum, out), before):
            assert np.array_equal(a, b)


def test_value_buffers_must_be_element_aligned():
    """An odd address for a bf16 buffer (or a float buffer off its 4-byte
    element) is rejected on every path, whatever the options choose:
    BSR with and without the matrix cores, SpMM, SDDMM, the row ops, the
    attention chain and SpMV."""
    lib = sw.load_library()
    P = ctypes.c_void_p
    ok, odd = P(64), P(65)
    for use_mfma in (1, 0):
        o = sw.Options(bsr_use_mfma=use_mfma)
        for fn in (lib.sw_bsr_spmm_bf16, lib.sw_bsr_spmm_bf16_f32out):
            for args in ((odd, ok, ok), (ok, odd, ok)):
                rc = fn(ok, ok, *args[:2], args[2], 32, 32, 2, 8, 16, o.ref,
                        None)
                assert rc == -3 and b"aligned" in lib.sw_last_error()
        rc = lib.sw_bsr_spmm_bf16(ok, ok, ok, ok, odd, 32, 32, 2, 8, 16,
                                  o.ref, None)
        assert rc == -3 and b"2-byte element" in lib.sw_last_error()
        rc = lib.sw_bsr_spmm_f32(ok, ok, ok, ok, P(66), 32, 32, 2, 8, 16,
                                 o.ref, None)
        assert rc == -3 and b"4-byte element" in lib.sw_last_error()
    assert lib.sw_spmm_csr_bf16(ok, ok, ok, ok, odd, 4, 4, 4, 8, None,
                                None) == -3
    assert lib.sw_sddmm_csr_bf16(ok, ok, ok, odd, ok, ok, 4, 4, 4, 4, 0, 1.0,
                                 0.0, None, None) == -3
    assert lib.sw_csr_row_reduce_bf16(ok, None, ok, odd, 4, 4, b"sum", None,
                                      None) == -3
    assert lib.sw_csr_rowwise_map_bf16(ok, None, ok, odd, ok, 4, 4, 0, None,
                                       None) == -3
    assert lib.sw_sparse_attention_bf16(ok, ok, ok, ok, ok, ok, odd, ok, ok,
                                        ok, 4, 4, 4, 4, 4, 1.0, 0.0, None,
                                        None) == -3
    assert lib.sw_spmv_csr_f32(ok, ok, ok, P(66), ok, 4, 4, 4, None,
                               None) == -3


def _cpu(*shape, dtype=None):
    import torch
    return torch.zeros(shape, dtype=dtype or torch.float32)


def test_mirror_rejects_mismatched_shapes():
    """The Python mirror checks every operand's size against rows, cols,
    nnz, k, d and dv before it calls the C ABI (a mismatch would otherwise be
    an out-of-bounds device access)."""
    import torch
    i32, bf = torch.int32, torch.bfloat16
    ro, col = _cpu(5, dtype=i32), _cpu(8, dtype=i32)
    cases = [
        ("output must hold rows", lambda: sw.spmv(ro, col, _cpu(8), _cpu(6),
                                                  _cpu(5))),
        ("same length", lambda: sw.spmv(ro, col, _cpu(7), _cpu(6), _cpu(4))),
        ("output [rows, k]", lambda: sw.spmm(ro, col, _cpu(8), _cpu(6, 3),
                                             _cpu(4, 2))),
        ("same length", lambda: sw.spmm(ro, col, _cpu(9), _cpu(6, 3),
                                        _cpu(4, 3))),
        ("nnzb * block_size^2", lambda: sw.bsr_spmm(
            _cpu(3, dtype=i32), _cpu(2, dtype=i32), _cpu(7), _cpu(4, 3),
            _cpu(4, 3), 2)),
        ("output [rows, k]", lambda: sw.bsr_spmm(
            _cpu(3, dtype=i32), _cpu(2, dtype=i32), _cpu(8), _cpu(4, 3),
            _cpu(5, 3), 2)),
        ("lhs must have rows", lambda: sw.sddmm(
            ro, col, _cpu(8), _cpu(3, 2), _cpu(2, 6), _cpu(8))),
        ("one value per stored entry", lambda: sw.sddmm(
            ro, col, _cpu(8), _cpu(4, 2), _cpu(2, 6), _cpu(7))),
        ("output must hold rows", lambda: sw.csr_row_reduce(
            ro, None, _cpu(8), _cpu(3))),
        ("row values must hold rows", lambda: sw.csr_rowwise_map(
            ro, None, _cpu(8), _cpu(3), _cpu(8))),
        ("same length", lambda: sw.csr_rowwise_map(
            ro, None, _cpu(8), _cpu(4), _cpu(7))),
        ("query must have rows", lambda: sw.sparse_attention(
            ro, col, _cpu(8), _cpu(3, 2), _cpu(2, 6), _cpu(6, 2), _cpu(8),
            _cpu(4), _cpu(4), _cpu(4, 2), 1.0)),
        ("head-dim rows", lambda: sw.sparse_attention(
            ro, col, _cpu(8), _cpu(4, 2), _cpu(3, 6), _cpu(6, 2), _cpu(8),
            _cpu(4), _cpu(4), _cpu(4, 2), 1.0)),
        ("one row per key", lambda: sw.sparse_attention(
            ro, col, _cpu(8), _cpu(4, 2), _cpu(2, 6), _cpu(5, 2), _cpu(8),
            _cpu(4), _cpu(4), _cpu(4, 2), 1.0)),
        ("one value per stored entry", lambda: sw.sparse_attention(
            ro, col, _cpu(8), _cpu(4, 2), _cpu(2, 6), _cpu(6, 2), _cpu(9),
            _cpu(4), _cpu(4), _cpu(4, 2), 1.0)),
        ("row maximum and row sum", lambda: sw.sparse_attention(
            ro, col, _cpu(8), _cpu(4, 2), _cpu(2, 6), _cpu(6, 2), _cpu(8),
            _cpu(3), _cpu(4), _cpu(4, 2), 1.0)),
        ("output [rows, dv]", lambda: sw.sparse_attention(
            ro, col, _cpu(8, dtype=bf), _cpu(4, 2, dtype=bf),
            _cpu(2, 6, dtype=bf), _cpu(6, 2, dtype=bf), _cpu(8, dtype=bf),
            _cpu(4, dtype=bf), _cpu(4, dtype=bf), _cpu(4, 3, dtype=bf), 1.0)),
    ]
    for needle, call in cases:
        with pytest.raises(ValueError, match=re.escape(needle)):
            call()
    # a shape error is also a SparseWaveError carrying the shape status
    with pytest.raises(sw.SparseWaveError) as e:
        cases[0][1]()
    assert e.value.code == -2
    with pytest.raises(TypeError, match="float32 or bfloat16"):
        sw.spmm(ro, col, _cpu(8, dtype=torch.float16), _cpu(6, 3),
                _cpu(4, 3))


def test_csr_nnz_limit():
    """nnz is capped a little below INT32_MAX so that the row loops' int32
    position arithmetic (which steps past a row's end by less than 2^16)
    cannot overflow; the entry points reject larger nnz before any launch."""
    lib = sw.load_library()
    fake = ctypes.c_void_p(16)
    limit = 2**31 - 1 - 65536
    for nnz in (limit + 1, 2**31 - 1):
        rc = lib.sw_spmv_csr_f32(fake, fake, fake, fake, fake, 4, 4, nnz,
                                 None, None)
        assert rc == -2 and b"at most" in lib.sw_last_error()
        rc = lib.sw_spmm_csr_f32(fake, fake, fake, fake, fake, 4, 4, nnz, 4,
                                 None, None)
        assert rc == -2
        rc = lib.sw_sddmm_csr_bf16(fake, fake, fake, fake, fake, fake, 4, 4,
                                   nnz, 4, 0, 1.0, 0.0, None, None)
        assert rc == -2


def test_slab_floor_rejects_shapes_it_does_not_run():
    """sw_bsr_slab_floor runs where the MFMA kernels run: 16-byte aligned
    rhs and output, k % 4 (fp32) or k % 8 (bf16), and a known element
    width pair; anything else fails before a launch."""
    lib = sw.load_library()
    P = ctypes.c_void_p
    ok = P(64)
    args = (ok, ok, ok, ok, ok, 32, 32, 2)
    assert lib.sw_bsr_slab_floor(*args, 8, 4, 2, None) == -3   # fp32 / bf16
    assert lib.sw_bsr_slab_floor(*args, 8, 3, 3, None) == -3
    assert lib.sw_bsr_slab_floor(*args, 12, 2, 2, None) == -3  # bf16, k % 8
    assert b"multiple of 8" in lib.sw_last_error()
    assert lib.sw_bsr_slab_floor(ok, ok, ok, P(72), ok, 32, 32, 2, 8, 4, 4,
                                 None) == -3                  # rhs alignment
    assert lib.sw_bsr_slab_floor(ok, ok, ok, ok, ok, 30, 32, 2, 8, 4, 4,
                                 None) == -2                  # rows % 16

