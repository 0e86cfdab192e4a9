"""Host-side matrix files (native reader/writers in libsparsewave_amd.so).

The first cases restate the reference's own tests of its harness
(test/Benchmark/spmv_benchmark_test.py:115-200,
test/Benchmark/spmm_benchmark_test.py:25-96) with their inputs and expected
values; tests/golden/tiny.mtx is test/Benchmark/Inputs/tiny.mtx.  The rest
pin the native code against scipy.io's Matrix Market reader, dense numpy
block sums, byte-level layouts and round trips, and the error paths."""
import math
import os
import struct

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp

from sparsewavecomp_amd import formats as F

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _mtx(tmp_path, text, name="m.mtx"):
    p = tmp_path / name
    p.write_text(text, encoding="utf-8")
    return p


SPMM_MTX = """%%MatrixMarket matrix coordinate real general
2 3 3
1 1 1
1 3 2
2 2 3
"""


# ---- the reference's harness tests ----------------------------------------


def test_general_converts_to_csr(tmp_path):
    m = F.read_matrix_market(_mtx(tmp_path, """%%MatrixMarket matrix coordinate real general
% a rectangular matrix with an empty row
3 4 3
1 4 2.5
1 2 -1
3 1 4
"""))
    assert (m["rows"], m["columns"], m["nnz"]) == (3, 4, 3)
    assert m["row_offsets"].tolist() == [0, 2, 2, 3]
    assert m["row_indices"].tolist() == [0, 0, 2]
    assert m["column_indices"].tolist() == [1, 3, 0]
    assert m["values"].tolist() == [-1.0, 2.5, 4.0]
    assert (m["min_row_nnz"], m["max_row_nnz"]) == (0, 2)
    assert m["mean_row_nnz"] == 1.0
    assert (m["field"], m["symmetry"], m["name"]) == ("real", "general", "m")


def test_symmetric_pattern_expands_off_diagonal(tmp_path):
    m = F.read_matrix_market(_mtx(tmp_path, """%%MatrixMarket matrix coordinate pattern symmetric
3 3 3
1 1
2 1
3 2
"""))
    assert m["nnz"] == 5
    assert m["row_offsets"].tolist() == [0, 2, 4, 5]
    assert m["column_indices"].tolist() == [0, 1, 0, 2, 1]
    assert m["values"].tolist() == [1.0] * 5


def test_entry_count_is_validated(tmp_path):
    p = _mtx(tmp_path, """%%MatrixMarket matrix coordinate integer general
2 2 2
1 1 1
""")
    with pytest.raises(ValueError, match="file contains 1"):
        F.read_matrix_market(p)


def test_csr_binary_header_and_dimensions(tmp_path):
    m = F.read_matrix_market(_mtx(tmp_path, """%%MatrixMarket matrix coordinate real general
2 3 2
1 2 2
2 3 3
"""))
    F.write_csr_binary(tmp_path / "matrix.csr", m)
    b = (tmp_path / "matrix.csr").read_bytes()
    assert b[:8] == F.CSR_BINARY_MAGIC
    assert struct.unpack("<QQQ", b[8:32]) == (2, 3, 2)
    assert struct.unpack("<3i", b[32:44]) == (0, 1, 2)      # row offsets
    assert struct.unpack("<2i", b[44:52]) == (1, 2)         # columns
    assert struct.unpack("<2f", b[52:60]) == (2.0, 3.0)     # values
    assert len(b) == 60


def test_coo_binary_preserves_duplicate_coordinates(tmp_path):
    m = F.read_matrix_market(_mtx(tmp_path, """%%MatrixMarket matrix coordinate real general
2 3 3
1 2 2
1 2 3
2 3 4
"""))
    F.write_coo_binary(tmp_path / "matrix.coo", m)
    b = (tmp_path / "matrix.coo").read_bytes()
    assert b[:8] == F.COO_BINARY_MAGIC
    assert struct.unpack("<QQQ", b[8:32]) == (2, 3, 3)
    assert struct.unpack("<3i", b[32:44]) == (0, 0, 1)
    assert struct.unpack("<3i", b[44:56]) == (1, 1, 2)
    assert struct.unpack("<3f", b[56:68]) == (2.0, 3.0, 4.0)  # file order


def test_converts_to_padded_bsr(tmp_path):
    m = F.read_matrix_market(_mtx(tmp_path, SPMM_MTX))
    bsr = F.convert_to_bsr(m, block_size=2)
    assert (bsr["rows"], bsr["columns"]) == (2, 4)
    assert bsr["block_row_offsets"].tolist() == [0, 2]
    assert bsr["block_column_indices"].tolist() == [0, 1]
    assert bsr["block_values"].tolist() == [1.0, 0.0, 0.0, 3.0,
                                            2.0, 0.0, 0.0, 0.0]
    assert bsr["nnzb"] == 2
    assert bsr["block_density"] == 1.0
    assert bsr["internal_zero_fraction"] == 0.625
    assert bsr["storage_overhead"] == 8.0 / 3.0
    F.write_bsr_binary(tmp_path / "spmm.bsr", bsr)
    assert (tmp_path / "spmm.bsr").read_bytes()[:8] == F.BSR_BINARY_MAGIC


def test_bsr_conversion_coalesces_duplicate_coordinates(tmp_path):
    m = dict(F.read_matrix_market(_mtx(tmp_path, SPMM_MTX)))
    m["nnz"] = 4
    m["row_indices"] = [0, 0, 0, 1]
    m["column_indices"] = [0, 0, 2, 1]
    m["values"] = [1.0, 4.0, 2.0, 3.0]
    m["row_offsets"] = None
    bsr = F.convert_to_bsr(m, block_size=2)
    assert bsr["block_values"][0] == 5.0
    assert bsr["storage_overhead"] == 8.0 / 3.0


def test_tiny_fixture(tmp_path):
    m = F.read_matrix_market(os.path.join(GOLDEN, "tiny.mtx"))
    assert (m["rows"], m["columns"], m["nnz"]) == (4, 5, 6)
    assert m["row_offsets"].tolist() == [0, 2, 3, 5, 6]
    assert m["column_indices"].tolist() == [0, 3, 1, 0, 2, 4]
    # the harness's expected SpMV output: row sums (vector of ones)
    y = np.add.reduceat(m["values"], m["row_offsets"][:-1])
    assert y.tolist() == [1.0, 3.0, 9.0, 6.0]
    assert F.benchmark_vector(5).tolist() == [1.0] * 5


# ---- independent pins ------------------------------------------------------


@pytest.mark.parametrize("symmetric", [False, True])
def test_matches_scipy_mmread(tmp_path, symmetric):
    rng = np.random.default_rng(3 + symmetric)
    n = 60
    a = sp.random(n, n if symmetric else 45, density=0.1, random_state=rng,
                  format="coo")
    a.data = rng.uniform(-4, 4, a.nnz).round(3)
    if symmetric:
        a = sp.tril(a + a.T).tocoo()
        a = (a + sp.tril(a, -1).T).tocoo()
    p = tmp_path / "r.mtx"
    scipy.io.mmwrite(str(p), a, symmetry="symmetric" if symmetric else None)
    m = F.read_matrix_market(p)
    ref = scipy.io.mmread(str(p)).tocsr()
    ref.sort_indices()
    assert m["symmetry"] == ("symmetric" if symmetric else "general")
    assert m["row_offsets"].tolist() == ref.indptr.tolist()
    assert m["column_indices"].tolist() == ref.indices.tolist()
    np.testing.assert_array_equal(m["values"], ref.data)


def test_bsr_blocks_match_dense_sums():
    rng = np.random.default_rng(5)
    rows, cols, nnz, b = 37, 29, 400, 4
    ri = rng.integers(0, rows, nnz).astype(np.int32)
    ci = rng.integers(0, cols, nnz).astype(np.int32)
    val = rng.uniform(-1, 1, nnz)
    m = {"rows": rows, "columns": cols, "nnz": nnz, "row_indices": ri,
         "column_indices": ci, "values": val}
    bsr = F.convert_to_bsr(m, b)
    dense = np.zeros((40, 32))
    np.add.at(dense, (ri, ci), val)
    got = np.zeros_like(dense)
    bro, bcol = bsr["block_row_offsets"], bsr["block_column_indices"]
    blocks = bsr["block_values"].reshape(-1, b, b)
    for br in range(40 // b):
        cols_here = bcol[bro[br]:bro[br + 1]]
        assert np.all(np.diff(cols_here) > 0)   # sorted, distinct blocks
        for q in range(bro[br], bro[br + 1]):
            got[br * b:(br + 1) * b, bcol[q] * b:(bcol[q] + 1) * b] = blocks[q]
    np.testing.assert_allclose(got, dense, rtol=0, atol=1e-12)
    occupied = len({(r, c) for r, c in zip(ri.tolist(), ci.tolist())})
    assert bsr["nnzb"] == len({(r // b, c // b) for r, c in
                               zip(ri.tolist(), ci.tolist())})
    assert bsr["storage_overhead"] == bsr["nnzb"] * b * b / occupied
    assert bsr["block_density"] == bsr["nnzb"] / (10 * 8)


def test_binary_round_trips(tmp_path):
    rng = np.random.default_rng(6)
    a = sp.random(300, 200, density=0.05, random_state=rng, format="coo")
    p = tmp_path / "r.mtx"
    scipy.io.mmwrite(str(p), a)
    m = F.read_matrix_market(p)
    F.write_csr_binary(tmp_path / "r.csr", m)
    F.write_coo_binary(tmp_path / "r.coo", m)
    f32 = m["values"].astype(np.float32).astype(np.float64)
    for got in (F.read_csr_binary(tmp_path / "r.csr"),
                F.read_matrix(tmp_path / "r.csr"),
                F.read_coo_binary(tmp_path / "r.coo")):
        assert got["row_offsets"].tolist() == m["row_offsets"].tolist()
        assert got["row_indices"].tolist() == m["row_indices"].tolist()
        assert got["column_indices"].tolist() == m["column_indices"].tolist()
        np.testing.assert_array_equal(got["values"], f32)
        assert got["max_row_nnz"] == m["max_row_nnz"]
    bsr = F.convert_to_bsr(m, 8)
    F.write_bsr_binary(tmp_path / "r.bsr", bsr)
    back = F.read_bsr_binary(tmp_path / "r.bsr")
    for k in ("rows", "columns", "nnzb", "block_size", "original_rows",
              "original_columns", "nnz", "block_density",
              "internal_zero_fraction", "storage_overhead"):
        assert back[k] == bsr[k], k
    for k in ("block_row_offsets", "block_column_indices",
              "input_row_indices", "input_column_indices"):
        assert back[k].tolist() == bsr[k].tolist(), k
    np.testing.assert_array_equal(
        back["block_values"],
        bsr["block_values"].astype(np.float32).astype(np.float64))


def test_unsorted_coo_file_has_no_row_offsets(tmp_path):
    m = {"rows": 3, "columns": 3, "nnz": 3, "row_indices": [2, 0, 1],
         "column_indices": [0, 1, 2], "values": [1.0, 2.0, 3.0]}
    F.write_coo_binary(tmp_path / "u.coo", m)
    got = F.read_coo_binary(tmp_path / "u.coo")
    assert got["row_offsets"] is None
    assert got["row_indices"].tolist() == [2, 0, 1]


def test_rhs_formula():
    b = F.benchmark_rhs(9, 3)
    assert b[0].tolist() == [1.0, 1.125, 1.25]
    assert b[6].tolist() == [1.75, 1.0, 1.125]
    assert b.dtype == np.float32


# ---- errors ----------------------------------------------------------------


HEADER = "%%MatrixMarket matrix coordinate real general\n"


@pytest.mark.parametrize("text,error", [
    ("%%MatrixMarket matrix array real general\n2 2\n", "coordinate matrix"),
    ("%%MatrixMarket matrix coordinate complex general\n1 1 0\n",
     "unsupported Matrix Market field 'complex'"),
    ("%%MatrixMarket matrix coordinate real hermitian\n1 1 0\n",
     "unsupported Matrix Market symmetry 'hermitian'"),
    (HEADER + "% only comments\n", "missing matrix dimensions"),
    (HEADER + "2 2\n", "invalid matrix dimensions"),
    (HEADER + "2 x 1\n", "invalid matrix dimensions"),
    (HEADER + "0 2 0\n", "must be nonnegative"),
    ("%%MatrixMarket matrix coordinate real symmetric\n2 3 0\n",
     "must be square"),
    (HEADER + "2 2 1\n1 1\n", ":3: expected 3 fields"),
    (HEADER + "2 2 1\n1 1 abc\n", ":3: invalid matrix entry"),
    (HEADER + "2 2 1\n1 1 0x10\n", ":3: invalid matrix entry"),
    (HEADER + "2 2 1\n% c\n3 1 1\n", ":4: matrix index is out of bounds"),
    (HEADER + "2 2 1\n0 1 1\n", "matrix index is out of bounds"),
    (HEADER + "2 2 1\n1 1 nan\n", "value must be finite"),
    (HEADER + "2 2 1\n1 1 inf\n", "value must be finite"),
    (HEADER + "2 2 1\n1 1 1e39\n", "must fit in f32"),
    ("%%MatrixMarket matrix coordinate integer general\n2 2 1\n1 1 1.5\n",
     "invalid matrix entry"),
])
def test_matrix_market_errors(tmp_path, text, error):
    with pytest.raises(ValueError, match=error):
        F.read_matrix_market(_mtx(tmp_path, text))


def test_integer_and_case_insensitive_field(tmp_path):
    m = F.read_matrix_market(_mtx(tmp_path, """%%MatrixMarket matrix coordinate INTEGER General
2 2 2

2 2 -7
1 2 +3
"""))
    assert m["values"].tolist() == [3.0, -7.0]
    assert m["field"] == "integer"


def test_binary_errors(tmp_path):
    p = tmp_path / "bad.csr"
    p.write_bytes(b"SWCSR002" + struct.pack("<QQQ", 1, 1, 0))
    with pytest.raises(ValueError, match="invalid CSR binary header"):
        F.read_csr_binary(p)
    p.write_bytes(F.CSR_BINARY_MAGIC + struct.pack("<QQQ", 2, 2, 2)
                  + struct.pack("<3i", 0, 1, 2))
    with pytest.raises(ValueError, match="could not read column indices"):
        F.read_csr_binary(p)
    p.write_bytes(F.CSR_BINARY_MAGIC + struct.pack("<QQQ", 2, 2, 2)
                  + struct.pack("<3i", 0, 1, 2) + struct.pack("<2i", 0, 2)
                  + struct.pack("<2f", 1, 1))
    with pytest.raises(ValueError, match="column index 2 at position 1"):
        F.read_csr_binary(p)
    p.write_bytes(F.CSR_BINARY_MAGIC + struct.pack("<QQQ", 2, 2, 2)
                  + struct.pack("<3i", 0, 2, 1) + struct.pack("<2i", 0, 1)
                  + struct.pack("<2f", 1, 1))
    with pytest.raises(ValueError, match="run from 0 to 2"):
        F.read_csr_binary(p)
    q = tmp_path / "bad.coo"
    q.write_bytes(F.COO_BINARY_MAGIC + struct.pack("<QQQ", 2, 2, 1)
                  + struct.pack("<i", 2) + struct.pack("<i", 0)
                  + struct.pack("<f", 1))
    with pytest.raises(ValueError, match="COO coordinate is out of bounds"):
        F.read_coo_binary(q)
    r = tmp_path / "bad.bsr"
    r.write_bytes(F.BSR_BINARY_MAGIC + struct.pack("<7Q", 3, 4, 0, 2, 3, 4, 0))
    with pytest.raises(ValueError, match="divisible by a positive block size"):
        F.read_bsr_binary(r)
    r.write_bytes(F.BSR_BINARY_MAGIC + struct.pack("<7Q", 4, 4, 0, 2, 5, 4, 0))
    with pytest.raises(ValueError, match="exceed the padded dimensions"):
        F.read_bsr_binary(r)
    with pytest.raises(ValueError, match="block size must be positive"):
        F.convert_to_bsr({"rows": 1, "columns": 1, "nnz": 0}, 0)
    with pytest.raises(ValueError, match="could not open"):
        F.read_matrix_market(tmp_path / "missing.mtx")
    big = {"rows": 1, "columns": 1, "nnz": 1, "row_offsets": [0, 1],
           "row_indices": [0], "column_indices": [0], "values": [1e39]}
    with pytest.raises(ValueError, match="must fit in f32"):
        F.write_csr_binary(tmp_path / "big.csr", big)
    assert math.isfinite(F.read_matrix_market(
        os.path.join(GOLDEN, "tiny.mtx"))["mean_row_nnz"])


@pytest.mark.parametrize("kind", ["csr", "coo", "bsr"])
def test_every_truncation_is_rejected(tmp_path, kind):
    """A binary cut short at any byte is an error, never a shorter matrix:
    the native readers check the length of every section they read."""
    m = F.read_matrix_market(os.path.join(GOLDEN, "tiny.mtx"))
    p = tmp_path / f"full.{kind}"
    if kind == "csr":
        F.write_csr_binary(p, m)
        read = F.read_csr_binary
    elif kind == "coo":
        F.write_coo_binary(p, m)
        read = F.read_coo_binary
    else:
        F.write_bsr_binary(p, F.convert_to_bsr(m, 2))
        read = F.read_bsr_binary
    data = p.read_bytes()
    read(p)
    q = tmp_path / f"cut.{kind}"
    for n in range(len(data)):
        q.write_bytes(data[:n])
        with pytest.raises(ValueError):
            read(q)
