"""The reference harness's path on the GPU: a Matrix Market file is read by
the native loader, converted (CSR / COO / padded BSR), moved to HBM and run
through the HIP kernels with the harness's operands (vector of ones,
rhs = 1 + ((row + column) mod 7) / 8), then checked against the oracle and,
for tiny.mtx (test/Benchmark/Inputs/tiny.mtx), against the harness's exact
expectation (row sums)."""
import os

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import formats as F
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import assert_within_bound

pytestmark = pytest.mark.gpu

TINY = os.path.join(os.path.dirname(__file__), "golden", "tiny.mtx")

SPMV = ["spmv-mapping=thread-per-row", "spmv-mapping=wave-per-row",
        "spmv-mapping=block-per-row spmv-block-size=128",
        "spmv-mapping=thread-per-position",
        "spmv-mapping=wave-per-position spmv-positions-per-lane=4"]


def _csr(m):
    return W.CSR(m["rows"], m["columns"], m["row_offsets"],
                 m["column_indices"], m["values"].astype(np.float32))


@pytest.mark.parametrize("opts", SPMV)
def test_tiny_spmv_exact(dev, opts):
    m = F.read_matrix_market(TINY)
    y = G.spmv(_csr(m), F.benchmark_vector(m["columns"]), opts)
    np.testing.assert_array_equal(y, np.array([1, 3, 9, 6], np.float32))


@pytest.mark.parametrize("opts", ["", "spmv-mapping=wave-per-position "
                                      "spmv-positions-per-lane=4"])
def test_tiny_coo_binary_exact(dev, tmp_path, opts):
    m = F.read_matrix_market(TINY)
    F.write_coo_binary(tmp_path / "t.coo", m)
    c = F.read_coo_binary(tmp_path / "t.coo")
    G.say(f"coo_spmv tiny opts='{opts}'")
    y = torch.full((c["rows"],), float("nan"), device=G.DEV)
    sw.coo_spmv(G.t(c["row_indices"]), G.t(c["column_indices"]),
                G.t(c["values"].astype(np.float32)),
                G.t(F.benchmark_vector(c["columns"])), y, options=opts or None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(),
                                  np.array([1, 3, 9, 6], np.float32))


@pytest.fixture(scope="module")
def random_mtx(tmp_path_factory):
    rng = np.random.default_rng(21)
    a = sp.random(2000, 1500, density=0.01, random_state=rng, format="coo")
    a.data = rng.uniform(-1, 1, a.nnz)
    p = tmp_path_factory.mktemp("mm") / "r.mtx"
    scipy.io.mmwrite(str(p), a)
    return F.read_matrix_market(p)


@pytest.mark.parametrize("opts", SPMV)
def test_matrix_market_spmv(dev, orc, random_mtx, opts):
    csr = _csr(random_mtx)
    x = F.benchmark_vector(csr.cols)
    y = G.spmv(csr, x, opts)
    ref = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    assert_within_bound(y, ref, orc.spmv_abs_bound(
        csr.row_offsets, csr.column_indices, csr.values, x))


@pytest.mark.parametrize("opts", [
    "spmm-mapping=thread-per-output",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=4",
    "spmm-mapping=wave-per-position spmm-positions-per-lane=8"])
def test_matrix_market_spmm(dev, orc, random_mtx, opts):
    csr = _csr(random_mtx)
    rhs = F.benchmark_rhs(csr.cols, 4)
    out = G.spmm(csr, rhs, opts)
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    assert_within_bound(out, ref, orc.spmm_abs_bound(
        csr.row_offsets, csr.column_indices, csr.values, rhs))


@pytest.mark.parametrize("b,opts", [(2, "bsr-use-mfma=0"), (16, ""),
                                    (16, "bsr-use-mfma=0")])
def test_matrix_market_bsr(dev, orc, tmp_path, random_mtx, b, opts):
    bsr = F.convert_to_bsr(random_mtx, b)
    F.write_bsr_binary(tmp_path / "r.bsr", bsr)
    bsr = F.read_bsr_binary(tmp_path / "r.bsr")
    k = 16
    rhs = F.benchmark_rhs(bsr["columns"], k)
    bval = bsr["block_values"].astype(np.float32)
    G.say(f"bsr_spmm from mtx b={b} nnzb={bsr['nnzb']} opts='{opts}'")
    out = torch.full((bsr["rows"], k), float("nan"), device=G.DEV)
    sw.bsr_spmm(G.t(bsr["block_row_offsets"]),
                G.t(bsr["block_column_indices"]), G.t(bval), G.t(rhs), out, b,
                options=opts or None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = orc.bsr_spmm(bsr["block_row_offsets"], bsr["block_column_indices"],
                       bval, rhs, b)
    bound = orc.bsr_abs_bound(bsr["block_row_offsets"],
                              bsr["block_column_indices"], bval, rhs, b)
    assert_within_bound(got, ref, bound)
    # the harness's expectation from the original COO entries
    # (benchmark/SparseBenchmarkUtils.cpp:313-324), in float64
    exp = np.zeros((bsr["rows"], k))
    np.add.at(exp, bsr["input_row_indices"],
              bsr["input_values"][:, None] *
              rhs[bsr["input_column_indices"]].astype(np.float64))
    assert_within_bound(got, exp, bound)
