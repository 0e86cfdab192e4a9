"""Seeded fuzz of every SpMV, COO and SpMM mapping against the CPU oracle.

Each seed draws a ragged CSR matrix whose shape and row-length mix vary with
the seed: empty rows, runs of empty rows, rows of 1-3 entries, rows longer
than a wave's share of positions (up to 3000 entries), and a matrix width
from a few columns (dense rows) to thousands.  Every mapping of the op runs
on it (the option lists of tests/test_gpu_spmv.py and test_gpu_spmm.py), and
every output must meet the fp32 bound |y - y_ref| <= 1e-5 sum |a x|; SpMM
runs K of 1, 3, 4, 17 and 64.  The same matrices as COO (row-sorted and
shuffled, with repeated coordinates) check the COO kernels."""
import os

import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import assert_within_bound
from tests.test_gpu_spmm import MAPPINGS as SPMM_MAPPINGS
from tests.test_gpu_spmv import MAPPINGS as SPMV_MAPPINGS

pytestmark = pytest.mark.gpu

# SW_FUZZ_SEEDS=N runs seeds 0 .. N-1 instead (a longer one-off run)
SEEDS = list(range(int(os.environ.get("SW_FUZZ_SEEDS", "6"))))


def _matrix(seed):
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.integers(1, 2500))
    cols = int(rng.choice([7, 64, 900, 4000]))
    kind = rng.integers(0, 3, rows)
    lengths = np.where(kind == 0, 0,
                       np.where(kind == 1, rng.integers(1, 4, rows),
                                rng.integers(4, 80, rows)))
    # a few long rows and a run of empty rows
    for r in rng.choice(rows, min(rows, 3), replace=False):
        lengths[r] = int(rng.integers(300, 3001))
    if rows > 40:
        s = int(rng.integers(0, rows - 30))
        lengths[s:s + 30] = 0
    lengths = np.minimum(lengths, cols)
    return W.csr_from_lengths(rng, lengths, cols), rng


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_spmv_every_mapping(dev, orc, seed):
    csr, rng = _matrix(seed)
    x = rng.uniform(-1, 1, csr.cols).astype(np.float32)
    ref = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    for opts in SPMV_MAPPINGS:
        y = G.spmv(csr, x, opts)
        assert_within_bound(y, ref, bound, what=f"seed {seed} {opts}")


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_coo(dev, orc, seed):
    csr, rng = _matrix(seed)
    x = rng.uniform(-1, 1, csr.cols).astype(np.float32)
    ri = np.repeat(np.arange(csr.rows, dtype=np.int32),
                   np.diff(csr.row_offsets))
    ci, val = csr.column_indices, csr.values
    # a shuffled copy with repeated coordinates (the value split in two)
    dup = rng.random(ci.size) < 0.1
    ri2 = np.concatenate([ri, ri[dup]])
    ci2 = np.concatenate([ci, ci[dup]])
    half = val.copy()
    half[dup] *= 0.5
    val2 = np.concatenate([half, half[dup]]).astype(np.float32)
    perm = rng.permutation(ri2.size)
    for rows_i, cols_i, vals_i in ((ri, ci, val),
                                   (ri2[perm], ci2[perm], val2[perm])):
        # the oracle's own per-row bound sum |val * x| over the entries
        ref, bound = orc.spmv_coo(csr.rows, rows_i, cols_i, vals_i, x)
        for opts in ("", "spmv-mapping=wave-per-position "
                         "spmv-positions-per-lane=4 spmv-block-size=64",
                     "spmv-mapping=wave-per-position spmv-positions-per-lane=1"):
            G.say(f"fuzz coo seed {seed} nnz={rows_i.size} opts='{opts}'")
            y = torch.full((csr.rows,), float("nan"), device=G.DEV)
            sw.coo_spmv(G.t(rows_i), G.t(cols_i), G.t(vals_i), G.t(x), y,
                        options=opts or None)
            torch.cuda.synchronize()
            assert_within_bound(y.cpu().numpy(), ref, bound,
                                what=f"seed {seed} coo {opts}")


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("k", [1, 3, 4, 17, 64])
def test_fuzz_spmm_every_mapping(dev, orc, seed, k):
    csr, rng = _matrix(seed)
    rhs = rng.uniform(-1, 1, (csr.cols, k)).astype(np.float32)
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, rhs)
    for opts in SPMM_MAPPINGS:
        out = G.spmm(csr, rhs, opts)
        assert_within_bound(out, ref, bound, what=f"seed {seed} K={k} {opts}")
