"""The rocSPARSE comparison runner computes the same products (so the bench
compares like with like)."""
import numpy as np
import pytest
import torch

from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import assert_within_bound

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("alg", ["default", "csr_adaptive", "csr_lrb",
                                 "csr_rowsplit"])
def test_rocsparse_spmv(dev, orc, alg):
    from sparsewavecomp_amd.rocsparse_runner import RocSparse
    csr = W.random_csr(4000, 3000, 25.0, 3, empty_fraction=0.1,
                       lognormal=True, max_len=3000)
    x = np.random.default_rng(3).uniform(-1, 1, 3000).astype(np.float32)
    # rocSPARSE computes alpha*A*x + beta*y and some algorithms (LRB) read y
    # even for beta = 0, so y starts at zero rather than NaN
    y = torch.zeros(csr.rows, device=G.DEV)
    G.say(f"rocsparse spmv {alg}")
    rs = RocSparse()
    run = rs.spmv(G.t(csr.row_offsets), G.t(csr.column_indices),
                  G.t(csr.values), G.t(x), y, alg=alg)
    run()
    torch.cuda.synchronize()
    ref = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    assert_within_bound(y.cpu().numpy(), ref, bound)


@pytest.mark.parametrize("alg", ["default", "csr_merge"])
def test_rocsparse_spmm(dev, orc, alg):
    from sparsewavecomp_amd.rocsparse_runner import RocSparse
    csr = W.random_csr(2000, 1500, 20.0, 4, empty_fraction=0.1)
    rhs = np.random.default_rng(4).uniform(-1, 1, (1500, 8)).astype(
        np.float32)
    out = torch.zeros((csr.rows, 8), device=G.DEV)
    G.say(f"rocsparse spmm {alg}")
    rs = RocSparse()
    run = rs.spmm(G.t(csr.row_offsets), G.t(csr.column_indices),
                  G.t(csr.values), G.t(rhs), out, alg=alg)
    run()
    torch.cuda.synchronize()
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, rhs)
    assert_within_bound(out.cpu().numpy(), ref, bound)
