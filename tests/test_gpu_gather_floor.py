"""The gather-floor diagnostic (sw_spmv_gather_floor_f32): every 512-entry
chunk's sum of values[p] * vector[column_indices[p]] against a float64 numpy
sum.  The kernel adds 8 entries per lane in order, then the 64 lane sums in a
tree, so its fp32 error stays far inside 1e-5 * sum |v * x| per chunk.

It is not a reference op: it measures the column/value reads and x gathers
that every SpMV schedule performs, and bench.py times it beside the SpMV."""
import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from tests import gpu_util as G
from tests._check import assert_within_bound

pytestmark = pytest.mark.gpu


def _expected(col, val, x):
    prod = val.astype(np.float64) * x[col].astype(np.float64)
    n = (len(val) + 511) // 512
    pad = np.zeros(n * 512 - len(val))
    chunks = np.concatenate([prod, pad]).reshape(n, 512)
    absc = np.concatenate([np.abs(prod), pad]).reshape(n, 512)
    return chunks.sum(axis=1), absc.sum(axis=1)


@pytest.mark.parametrize("nnz,offset", [(1, 0), (7, 0), (512, 0), (513, 0),
                                        (100_003, 0), (100_003, 1),
                                        (1 << 20, 0), (1 << 20, 3)])
def test_gather_floor_chunks(dev, nnz, offset):
    rng = np.random.default_rng(nnz + offset)
    m = 50_000
    col = rng.integers(0, m, nnz).astype(np.int32)
    val = rng.uniform(-1, 1, nnz).astype(np.float32)
    x = rng.uniform(-1, 1, m).astype(np.float32)
    G.say(f"gather floor nnz={nnz} offset={offset}")
    # offset > 0 starts col/val off a 16-byte boundary (the scalar path)
    pad = lambda a: G.t(np.concatenate([np.zeros(offset, a.dtype), a]))[offset:]
    n = (nnz + 511) // 512
    part = torch.full((n,), float("nan"), device=G.DEV)
    sw.spmv_gather_floor(pad(col), pad(val), G.t(x), part)
    torch.cuda.synchronize()
    ref, bound = _expected(col, val, x)
    assert_within_bound(part.cpu().numpy(), ref, bound, what="partial sums")


def test_gather_floor_rejects_short_partial(dev):
    col = G.t(np.zeros(1024, np.int32))
    val = G.t(np.ones(1024, np.float32))
    x = G.t(np.ones(4, np.float32))
    with pytest.raises(sw.SparseWaveError):
        sw.spmv_gather_floor(col, val, x, torch.empty(1, device=G.DEV))
