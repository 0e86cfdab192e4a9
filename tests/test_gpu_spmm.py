"""GPU parity of sparsewave.spmm (thread-per-output, wave-per-row-tile,
thread-per-position) against the CPU oracle, per output element
|C - C_ref| <= 1e-5 * sum_p |a_rp * B[col_p, c]|."""
import numpy as np
import pytest

from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import assert_within_bound

pytestmark = pytest.mark.gpu

MAPPINGS = [
    "spmm-mapping=thread-per-output",
    "spmm-mapping=thread-per-output spmm-block-size=96",
    "spmm-mapping=wave-per-row-tile",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=1",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=2",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=3",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=8",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=16",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=32",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=4 spmm-lanes-per-row=16",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=4 spmm-lanes-per-row=4",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=32 spmm-lanes-per-row=8",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=5 spmm-block-size=128",
    "spmm-mapping=thread-per-position",
    "spmm-mapping=thread-per-position spmm-position-chunk-size=3",
    "spmm-mapping=wave-per-position",
    "spmm-mapping=wave-per-position spmm-positions-per-lane=1",
    "spmm-mapping=wave-per-position spmm-positions-per-lane=2 "
    "spmm-block-size=64",
    "spmm-mapping=wave-per-position spmm-positions-per-lane=8",
    "spmm-mapping=wave-per-position spmm-positions-per-lane=16 "
    "spmm-block-size=128",
    "spmm-mapping=row-tile-mfma",
    "spmm-mapping=wave-per-row-tile-lds",
    "spmm-mapping=wave-per-row-tile-lds spmm-tile-size=32",
    "spmm-mapping=wave-per-row-tile-lds spmm-tile-size=12",
    "spmm-mapping=wave-per-row-tile-lds spmm-tile-size=3",
    "spmm-mapping=wave-per-row-balanced",
    "spmm-mapping=wave-per-row-balanced spmm-positions-per-lane=1 "
    "spmm-block-size=64",
    # block sizes above the row-owner kernel's 256-thread launch bound
    "spmm-mapping=wave-per-row-balanced spmm-block-size=512",
    "spmm-mapping=wave-per-row-balanced spmm-block-size=1024",
]


@pytest.mark.parametrize("opts", ["spmm-mapping=row-tile-mfma",
                                  "spmm-mapping=wave-per-position"])
@pytest.mark.parametrize("k", [16, 64, 80, 8])
@pytest.mark.parametrize("block,window", [(64, 4), (16, 3), (32, 2)])
def test_block_structured(dev, orc, opts, k, block, window):
    """Block / causal masks: the 16-row tiles take the MFMA path (rows in a
    tile are prefixes of the tile's last row); a few rows are perturbed so
    some tiles fall back."""
    mask = W.attention_mask(seq=1024, block=block, window=window,
                            random_blocks=2, seed=block)
    vals = np.random.default_rng(k).uniform(-1, 1, mask.nnz).astype(
        np.float32)
    csr = W.CSR(mask.rows, mask.cols, mask.row_offsets,
                mask.column_indices.copy(), vals)
    # break the shared structure of a few tiles: drop the first column of
    # rows 37 and 500 (shift their entries left by one position)
    for r in (37, 500):
        a, b = csr.row_offsets[r], csr.row_offsets[r + 1]
        if b - a > 1:
            csr.column_indices[a:b - 1] = csr.column_indices[a + 1:b]
            csr.column_indices[b - 1] = min(csr.column_indices[b - 2] + 1,
                                            mask.cols - 1)
            if csr.column_indices[b - 1] <= csr.column_indices[b - 2]:
                csr.column_indices[b - 1] = csr.column_indices[b - 2]
    # keep columns strictly increasing inside each row
    ok = all(np.all(np.diff(csr.column_indices[a:b]) > 0) for a, b in
             zip(csr.row_offsets[:-1], csr.row_offsets[1:]))
    if not ok:
        pytest.skip("perturbation produced a duplicate column")
    rhs = np.random.default_rng(7).uniform(-1, 1, (mask.cols, k)).astype(
        np.float32)
    _check(orc, csr, rhs, G.spmm(csr, rhs, opts))


def _check(orc, csr, rhs, out):
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, rhs)
    assert_within_bound(out, ref, bound)


@pytest.mark.parametrize("opts", MAPPINGS)
@pytest.mark.parametrize("case", ["spmm", "spmm_torch_example"])
def test_golden(dev, golden, opts, case):
    g = golden[case]
    csr = W.CSR(g["rows"], g["cols"], np.array(g["row_offsets"], np.int32),
                np.array(g["column_indices"], np.int32),
                np.array(g["values"], np.float32))
    out = G.spmm(csr, np.array(g["rhs"], np.float32), opts)
    np.testing.assert_array_equal(out, np.array(g["expected"], np.float32))


@pytest.mark.parametrize("opts", MAPPINGS)
@pytest.mark.parametrize("k", [1, 4, 7, 64, 100])
def test_ragged(dev, orc, opts, k):
    csr = W.random_csr(700, 600, 15.0, k, empty_fraction=0.25,
                       max_len=600, lognormal=True)
    rhs = np.random.default_rng(k).uniform(-1, 1, (600, k)).astype(np.float32)
    _check(orc, csr, rhs, G.spmm(csr, rhs, opts))


@pytest.mark.parametrize("opts", ["spmm-mapping=row-tile-mfma",
                                  "spmm-mapping=thread-per-output"])
@pytest.mark.parametrize("k", [16, 64, 80])
def test_block_structured_non_finite_rhs(dev, orc, opts, k):
    """inf / NaN in B rows that the causal diagonal block of a 16-row tile
    names for its longer rows only: just the rows holding those entries are
    non-finite, as in the reference (the MFMA tiles that meet a non-finite
    output are recomputed row by row)."""
    mask = W.attention_mask(seq=512, block=64, window=3, random_blocks=1,
                            seed=5)
    rng = np.random.default_rng(k + 1)
    vals = rng.uniform(-1, 1, mask.nnz).astype(np.float32)
    csr = W.CSR(mask.rows, mask.cols, mask.row_offsets,
                mask.column_indices, vals)
    rhs = rng.uniform(-1, 1, (mask.cols, k)).astype(np.float32)
    rhs[70, 1] = np.inf       # diagonal block of rows 64..127: rows >= 70
    rhs[200, k - 1] = np.nan
    rhs[333, :] = -np.inf
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    out = G.spmm(csr, rhs, opts)
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(out), cls(ref))
    fin = np.isfinite(ref)
    assert (~fin).any() and fin[64:70].all()
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, np.nan_to_num(rhs, posinf=0,
                                                         neginf=0))
    assert_within_bound(out[fin], ref[fin], bound[fin])


@pytest.mark.parametrize("opts", MAPPINGS)
def test_non_finite_values(dev, orc, opts):
    """inf and NaN in the values and in B propagate per output element as in
    the reference's sequential sum (the class NaN / +inf / -inf does not
    depend on the order); finite elements meet the usual bound."""
    k = 8
    csr = W.random_csr(600, 500, 12.0, 12, empty_fraction=0.1, max_len=400,
                       lognormal=True)
    rng = np.random.default_rng(12)
    val = csr.values.copy()
    pick = rng.choice(csr.nnz, 24, replace=False)
    val[pick[:8]] = np.inf
    val[pick[8:16]] = -np.inf
    val[pick[16:]] = np.nan
    csr = W.CSR(csr.rows, csr.cols, csr.row_offsets, csr.column_indices, val)
    rhs = rng.uniform(-1, 1, (csr.cols, k)).astype(np.float32)
    rhs[rng.choice(csr.cols, 4, replace=False), rng.integers(0, k, 4)] = np.nan
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    out = G.spmm(csr, rhs, opts)
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(out), cls(ref))
    fin = np.isfinite(ref)
    assert (~fin).sum() > 20
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               np.where(np.isfinite(val), val, 0).astype(
                                   np.float32), np.nan_to_num(rhs))
    assert_within_bound(out[fin], ref[fin], bound[fin])


def test_rhs_past_four_gib(dev):
    """A 4 GiB+ right-hand side: kernels that address B with 32-bit byte
    offsets when 4 * rows(B) * K fits must take their 64-bit form here."""
    import torch
    import sparsewavecomp_amd as sw
    k = 64
    brows = (1 << 24) + 32          # 4 * brows * k > 2^32
    rng = np.random.default_rng(9)
    rows, per_row = 32, 8
    pool = np.concatenate([rng.choice(1 << 16, 16, replace=False),
                           (1 << 24) - 16 + np.arange(48)])
    rc = [np.sort(rng.choice(pool, per_row, replace=False)) for _ in range(rows)]
    col = np.concatenate(rc).astype(np.int32)
    ro = np.arange(0, rows * per_row + 1, per_row, dtype=np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    bp = rng.uniform(-1, 1, (pool.size, k)).astype(np.float32)
    rhs = torch.zeros((brows, k), dtype=torch.float32, device=G.DEV)
    rhs[G.t(pool.astype(np.int64))] = G.t(bp)
    where = {c: j for j, c in enumerate(pool.tolist())}
    bg = bp[[where[c] for c in col.tolist()]].astype(np.float64)
    prod = val.astype(np.float64)[:, None] * bg
    ref = prod.reshape(rows, per_row, k).sum(axis=1)
    bound = np.abs(prod).reshape(rows, per_row, k).sum(axis=1)
    for opts in ("spmm-mapping=thread-per-output",
                 "spmm-mapping=wave-per-row-tile spmm-tile-size=32",
                 "spmm-mapping=wave-per-position"):
        G.say(f"rhs of {brows} x {k}, {opts}")
        out = torch.full((rows, k), float("nan"), device=G.DEV)
        sw.spmm(G.t(ro), G.t(col), G.t(val), rhs, out, options=opts)
        torch.cuda.synchronize()
        assert_within_bound(out.cpu().numpy(), ref, bound)
    del rhs
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def config3():
    csr, _ = W.config2(seed=0)
    return csr


@pytest.mark.parametrize("k,opts", [
    (4, "spmm-mapping=wave-per-row-tile spmm-tile-size=4"),
    (4, "spmm-mapping=wave-per-row-tile spmm-tile-size=4 spmm-lanes-per-row=16"),
    (64, "spmm-mapping=wave-per-row-tile spmm-tile-size=32 spmm-lanes-per-row=16"),
    (4, "spmm-mapping=wave-per-position spmm-positions-per-lane=4 "
        "spmm-block-size=64"),
    (64, "spmm-mapping=wave-per-position spmm-positions-per-lane=8 "
         "spmm-block-size=64"),
    (64, "spmm-mapping=wave-per-row-balanced spmm-positions-per-lane=4 "
         "spmm-block-size=64"),
    (4, "spmm-mapping=wave-per-row-balanced spmm-positions-per-lane=4"),
    # the exact mappings bench.py times on configuration 3
    (4, ""),   # the reference's default, thread-per-output
    (64, ""),
    (4, "spmm-mapping=wave-per-position spmm-positions-per-lane=8 "
        "spmm-block-size=256"),
    (4, "spmm-mapping=wave-per-row-tile spmm-tile-size=4 "
        "spmm-block-size=64"),
    (4, "spmm-mapping=wave-per-row-tile-lds spmm-tile-size=4"),
    (64, "spmm-mapping=wave-per-position spmm-positions-per-lane=16 "
         "spmm-block-size=64"),
    (64, "spmm-mapping=wave-per-row-tile spmm-tile-size=32 "
         "spmm-lanes-per-row=64 spmm-block-size=64"),
    (64, "spmm-mapping=wave-per-row-tile-lds spmm-tile-size=32"),
])
def test_config3_full_size(dev, orc, config3, k, opts):
    csr = config3
    rhs = W.config3_rhs(csr.cols, k, seed=0)
    out = G.spmm(csr, rhs, opts)
    # full-size check on a row sample keeps the oracle within seconds
    rows = np.sort(np.random.default_rng(k).choice(csr.rows, 20000,
                                                   replace=False))
    rows = np.concatenate([rows, np.argsort(np.diff(csr.row_offsets))[-50:]])
    sub = _row_subset(csr, rows)
    _check(orc, sub, rhs, out[rows])
    assert np.all(np.isfinite(out))  # every row written (output NaN-filled)


def _row_subset(csr, rows):
    ro = csr.row_offsets
    lengths = (ro[rows + 1] - ro[rows]).astype(np.int64)
    new_ro = np.zeros(rows.size + 1, np.int64)
    np.cumsum(lengths, out=new_ro[1:])
    idx = np.concatenate([np.arange(ro[r], ro[r + 1]) for r in rows])
    return W.CSR(rows.size, csr.cols, new_ro.astype(np.int32),
                 csr.column_indices[idx], csr.values[idx])
