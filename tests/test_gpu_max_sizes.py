"""SpMV, SpMM and the row ops at the largest sizes the entry points accept.

1. nnz at the cap of the CSR entry points.  check_csr caps nnz at
   INT32_MAX - 2^16 (the row loops step a 32-bit position past a row's end
   by less than 2^16, so no position they compute overflows; test_capi.py
   checks that one more is refused).  2^21 rows of 1023 or 1024 entries and
   an empty last row put the last positions within 2^16 of 2^31 and the
   byte offsets of the column and value arrays past 8 GiB (every kernel's
   64-bit form).  The position SpMMs then launch more than 2^32 - 1
   work-items (thread-per-position at K = 4: 8.6e9; wave-per-position at
   K = 64: 4.3e9), which the launchers fold into (x, y) grids: a 1-D launch
   that large is cut short without an error, and the last rows of the
   output were left unwritten before the fold.
2. Rows past one grid dimension: 2^26 + 2^20 rows put wave-per-row and
   block-per-row SpMV (64 work-items per row) and the wave row reduction and
   row-wise map past 2^32 - 1 work-items too.
3. COO past 2^31 entries (coo_spmv has no nnz cap: each entry carries its
   row), through the reference's kernel and the run-segmented one.
4. BSR past 8.4 million block rows, where the matrix-core kernels' 1-D x
   ends and the thread-per-output kernel takes over (fp32 and bf16).

Values, x and the right-hand sides are ones (the map's row values zero), so
every product output is a row length, exact in fp32, and every mapping must
reproduce it bit for bit; the map gives one value, exp(1), at every entry.
Device memory: about 17 GiB for the first case (25 GiB with the bf16 SpMM),
1 GiB for the second, 43 GiB at the peak of the third, 13 GiB for the
fourth.
"""
import pytest
import torch

import sparsewavecomp_amd as sw
from tests import gpu_util as G
from tests.test_gpu_spmv import MAPPINGS as SPMV_MAPPINGS

pytestmark = pytest.mark.gpu

LIMIT = 2**31 - 1 - 65536
ROWS = (1 << 21) + 1
COLS = 1 << 16

SPMM_MAPPINGS = [
    ("spmm-mapping=thread-per-output", 4),
    ("spmm-mapping=wave-per-row-tile spmm-tile-size=4 spmm-block-size=64", 4),
    ("spmm-mapping=wave-per-row-tile spmm-tile-size=4 spmm-lanes-per-row=16",
     4),
    ("spmm-mapping=thread-per-position", 4),
    ("spmm-mapping=wave-per-position spmm-positions-per-lane=8 "
     "spmm-block-size=256", 4),
    ("spmm-mapping=wave-per-position spmm-positions-per-lane=8 "
     "spmm-block-size=256", 64),
    ("spmm-mapping=wave-per-row-tile spmm-tile-size=32 spmm-lanes-per-row=64 "
     "spmm-block-size=64", 64),
]


@pytest.fixture(scope="module")
def big(dev):
    lengths = torch.full((ROWS,), 1024, dtype=torch.int64, device=G.DEV)
    lengths[:65537] = 1023
    lengths[-1] = 0  # an empty last row: its offsets both equal nnz
    ro = torch.zeros(ROWS + 1, dtype=torch.int64, device=G.DEV)
    ro[1:] = torch.cumsum(lengths, 0)
    nnz = int(ro[-1])
    assert nnz == LIMIT
    col = torch.arange(nnz, dtype=torch.int32, device=G.DEV)
    col.remainder_(COLS)
    val = torch.ones(nnz, dtype=torch.float32, device=G.DEV)
    yield ro.to(torch.int32), col, val, lengths.to(torch.float32)
    del col, val
    torch.cuda.empty_cache()


@pytest.mark.parametrize("opts", SPMV_MAPPINGS)
def test_spmv_at_the_nnz_limit(big, opts):
    ro, col, val, want = big
    x = torch.ones(COLS, dtype=torch.float32, device=G.DEV)
    G.say(f"spmv nnz={LIMIT} rows={ROWS} opts='{opts}'")
    y = torch.full((ROWS,), float("nan"), device=G.DEV)
    sw.spmv(ro, col, val, x, y, options=opts)
    torch.cuda.synchronize()
    assert torch.equal(y, want)


@pytest.mark.parametrize("opts,k", SPMM_MAPPINGS)
def test_spmm_at_the_nnz_limit(big, opts, k):
    ro, col, val, want = big
    rhs = torch.ones((COLS, k), dtype=torch.float32, device=G.DEV)
    G.say(f"spmm nnz={LIMIT} rows={ROWS} k={k} opts='{opts}'")
    out = torch.full((ROWS, k), float("nan"), device=G.DEV)
    sw.spmm(ro, col, val, rhs, out, options=opts)
    torch.cuda.synchronize()
    assert torch.equal(out, want[:, None].expand(ROWS, k))


MANY_ROWS = (1 << 26) + (1 << 20)


@pytest.fixture(scope="module")
def many_rows(dev):
    """MANY_ROWS rows alternating between 0 and 1 entries."""
    lengths = (torch.arange(MANY_ROWS, device=G.DEV) % 2).to(torch.int64)
    ro = torch.zeros(MANY_ROWS + 1, dtype=torch.int64, device=G.DEV)
    ro[1:] = torch.cumsum(lengths, 0)
    nnz = int(ro[-1])
    col = torch.arange(nnz, dtype=torch.int32, device=G.DEV)
    col.remainder_(COLS)
    val = torch.ones(nnz, dtype=torch.float32, device=G.DEV)
    yield ro.to(torch.int32), col, val, lengths.to(torch.float32)
    del col, val
    torch.cuda.empty_cache()


@pytest.mark.parametrize("opts", [
    "spmv-mapping=block-per-row spmv-block-size=64",
    "spmv-mapping=wave-per-row spmv-block-size=64",
    "spmv-mapping=wave-per-row spmv-lanes-per-row=32",
    "spmv-mapping=thread-per-row",
    "spmv-mapping=wave-per-position spmv-positions-per-lane=4 "
    "spmv-block-size=64",
])
def test_spmv_rows_past_one_grid_dimension(many_rows, opts):
    ro, col, val, want = many_rows
    x = torch.ones(COLS, dtype=torch.float32, device=G.DEV)
    G.say(f"spmv rows={MANY_ROWS} opts='{opts}'")
    y = torch.full((MANY_ROWS,), float("nan"), device=G.DEV)
    sw.spmv(ro, col, val, x, y, options=opts)
    torch.cuda.synchronize()
    assert torch.equal(y, want)


def test_row_ops_rows_past_one_grid_dimension(many_rows):
    """The wave row reduction (64 work-items a row) and the wave row-wise
    map: row sums are the lengths, and exp(1 - 0) is the same value (e to
    fp32 accuracy) at every entry."""
    ro, col, val, want = many_rows
    opts = "sddmm-lanes-per-row=64"
    G.say(f"row reduce / row-wise map rows={MANY_ROWS} opts='{opts}'")
    s = torch.full((MANY_ROWS,), float("nan"), device=G.DEV)
    sw.csr_row_reduce(ro, col, val, s, kind="sum", options=opts)
    torch.cuda.synchronize()
    assert torch.equal(s, want)
    zero = torch.zeros(MANY_ROWS, dtype=torch.float32, device=G.DEV)
    out = torch.full_like(val, float("nan"))
    sw.csr_rowwise_map(ro, col, val, zero, out, kind=sw.MAP_EXP_SUB,
                       options=opts)
    torch.cuda.synchronize()
    # every entry the same value, expf(1) within an ulp of e
    assert torch.equal(out, out[:1].expand_as(out))
    assert abs(float(out[0]) - 2.718281828459045) <= 2.4e-7


@pytest.mark.parametrize("opts", [
    "spmm-mapping=thread-per-output",
    "spmm-mapping=wave-per-row-tile spmm-tile-size=4 spmm-block-size=64",
])
def test_bf16_spmm_at_the_nnz_limit(big, opts):
    """The bf16 SpMM (every value buffer bf16, fp32 sums, one rounding) at
    the nnz cap: row lengths 1023 and 1024 both round to 1024 in bf16 (8
    significant bits), the empty last row to 0."""
    ro, col, _, want = big
    k = 4
    val = torch.ones(LIMIT, dtype=torch.bfloat16, device=G.DEV)
    rhs = torch.ones((COLS, k), dtype=torch.bfloat16, device=G.DEV)
    G.say(f"bf16 spmm nnz={LIMIT} rows={ROWS} k={k} opts='{opts}'")
    out = torch.full((ROWS, k), float("nan"), dtype=torch.bfloat16,
                     device=G.DEV)
    sw.spmm(ro, col, val, rhs, out, options=opts)
    torch.cuda.synchronize()
    expect = want.to(torch.bfloat16)[:, None].expand(ROWS, k)
    assert float(expect[0, 0]) == 1024.0 and float(expect[-1, 0]) == 0.0
    assert torch.equal(out, expect)
    del val
    torch.cuda.empty_cache()


@pytest.mark.parametrize("opts", [
    None,  # the reference's thread-per-nonzero kernel
    "spmv-mapping=wave-per-position spmv-positions-per-lane=4 "
    "spmv-block-size=64",
])
def test_coo_past_two_to_the_31_entries(dev, opts):
    """COO entries carry their row, so coo_spmv has no nnz cap: 2^31 + 2^20
    row-sorted entries (rows of 1024, past every 32-bit position), their
    positions and byte offsets 64-bit in both kernels.  Values and x are
    ones: each row sums to 1024 exactly."""
    nnz = (1 << 31) + (1 << 20)
    rows = nnz // 1024
    p = torch.arange(nnz, dtype=torch.int64, device=G.DEV)
    ri = torch.div(p, 1024, rounding_mode="floor").to(torch.int32)
    col = p.remainder_(COLS).to(torch.int32)
    del p
    val = torch.ones(nnz, dtype=torch.float32, device=G.DEV)
    x = torch.ones(COLS, dtype=torch.float32, device=G.DEV)
    G.say(f"coo nnz={nnz} rows={rows} opts='{opts}'")
    y = torch.full((rows,), float("nan"), device=G.DEV)
    sw.coo_spmv(ri, col, val, x, y, options=opts)
    torch.cuda.synchronize()
    assert torch.equal(y, torch.full_like(y, 1024.0))
    del ri, col, val
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_bsr_block_rows_past_the_matrix_core_grid(dev, dt):
    """The BSR matrix-core kernels index block rows by blockIdx.x alone, so
    past 2^32 - 1 work-items in x (about 8.4 million block rows) the BSR
    SpMM takes its thread-per-output kernel, whose launch folds.  Here
    2^23 + 2^16 block rows of one 16 x 16 block of ones on the diagonal,
    times a right-hand side of ones (K = 4): every output is 16, exact in
    fp32 and in bf16."""
    nbr = (1 << 23) + (1 << 16)
    rows, k = nbr * 16, 4
    bro = torch.arange(nbr + 1, dtype=torch.int32, device=G.DEV)
    bcol = torch.arange(nbr, dtype=torch.int32, device=G.DEV)
    bval = torch.ones(nbr * 256, dtype=dt, device=G.DEV)
    rhs = torch.ones((rows, k), dtype=dt, device=G.DEV)
    out = torch.full((rows, k), float("nan"), dtype=dt, device=G.DEV)
    G.say(f"bsr block rows={nbr} dtype={dt}")
    sw.bsr_spmm(bro, bcol, bval, rhs, out, block_size=16)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.full_like(out, 16.0))
    del bval, rhs, out
    torch.cuda.empty_cache()
