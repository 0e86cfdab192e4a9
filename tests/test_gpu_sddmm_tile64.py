"""The thread-per-row SDDMM's 64-row wave tiles against the CPU oracle.

With the reference's thread-per-row mapping, workgroups of whole waves up to
256 work-items and kdim 64 or 128, each wave first tries its 64 consecutive
rows as one matrix-core tile: its structure check reads every column index
of the tile (16-byte windows, each kept inside the tile's positions) and
accepts the tile when every row's columns are a prefix of its last row's,
which holds at most 512 entries and at least 4; other tiles run one row per
work-item.  The masks here are built from 64-row tiles of each kind the
check tells apart:
* prefix tiles with last rows of 1 .. 513 entries (1-3 and 513 take the
  rows' own path), leading rows empty or full;
* prefix tiles with one row's first or last column replaced, or one row
  longer than the last (the check fails);
* tiles of empty rows and of independent random rows;
and the matrix ends in a prefix tile whose last row holds 4 entries (its
windows clamped at the arrays' end), 2 entries, or in a partial tile of 37
rows.  fp32 within the op bar (1e-5 sum |terms|), bf16 within the fp32 bar
plus one rounding and rel-L2 <= 1e-2, for every combine kind."""
import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import assert_within_bound
from tests.test_gpu_bf16 import _sddmm, _sddmm_check

pytestmark = pytest.mark.gpu

COLS = 1500
LAST_LENGTHS = [1, 2, 3, 4, 5, 15, 16, 17, 63, 64, 65, 255, 256, 257, 383,
                384, 511, 512, 513]
# thread-per-row in whole-wave workgroups of 256, 128 and 64 work-items
OPTS = ["", "sddmm-block-size=128", "sddmm-block-size=64"]


def _prefix_tile(rng, nt, last, leading_empty=False, full=False):
    base = np.sort(rng.choice(COLS, last, replace=False))
    if full:
        lens = np.full(nt, last)
    else:
        lens = np.sort(rng.integers(0 if leading_empty else 1, last + 1, nt))
        lens[-1] = last
    return [base[:n].copy() for n in lens], base


def _tile64_mask(seed, ending):
    """(csr with U(-1, 1) values, rng)."""
    rng = np.random.default_rng(4000 + seed)
    rows_cols = []
    for k, last in enumerate(LAST_LENGTHS):
        tile, _ = _prefix_tile(rng, 64, last, leading_empty=k % 3 == 1,
                               full=k % 3 == 2)
        rows_cols += tile
    for change in ("first", "last", "longer"):
        tile, base = _prefix_tile(rng, 64, 300)
        others = np.setdiff1d(np.arange(COLS), base)
        r = int(rng.integers(1, 62))
        if change == "longer":
            tile[r] = np.sort(np.concatenate(
                [base, rng.choice(others, 5, replace=False)]))
        elif tile[r].size:
            at = 0 if change == "first" else tile[r].size - 1
            tile[r][at] = rng.choice(others)
        else:
            tile[r] = np.array([rng.choice(others)])
        rows_cols += tile
    rows_cols += [np.zeros(0, np.int64) for _ in range(64)]
    rows_cols += [np.sort(rng.choice(COLS, int(rng.integers(0, 200)),
                                     replace=False)) for _ in range(64)]
    if ending == "last4":
        rows_cols += _prefix_tile(rng, 64, 4, full=True)[0]
    elif ending == "last2":
        rows_cols += _prefix_tile(rng, 64, 2)[0]
    else:
        rows_cols += _prefix_tile(rng, 37, 200)[0]
    lengths = np.array([c.size for c in rows_cols])
    ro = np.zeros(len(rows_cols) + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(rows_cols).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    return W.CSR(len(rows_cols), COLS, ro, col, val), rng


@pytest.mark.parametrize("ending", ["last4", "last2", "partial"])
@pytest.mark.parametrize("kdim", [64, 128])
def test_sddmm_wave_tiles_f32(dev, orc, kdim, ending):
    csr, rng = _tile64_mask(kdim, ending)
    lhs = rng.standard_normal((csr.rows, kdim)).astype(np.float32)
    rhs = rng.standard_normal((kdim, csr.cols)).astype(np.float32)
    rows = np.repeat(np.arange(csr.rows), np.diff(csr.row_offsets))
    absd = (np.abs(lhs.astype(np.float64)) @ np.abs(rhs.astype(np.float64)))[
        rows, csr.column_indices]
    v = np.abs(csr.values.astype(np.float64))
    for kind in (sw.SDDMM_MUL, sw.SDDMM_AFFINE, sw.SDDMM_DOT):
        ref = orc.sddmm(csr.row_offsets, csr.column_indices, csr.values, lhs,
                        rhs, kind, 0.3, 0.7)
        bound = {sw.SDDMM_MUL: v * absd, sw.SDDMM_AFFINE: 0.7 * v + 0.3 * absd,
                 sw.SDDMM_DOT: absd}[kind]
        for opts in OPTS:
            G.say(f"sddmm wave tiles {ending} kdim={kdim} kind={kind} "
                  f"opts='{opts}'")
            out = torch.full((csr.nnz,), float("nan"), device=G.DEV)
            sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices),
                     G.t(csr.values), G.t(lhs), G.t(rhs), out, kind, 0.3, 0.7,
                     options=opts or None)
            torch.cuda.synchronize()
            assert_within_bound(out.cpu().numpy(), ref, bound + 1e-30,
                                what=f"{ending} kind {kind} {opts}")


@pytest.mark.parametrize("ending", ["last4", "last2", "partial"])
@pytest.mark.parametrize("kdim", [64, 128])
def test_sddmm_wave_tiles_bf16(dev, orc, kdim, ending):
    csr, rng = _tile64_mask(10 + kdim, ending)
    lhs = rng.standard_normal((csr.rows, kdim)).astype(np.float32)
    rhs = rng.standard_normal((kdim, csr.cols)).astype(np.float32)
    for kind in (sw.SDDMM_MUL, sw.SDDMM_AFFINE, sw.SDDMM_DOT):
        for opts in OPTS:
            got = _sddmm(csr, csr.values, lhs, rhs, kind, 0.3, 0.7,
                         opts or None)
            _sddmm_check(orc, csr, csr.values, lhs, rhs, kind, 0.3, 0.7, got)
