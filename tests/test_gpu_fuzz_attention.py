"""Seeded fuzz of SDDMM, the CSR row ops, the sparse-attention chain and BSR
SpMM against the CPU oracle.

Each seed draws an attention mask built from 16-row tiles, each tile one of
the cases the 16-row tile kernels tell apart:
* prefix tiles, where every row's columns are a prefix of the tile's last row
  (the register-tile path); last rows of 1 to 600 entries, so some pass the
  512-entry limit and run row by row;
* prefix tiles whose leading rows are empty;
* prefix tiles with one column of one row replaced (the structure check
  fails, so the tile runs row by row);
* rows of independent random columns;
* tiles of empty rows;
and a partial last tile.  The widths d and dv include values the fused
kernel takes (d of 64 or 128, dv a multiple of 16) and values it leaves to
the six-op schedule (d of 256 takes the SDDMM's four-step MFMA tile).  Every
SDDMM mapping and every attention schedule runs on it in fp32 and bf16, the
row ops in fp32, and a ragged BSR matrix (block rows of 0 to 9 blocks) runs
through the fp32 and bf16 BSR kernels.

Bars: the fp32 op bars (1e-5 sum |terms|), the attention bounds derived from
them (tests/_attention_check.py), and for bf16 the fp32 bar plus one
rounding, and rel-L2 <= 1e-2."""
import os

import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._attention_check import check_attention_f32
from tests._check import BF16_REL_L2, assert_within_bound, rel_l2
from tests.test_gpu_bf16 import (BF, ROW_OPTS as BF16_ROW_OPTS,
                                 _attention_bf16, _bsr_bf16,
                                 _check_attention_bf16, _sddmm, _sddmm_check,
                                 assert_bf16_within_bound)
from tests.test_gpu_bsr_attention import (ATT_OPTS, BSR_OPTS, ROW_OPTS,
                                          _bsr_run)

pytestmark = pytest.mark.gpu

# SW_FUZZ_SEEDS=N runs seeds 0 .. N-1 instead (a longer one-off run)
SEEDS = list(range(int(os.environ.get("SW_FUZZ_SEEDS", "5"))))


def _mask(seed):
    """(csr with U(-1, 1) mask values, rng)."""
    rng = np.random.default_rng(2000 + seed)
    rows = int(rng.integers(20, 400))
    cols = int(rng.choice([48, 300, 1100]))
    rows_cols = []
    for t0 in range(0, rows, 16):
        nt = min(16, rows - t0)
        kind = 0 if t0 == 0 else int(rng.integers(0, 5))
        if kind <= 2:
            last = int(rng.integers(1, min(cols, 600) + 1))
            base = np.sort(rng.choice(cols, last, replace=False))
            lens = np.sort(rng.integers(0 if kind == 1 else 1, last + 1, nt))
            lens[-1] = last
            tile = [base[:n].copy() for n in lens]
            others = np.setdiff1d(np.arange(cols), base)
            if kind == 2 and nt > 1 and others.size:
                r = int(rng.integers(0, nt - 1))
                if tile[r].size:
                    tile[r][int(rng.integers(0, tile[r].size))] = \
                        rng.choice(others)
                    tile[r] = np.sort(tile[r])
        elif kind == 3:
            tile = [np.sort(rng.choice(cols, int(rng.integers(
                0, min(cols, 80) + 1)), replace=False)) for _ in range(nt)]
        else:
            tile = [np.zeros(0, np.int64) for _ in range(nt)]
        rows_cols += tile
    lengths = np.array([c.size for c in rows_cols])
    ro = np.zeros(rows + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(rows_cols).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    return W.CSR(rows, cols, ro, col, val), rng


def _widths(seed):
    """(d, dv): each seed a different pair, every width once per 5 seeds."""
    return ([64, 128, 32, 100, 256][seed % 5],
            [64, 16, 80, 128, 24][(3 * seed) % 5])


def _inputs(csr, rng, d, dv):
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    # the attention scale 1/sqrt(d) times 0.5 .. 2: rounding q and K^T to
    # bf16 moves a score by about alpha sqrt(d) 2^-9, which the bf16
    # chain's rel-L2 bar against the unrounded fp32 chain assumes is small
    alpha = float(rng.uniform(0.5, 2.0)) / float(np.sqrt(d))
    beta = float(rng.choice([0.0, 0.5]))
    return q, kt, v, alpha, beta


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention_f32(dev, orc, seed):
    csr, rng = _mask(seed)
    d, dv = _widths(seed)
    q, kt, v, alpha, beta = _inputs(csr, rng, d, dv)
    refs = orc.sparse_attention(csr.row_offsets, csr.column_indices,
                                csr.values, q, kt, v, alpha, beta)
    nan = float("nan")
    for opts in ATT_OPTS:
        G.say(f"fuzz attention seed {seed} rows={csr.rows} nnz={csr.nnz} "
              f"d={d} dv={dv} opts='{opts}'")
        scores = torch.full((csr.nnz,), nan, device=G.DEV)
        rmax = torch.full((csr.rows,), nan, device=G.DEV)
        rsum = torch.full((csr.rows,), nan, device=G.DEV)
        out = torch.full((csr.rows, dv), nan, device=G.DEV)
        sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                            G.t(csr.values), G.t(q), G.t(kt), G.t(v), scores,
                            rmax, rsum, out, alpha, beta, options=opts)
        torch.cuda.synchronize()
        check_attention_f32(orc, csr, csr.values, q, kt, v, alpha, beta,
                            scores.cpu().numpy(), rmax.cpu().numpy(),
                            rsum.cpu().numpy(), out.cpu().numpy(), refs)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention_bf16(dev, orc, seed):
    csr, rng = _mask(seed)
    d, dv = _widths(seed)
    q, kt, v, alpha, beta = _inputs(csr, rng, d, dv)
    for opts in ATT_OPTS:
        got = _attention_bf16(csr, csr.values, q, kt, v, alpha, beta, opts)
        _check_attention_bf16(orc, csr, csr.values, q, kt, v, alpha, beta,
                              got)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_sddmm(dev, orc, seed):
    csr, rng = _mask(seed)
    d, _ = _widths(seed)
    lhs = rng.standard_normal((csr.rows, d)).astype(np.float32)
    rhs = rng.standard_normal((d, csr.cols)).astype(np.float32)
    rows = np.repeat(np.arange(csr.rows), np.diff(csr.row_offsets))
    absd = (np.abs(lhs.astype(np.float64)) @ np.abs(rhs.astype(np.float64)))[
        rows, csr.column_indices]
    v = np.abs(csr.values.astype(np.float64))
    for kind in (sw.SDDMM_MUL, sw.SDDMM_AFFINE, sw.SDDMM_DOT):
        ref = orc.sddmm(csr.row_offsets, csr.column_indices, csr.values, lhs,
                        rhs, kind, 0.3, 0.7)
        bound = {sw.SDDMM_MUL: v * absd, sw.SDDMM_AFFINE: 0.7 * v + 0.3 * absd,
                 sw.SDDMM_DOT: absd}[kind]
        for opts in ROW_OPTS:
            G.say(f"fuzz sddmm seed {seed} d={d} kind={kind} opts='{opts}'")
            out = torch.full((csr.nnz,), float("nan"), device=G.DEV)
            sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices),
                     G.t(csr.values), G.t(lhs), G.t(rhs), out, kind, 0.3, 0.7,
                     options=opts)
            torch.cuda.synchronize()
            assert_within_bound(out.cpu().numpy(), ref, bound + 1e-30,
                                what=f"seed {seed} kind {kind} {opts}")
        for opts in BF16_ROW_OPTS:
            got = _sddmm(csr, csr.values, lhs, rhs, kind, 0.3, 0.7, opts)
            _sddmm_check(orc, csr, csr.values, lhs, rhs, kind, 0.3, 0.7, got)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_row_ops(dev, orc, seed):
    csr, rng = _mask(seed)
    ro, vals = G.t(csr.row_offsets), G.t(csr.values)
    cs = np.concatenate([[0.0], np.cumsum(np.abs(csr.values.astype(
        np.float64)))])
    bound = cs[csr.row_offsets[1:]] - cs[csr.row_offsets[:-1]]
    rowv = rng.uniform(0.5, 2, csr.rows).astype(np.float32)
    for opts in ROW_OPTS:
        G.say(f"fuzz row ops seed {seed} rows={csr.rows} opts='{opts}'")
        out = torch.full((csr.rows,), float("nan"), device=G.DEV)
        sw.csr_row_reduce(ro, None, vals, out, "max", options=opts)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(
            out.cpu().numpy(),
            orc.row_reduce(csr.row_offsets, csr.values, orc.REDUCE_MAX))
        sw.csr_row_reduce(ro, None, vals, out, "sum", options=opts)
        torch.cuda.synchronize()
        ref = orc.row_reduce(csr.row_offsets, csr.values, orc.REDUCE_SUM)
        assert_within_bound(out.cpu().numpy(), ref, bound,
                            what=f"row sum seed {seed} {opts}")
        for kind in (sw.MAP_EXP_SUB, sw.MAP_DIV, sw.MAP_SUB, sw.MAP_MUL):
            o = torch.full((csr.nnz,), float("nan"), device=G.DEV)
            sw.csr_rowwise_map(ro, None, vals, G.t(rowv), o, kind,
                               options=opts)
            torch.cuda.synchronize()
            ref = orc.rowwise_map(csr.row_offsets, csr.values, rowv, kind)
            np.testing.assert_allclose(o.cpu().numpy(), ref, rtol=2e-6,
                                       atol=1e-7)


def _bsr(seed):
    rng = np.random.default_rng(3000 + seed)
    b = int(rng.choice([16, 16, 4, 8, 1]))
    nbr = int(rng.integers(1, 80))
    counts = rng.integers(0, 10, nbr)
    counts = np.minimum(counts, nbr)
    cols = [np.sort(rng.choice(nbr, c, replace=False)) for c in counts]
    bro = np.zeros(nbr + 1, np.int32)
    np.cumsum(counts, out=bro[1:])
    bcol = (np.concatenate(cols) if counts.sum() else np.zeros(0)).astype(
        np.int32)
    vals = rng.standard_normal(bcol.size * b * b).astype(np.float32)
    k = int(rng.choice([1, 4, 8, 30, 40, 64, 128, 200]))
    rhs = rng.standard_normal((nbr * b, k)).astype(np.float32)
    return W.BSR(rows=nbr * b, cols=nbr * b, block_size=b,
                 block_row_offsets=bro, block_column_indices=bcol,
                 block_values=vals), rhs


@pytest.mark.parametrize("seed", list(range(8)))
def test_fuzz_bsr(dev, orc, seed):
    bsr, rhs = _bsr(seed)
    b = bsr.block_size
    args = (bsr.block_row_offsets, bsr.block_column_indices)
    ref = orc.bsr_spmm(*args, bsr.block_values, rhs, b)
    bound = orc.bsr_abs_bound(*args, bsr.block_values, rhs, b)
    for opts in BSR_OPTS:
        out = _bsr_run(bsr, rhs, opts)
        assert_within_bound(out, ref, bound, what=f"seed {seed} {opts}")
    vb, rb = orc.as_bf16(bsr.block_values), orc.as_bf16(rhs)
    ref_b = orc.bsr_spmm(*args, vb, rb, b)
    bound_b = orc.bsr_abs_bound(*args, vb, rb, b)
    for opts in ("bsr-use-mfma=1", "bsr-use-mfma=0"):
        for out_dtype in (BF, torch.float32):
            got = _bsr_bf16(bsr, rhs, opts, out_dtype)
            if out_dtype == BF:
                assert_bf16_within_bound(got, ref_b, bound_b,
                                         what=f"seed {seed} {opts}")
            else:
                assert_within_bound(got, ref_b, bound_b,
                                    what=f"seed {seed} {opts}")
            if np.any(ref):
                assert rel_l2(got, ref) <= BF16_REL_L2


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_attention_bundle(dev, orc, tmp_path, seed):
    """The lrrt attention bundle built for each fuzz mask's shapes (its
    kernels specialise rows, key rows, d and dv), its six kernels launched in
    order as a runtime does, against the oracle with the chain's derived
    bounds.  The masks' 16-row tiles give the output kernel prefix tiles,
    fallback tiles and empty tiles; the scores kernel's 64-row tiles mostly
    take its rows' own path, and d of 64 and 128 its matrix-core tiles."""
    from sparsewavecomp_amd import bundle as B
    from sparsewavecomp_amd.bundle.runtime import Bundle
    csr, rng = _mask(seed)
    d, dv = _widths(seed)
    q, kt, v, alpha, beta = _inputs(csr, rng, d, dv)
    B.build_attention_bundle(tmp_path / "b", rows=csr.rows, key_rows=csr.cols,
                             head_dim=d, value_cols=dv, alpha=alpha,
                             beta=beta)
    bun = Bundle(tmp_path / "b")
    nan = float("nan")
    bufs = {"rowOffsets": G.t(csr.row_offsets),
            "columnIndices": G.t(csr.column_indices),
            "maskValues": G.t(csr.values), "query": G.t(q),
            "transposedKey": G.t(kt), "value": G.t(v),
            "scores": torch.full((max(csr.nnz, 1),), nan, device=G.DEV),
            "rowMaximum": torch.full((csr.rows,), nan, device=G.DEV),
            "rowSum": torch.full((csr.rows,), nan, device=G.DEV),
            "output": torch.full((csr.rows, dv), nan, device=G.DEV)}
    ptrs = {k: t.data_ptr() for k, t in bufs.items()}
    G.say(f"fuzz attention bundle seed {seed} rows={csr.rows} "
          f"nnz={csr.nnz} d={d} dv={dv}")
    for name in B.ATTENTION_ORDER:
        bun.launch(name, csr.rows * dv if name == "sparse_attention_output"
                   else csr.rows, ptrs)
    torch.cuda.synchronize()
    bun.close()
    refs = orc.sparse_attention(csr.row_offsets, csr.column_indices,
                                csr.values, q, kt, v, alpha, beta)
    check_attention_f32(orc, csr, csr.values, q, kt, v, alpha, beta,
                        bufs["scores"].cpu().numpy()[:csr.nnz],
                        bufs["rowMaximum"].cpu().numpy(),
                        bufs["rowSum"].cpu().numpy(),
                        bufs["output"].cpu().numpy(), refs)
