"""GPU parity of BSR SpMM (thread-per-output and MFMA, fp32 and bf16), SDDMM,
CSR row reduce / row-wise map and the six-kernel sparse attention chain."""
import math

import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._attention_check import check_attention_f32
from tests._check import BF16_REL_L2, assert_within_bound, rel_l2

pytestmark = pytest.mark.gpu


def _bsr_run(bsr, rhs, opts, bf16=False):
    G.say(f"bsr rows={bsr.rows} nnzb={bsr.nnzb} b={bsr.block_size} "
          f"k={rhs.shape[1]} bf16={bf16} opts='{opts}'")
    dt = torch.bfloat16 if bf16 else None
    out = torch.full((bsr.rows, rhs.shape[1]), float("nan"), device=G.DEV)
    sw.bsr_spmm(G.t(bsr.block_row_offsets), G.t(bsr.block_column_indices),
                G.t(bsr.block_values, dt), G.t(rhs, dt), out,
                bsr.block_size, options=opts)
    torch.cuda.synchronize()
    return out.cpu().numpy()


BSR_OPTS = ["bsr-use-mfma=1", "bsr-use-mfma=0",
            "bsr-use-mfma=0 spmm-block-size=64"]


@pytest.mark.parametrize("opts", BSR_OPTS)
def test_bsr_golden(dev, golden, opts):
    g = golden["bsr_spmm"]
    bsr = W.BSR(g["rows"], g["cols"], g["block_size"],
                np.array(g["block_row_offsets"], np.int32),
                np.array(g["block_column_indices"], np.int32),
                np.array(g["block_values"], np.float32))
    out = _bsr_run(bsr, np.array(g["rhs"], np.float32), opts)
    np.testing.assert_array_equal(out, np.array(g["expected"], np.float32))


@pytest.mark.parametrize("opts", BSR_OPTS)
# k % 4 == 0 takes the column-interleaved MFMA kernels (partial strips at 40
# and 200), other k the scalar-load MFMA kernels
@pytest.mark.parametrize("b,k", [(16, 128), (16, 40), (16, 200), (16, 30),
                                 (16, 7), (4, 9), (4, 64), (8, 128)])
def test_bsr_fp32(dev, orc, opts, b, k):
    bsr = W.bsr_banded(seed=b + k, rows=b * 96, block_size=b,
                       blocks_per_row=6, band=3, band_blocks=3,
                       value_std=0.5)
    rhs = np.random.default_rng(k).standard_normal((bsr.cols, k)).astype(
        np.float32)
    out = _bsr_run(bsr, rhs, opts)
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                       bsr.block_values, rhs, b)
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              bsr.block_values, rhs, b)
    assert_within_bound(out, ref, bound)


@pytest.mark.parametrize("opts", BSR_OPTS)
@pytest.mark.parametrize("k", [128, 30])
def test_bsr_non_finite(dev, orc, opts, k):
    """inf / NaN in block values and in B: each output is NaN / +inf / -inf
    exactly when the oracle's is.  Stored blocks are dense, so an explicit
    zero of a block times an inf of B is NaN in the reference as well."""
    b = 16
    bsr = W.bsr_banded(seed=k, rows=b * 64, block_size=b, blocks_per_row=6,
                       band=3, band_blocks=3, value_std=0.5)
    rng = np.random.default_rng(k + 2)
    vals = bsr.block_values.copy()
    flat = vals.reshape(-1)
    pick = rng.choice(flat.size, 6, replace=False)
    flat[pick[:2]] = np.inf
    flat[pick[2:4]] = -np.inf
    flat[pick[4:]] = np.nan
    bsr = W.BSR(bsr.rows, bsr.cols, b, bsr.block_row_offsets,
                bsr.block_column_indices, vals)
    rhs = rng.standard_normal((bsr.cols, k)).astype(np.float32)
    rhs[rng.integers(0, bsr.cols), rng.integers(0, k)] = np.inf
    out = _bsr_run(bsr, rhs, opts)
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                       bsr.block_values, rhs, b)
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(out), cls(ref))
    fin = np.isfinite(ref)
    assert (~fin).any() and fin.any()
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              np.nan_to_num(vals, posinf=0, neginf=0),
                              np.nan_to_num(rhs, posinf=0, neginf=0), b)
    assert_within_bound(out[fin], ref[fin], bound[fin])


@pytest.mark.parametrize("opts", ["bsr-use-mfma=1", "bsr-use-mfma=0"])
@pytest.mark.parametrize("k", [128, 36, 30])
def test_bsr_bf16(dev, orc, opts, k):
    bsr = W.bsr_banded(seed=3, rows=16 * 128, block_size=16)
    rhs = np.random.default_rng(3).standard_normal((bsr.cols, k)).astype(
        np.float32)
    out = _bsr_run(bsr, rhs, opts, bf16=True)
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                       bsr.block_values, rhs, 16)
    assert rel_l2(out, ref) <= BF16_REL_L2
    # against the oracle on bf16-rounded inputs the fp32 bound holds
    vb, rb = G.bf16_round(bsr.block_values), G.bf16_round(rhs)
    ref_b = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices, vb,
                         rb, 16)
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              vb, rb, 16)
    assert_within_bound(out, ref_b, bound)


def _ragged_bsr(seed, b=16):
    """Block rows of 0 to 9 blocks: the MFMA kernels split a block row's
    blocks over several waves, so rows with fewer blocks than waves, empty
    rows and rows whose count is not a multiple of the split all occur."""
    rng = np.random.default_rng(seed)
    counts = np.array([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 0, 1, 0, 5] * 4)
    nbr = counts.size
    cols = [np.sort(rng.choice(nbr, c, replace=False)) for c in counts]
    bro = np.zeros(nbr + 1, np.int32)
    np.cumsum(counts, out=bro[1:])
    bcol = np.concatenate(cols).astype(np.int32)
    vals = rng.standard_normal(bcol.size * b * b).astype(np.float32)
    return W.BSR(rows=nbr * b, cols=nbr * b, block_size=b,
                 block_row_offsets=bro, block_column_indices=bcol,
                 block_values=vals)


@pytest.mark.parametrize("k", [128, 64, 200, 36])
def test_bsr_ragged_block_rows(dev, orc, k):
    bsr = _ragged_bsr(k)
    rhs = np.random.default_rng(k + 1).standard_normal(
        (bsr.cols, k)).astype(np.float32)
    out = _bsr_run(bsr, rhs, "bsr-use-mfma=1")
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                       bsr.block_values, rhs, 16)
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              bsr.block_values, rhs, 16)
    assert_within_bound(out, ref, bound)


@pytest.mark.parametrize("opts", ["bsr-use-mfma=1",
                                  # the reference's thread-per-output
                                  # mapping, as bench.py times it
                                  "bsr-use-mfma=0"])
def test_bsr_config4_sample(dev, orc, opts):
    bsr, rhs = W.config4(seed=0)
    out = _bsr_run(bsr, rhs, opts)
    # check 400 block rows (first, last, random) of the full-size product
    brs = np.unique(np.concatenate([
        [0, 1, bsr.rows // 16 - 1],
        np.random.default_rng(0).choice(bsr.rows // 16, 400, replace=False)]))
    bro = bsr.block_row_offsets
    counts = bro[brs + 1] - bro[brs]
    sub_ro = np.zeros(brs.size + 1, np.int64)
    np.cumsum(counts, out=sub_ro[1:])
    idx = np.concatenate([np.arange(bro[b], bro[b + 1]) for b in brs])
    sub_vals = bsr.block_values.reshape(-1, 256)[idx].ravel()
    ref = orc.bsr_spmm(sub_ro.astype(np.int32), bsr.block_column_indices[idx],
                       sub_vals, rhs, 16)
    bound = orc.bsr_abs_bound(sub_ro.astype(np.int32),
                              bsr.block_column_indices[idx], sub_vals, rhs, 16)
    rows = (brs[:, None] * 16 + np.arange(16)[None, :]).ravel()
    assert_within_bound(out[rows], ref, bound)


# ---- SDDMM / row reduce / row-wise map / attention -------------------------

ROW_OPTS = ["", "sddmm-lanes-per-row=64", "sddmm-block-size=64",
            "sddmm-block-size=512", "sddmm-block-size=1024",
            "sddmm-mapping=row-tile-mfma", "sddmm-mapping=wave-per-row"]


@pytest.mark.parametrize("opts", ROW_OPTS)
def test_sddmm_golden_and_random(dev, orc, golden, opts):
    g = golden["sddmm"]
    ro = np.array(g["row_offsets"], np.int32)
    col = np.array(g["column_indices"], np.int32)
    val = np.array(g["values"], np.float32)
    lhs = np.array(g["lhs"], np.float32)
    rhs = np.array(g["rhs"], np.float32)
    out = torch.empty(3, device=G.DEV)
    G.say(f"sddmm golden opts='{opts}'")
    sw.sddmm(G.t(ro), G.t(col), G.t(val), G.t(lhs), G.t(rhs), out,
             sw.SDDMM_MUL, options=opts)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), g["expected"])
    csr = W.random_csr(500, 300, 40.0, 2, empty_fraction=0.2)
    rng = np.random.default_rng(2)
    for kdim in (1, 64, 100, 128):
        lhs = rng.standard_normal((500, kdim)).astype(np.float32)
        rhs = rng.standard_normal((kdim, 300)).astype(np.float32)
        for kind in (sw.SDDMM_MUL, sw.SDDMM_AFFINE, sw.SDDMM_DOT):
            out = torch.empty(csr.nnz, device=G.DEV)
            G.say(f"sddmm kdim={kdim} kind={kind} opts='{opts}'")
            sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices),
                     G.t(csr.values), G.t(lhs), G.t(rhs), out, kind, 0.3, 0.7,
                     options=opts)
            torch.cuda.synchronize()
            ref = orc.sddmm(csr.row_offsets, csr.column_indices, csr.values,
                            lhs, rhs, kind, 0.3, 0.7)
            rows = np.repeat(np.arange(500), np.diff(csr.row_offsets))
            absd = np.abs(lhs.astype(np.float64)) @ np.abs(
                rhs.astype(np.float64))
            b = absd[rows, csr.column_indices]
            v = np.abs(csr.values.astype(np.float64))
            bound = {sw.SDDMM_MUL: v * b, sw.SDDMM_AFFINE: 0.7 * v + 0.3 * b,
                     sw.SDDMM_DOT: b}[kind]
            assert_within_bound(out.cpu().numpy(), ref, bound + 1e-30)


def _tile_structure_csr():
    """87 rows in 16-row tiles exercising each path of the MFMA tile
    kernels: prefix-structured tiles (the MFMA path), a row with the last
    row's length but one different column (recomputed after the shared
    check), a row longer than the tile's last row (row path from the start),
    empty rows, a mismatch deep in the row (a later wave's chunk), and a
    partial last tile."""
    rng = np.random.default_rng(31)
    cols = 300
    rows_cols = []
    for tile in range(6):
        nt = 16 if tile < 5 else 7
        base = np.sort(rng.choice(cols, 200, replace=False))
        lens = np.sort(rng.integers(1, 201, nt))
        lens[-1] = 200
        if tile == 3:
            lens[:5] = 0
        tile_rows = [base[:n].copy() for n in lens]
        if tile == 1:                       # same length, one column differs
            tile_rows[5] = tile_rows[-1][:lens[5]].copy()
            spare = np.setdiff1d(np.arange(cols), base)[0]
            tile_rows[5][min(10, lens[5] - 1)] = spare
            tile_rows[5] = np.sort(tile_rows[5])
        if tile == 2:                       # a row longer than the last
            extra = np.setdiff1d(np.arange(cols), base)[:5]
            tile_rows[3] = np.sort(np.concatenate([base, extra]))
        if tile == 4:                       # mismatch at position 150
            tile_rows[9] = base[:200].copy()
            tile_rows[9][150] = np.setdiff1d(np.arange(cols), base)[1]
            tile_rows[9] = np.sort(tile_rows[9])
            tile_rows[-1] = base.copy()
        rows_cols += tile_rows
    lengths = np.array([len(c) for c in rows_cols])
    ro = np.zeros(len(rows_cols) + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(rows_cols).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    return W.CSR(len(rows_cols), cols, ro, col, val)


@pytest.mark.parametrize("shape", ["structure", "long"])
@pytest.mark.parametrize("kdim", [64, 128])
@pytest.mark.parametrize("kind", ["mul", "affine", "dot"])
def test_sddmm_tile_structure_paths(dev, orc, kind, kdim, shape):
    """Each path of the SDDMM tiles (see the two matrices' docstrings), for
    each combine kind."""
    csr = _tile_structure_csr() if shape == "structure" else _long_prefix_csr()
    rng = np.random.default_rng(5)
    lhs = rng.standard_normal((csr.rows, kdim)).astype(np.float32)
    rhs = rng.standard_normal((kdim, csr.cols)).astype(np.float32)
    k = {"mul": sw.SDDMM_MUL, "affine": sw.SDDMM_AFFINE,
         "dot": sw.SDDMM_DOT}[kind]
    out = torch.full((csr.nnz,), float("nan"), device=G.DEV)
    G.say(f"sddmm tile {shape} paths kind={kind} kdim={kdim}")
    sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices), G.t(csr.values),
             G.t(lhs), G.t(rhs), out, k, 0.3, 0.7,
             options="sddmm-mapping=row-tile-mfma")
    torch.cuda.synchronize()
    ref = orc.sddmm(csr.row_offsets, csr.column_indices, csr.values, lhs, rhs,
                    k, 0.3, 0.7)
    rows = np.repeat(np.arange(csr.rows), np.diff(csr.row_offsets))
    b = (np.abs(lhs.astype(np.float64)) @ np.abs(rhs.astype(np.float64)))[
        rows, csr.column_indices]
    v = np.abs(csr.values.astype(np.float64))
    bound = {"mul": v * b, "affine": 0.7 * v + 0.3 * b, "dot": b}[kind]
    assert_within_bound(out.cpu().numpy(), ref, bound + 1e-30)


@pytest.mark.parametrize("k", [16, 64, 80])
def test_spmm_tile_structure_paths(dev, orc, k):
    csr = _tile_structure_csr()
    rhs = np.random.default_rng(k).standard_normal((csr.cols, k)).astype(
        np.float32)
    out = G.spmm(csr, rhs, "spmm-mapping=row-tile-mfma")
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, rhs)
    assert_within_bound(out, ref, bound)


@pytest.mark.parametrize("opts", ROW_OPTS)
def test_row_reduce_and_map(dev, orc, golden, opts):
    g = golden["row_reduce"]
    ro = G.t(np.array(g["row_offsets"], np.int32))
    val = G.t(np.array(g["values"], np.float32))
    s = torch.empty(3, device=G.DEV)
    m = torch.empty(3, device=G.DEV)
    G.say(f"row_reduce golden opts='{opts}'")
    sw.csr_row_reduce(ro, None, val, s, "sum", options=opts)
    sw.csr_row_reduce(ro, None, val, m, "max", options=opts)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), g["expected_sum"])
    np.testing.assert_array_equal(
        m.cpu().numpy(), [float(v) for v in g["expected_max"]])
    # softmax golden through the four row ops
    gs = golden["softmax"]
    e = torch.empty(4, device=G.DEV)
    sw.csr_rowwise_map(ro, None, val, m, e, sw.MAP_EXP_SUB, options=opts)
    sw.csr_row_reduce(ro, None, e, s, "sum", options=opts)
    sw.csr_rowwise_map(ro, None, e, s, e, sw.MAP_DIV, options=opts)
    torch.cuda.synchronize()
    np.testing.assert_allclose(e.cpu().numpy(), gs["expected"], rtol=0,
                               atol=5e-7)
    # random rows, NaN propagation in max
    csr = W.random_csr(2000, 500, 30.0, 7, empty_fraction=0.2,
                       lognormal=True, max_len=500)
    vals = csr.values.copy()
    vals[5] = np.nan
    out = torch.empty(csr.rows, device=G.DEV)
    for kind, okind in (("sum", orc.REDUCE_SUM), ("max", orc.REDUCE_MAX)):
        sw.csr_row_reduce(G.t(csr.row_offsets), None, G.t(vals), out, kind,
                          options=opts)
        torch.cuda.synchronize()
        ref = orc.row_reduce(csr.row_offsets, vals, okind)
        got = out.cpu().numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        ok = ~np.isnan(ref)
        if kind == "max":
            np.testing.assert_array_equal(got[ok], ref[ok])
        else:
            lens = np.diff(csr.row_offsets)
            absb = np.array([np.abs(vals[a:b]).sum() for a, b in
                             zip(csr.row_offsets[:-1], csr.row_offsets[1:])])
            assert np.all(np.abs(got[ok] - ref[ok]) <= 1e-5 * absb[ok] + 0)
            del lens
    # the sign of a zero maximum: +0 is above -0 in either order
    zs = np.array([-0.0, 0.0, 0.0, -0.0, -0.0, -0.0, -0.0, 0.0], np.float32)
    zro = np.array([0, 2, 4, 6, 7, 8], np.int32)
    zout = torch.empty(5, device=G.DEV)
    sw.csr_row_reduce(G.t(zro), None, G.t(zs), zout, "max", options=opts)
    torch.cuda.synchronize()
    zref = orc.row_reduce(zro, zs, orc.REDUCE_MAX)
    np.testing.assert_array_equal(np.signbit(zout.cpu().numpy()),
                                  np.signbit(zref))
    np.testing.assert_array_equal(np.signbit(zref),
                                  [False, False, True, True, False])
    rowv = np.random.default_rng(1).uniform(0.5, 2, csr.rows).astype(
        np.float32)
    for kind in (sw.MAP_EXP_SUB, sw.MAP_DIV, sw.MAP_SUB, sw.MAP_MUL):
        o = torch.empty(csr.nnz, device=G.DEV)
        sw.csr_rowwise_map(G.t(csr.row_offsets), None, G.t(csr.values),
                           G.t(rowv), o, kind, options=opts)
        torch.cuda.synchronize()
        ref = orc.rowwise_map(csr.row_offsets, csr.values, rowv, kind)
        np.testing.assert_allclose(o.cpu().numpy(), ref, rtol=2e-6, atol=1e-7)


def _attention(mask, q, kt, v, alpha, opts, everything=False):
    G.say(f"attention rows={mask.rows} nnz={mask.nnz} opts='{opts}'")
    rows = mask.rows
    scores = torch.empty(mask.nnz, device=G.DEV)
    rmax = torch.empty(rows, device=G.DEV)
    rsum = torch.empty(rows, device=G.DEV)
    out = torch.full((rows, v.shape[1]), float("nan"), device=G.DEV)
    sw.sparse_attention(G.t(mask.row_offsets), G.t(mask.column_indices),
                        G.t(mask.values), G.t(q), G.t(kt), G.t(v), scores,
                        rmax, rsum, out, alpha, 0.0, options=opts)
    torch.cuda.synchronize()
    if everything:
        return (out.cpu().numpy(), scores.cpu().numpy(), rmax.cpu().numpy(),
                rsum.cpu().numpy())
    return out.cpu().numpy(), scores.cpu().numpy()


ATT_OPTS = ["", "sddmm-lanes-per-row=64 spmm-mapping=wave-per-row-tile "
            "spmm-tile-size=32 spmm-lanes-per-row=16",
            "sddmm-mapping=row-tile-mfma sddmm-lanes-per-row=64 "
            "spmm-mapping=row-tile-mfma"]


@pytest.mark.parametrize("opts", ATT_OPTS)
def test_attention_golden(dev, golden, opts):
    g = golden["attention"]
    mask = W.CSR(2, 3, np.array(g["row_offsets"], np.int32),
                 np.array(g["column_indices"], np.int32),
                 np.array(g["mask_values"], np.float32))
    out, _ = _attention(mask, np.array(g["query"], np.float32),
                        np.array(g["transposed_key"], np.float32),
                        np.array(g["value"], np.float32), g["alpha"], opts)
    np.testing.assert_allclose(np.floor(out.astype(np.float64) * 1e4) / 1e4,
                               g["expected"], rtol=0, atol=1e-9)


@pytest.mark.parametrize("opts", ATT_OPTS)
@pytest.mark.parametrize("seq", [1024, 8192])
def test_attention_config5(dev, orc, opts, seq):
    mask, q, kt, v, alpha = W.config5(seed=0, seq=seq)
    out, scores, rmax, rsum = _attention(mask, q, kt, v, alpha, opts,
                                         everything=True)
    check_attention_f32(orc, mask, mask.values, q, kt, v, alpha, 0.0, scores,
                        rmax, rsum, out)
    assert math.isfinite(float(out.sum()))


FUSED = ("sddmm-mapping=row-tile-mfma sddmm-lanes-per-row=64 "
         "spmm-mapping=row-tile-mfma")


def _long_prefix_csr():
    """Tiles with the shared (prefix) column structure whose last rows hold
    700, 512 and 513 entries: the fused kernel keeps at most 512 scores per
    row in LDS and computes longer tiles row by row."""
    rng = np.random.default_rng(41)
    cols = 900
    rows_cols = []
    for last in (700, 512, 513):
        base = np.sort(rng.choice(cols, last, replace=False))
        lens = np.sort(rng.integers(1, last + 1, 16))
        lens[-1] = last
        rows_cols += [base[:n].copy() for n in lens]
    lengths = np.array([len(c) for c in rows_cols])
    ro = np.zeros(len(rows_cols) + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(rows_cols).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    return W.CSR(len(rows_cols), cols, ro, col, val)


def _attention_case(orc, csr, d, dv, options, alpha=0.125, beta=0.5):
    rng = np.random.default_rng(d + dv)
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    nan = float("nan")
    scores = torch.full((csr.nnz,), nan, device=G.DEV)
    rmax = torch.full((csr.rows,), nan, device=G.DEV)
    rsum = torch.full((csr.rows,), nan, device=G.DEV)
    out = torch.full((csr.rows, dv), nan, device=G.DEV)
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        G.t(csr.values), G.t(q), G.t(kt), G.t(v), scores,
                        rmax, rsum, out, alpha, beta, options=options)
    torch.cuda.synchronize()
    s_ref, m_ref, sum_ref, ref = orc.sparse_attention(
        csr.row_offsets, csr.column_indices, csr.values, q, kt, v, alpha,
        beta)
    return (scores, rmax, rsum, out, (s_ref, m_ref, sum_ref, ref), v,
            (csr.values, q, kt, alpha, beta))


@pytest.mark.parametrize("shape", ["structure", "long"])
@pytest.mark.parametrize("d,dv", [(64, 64), (128, 16), (64, 80), (128, 128)])
def test_attention_fused_paths(dev, orc, shape, d, dv):
    """The one-kernel attention chain: register tiles, the row-by-row path
    (columns not shared, a row longer than the last, a deep mismatch, rows
    over 512 entries), empty rows, a partial last tile, d of 64 and 128, dv
    of one to eight 16-column tiles, and a non-zero mask weight."""
    csr = _tile_structure_csr() if shape == "structure" else _long_prefix_csr()
    G.say(f"fused attention {shape} rows={csr.rows} nnz={csr.nnz} d={d} "
          f"dv={dv}")
    _check_attention(orc, csr, *_attention_case(orc, csr, d, dv, FUSED))


@pytest.mark.parametrize("opts", ATT_OPTS)
@pytest.mark.parametrize("alpha,low", [(1.0, -40.0), (1.6, -95.0)])
def test_attention_wide_score_range(dev, orc, opts, alpha, low):
    """Scores spread over about 70 (alpha = 1) or over 100 (alpha = 1.6)
    below their row's maximum (N(0, 1) operands, d = 64), so the
    exponentials run over a wide range of arguments: the fused kernel's exp2
    of the score times log2 e and its reciprocal row sums against the
    oracle's expf and division.  Below -87.3 expf is subnormal, which
    v_exp_f32 flushes to zero: the checker's absolute 2^-126 on each
    probability covers that (the row sum is at least 1)."""
    mask, _, _, _, _ = W.config5(seed=0, seq=1024)
    G.say(f"attention wide score range opts='{opts}'")
    got = _attention_case(orc, mask, 64, 64, opts, alpha=alpha, beta=0.0)
    s_ref = got[4][0]
    assert float(np.log(s_ref[s_ref > 0]).min()) < low
    _check_attention(orc, mask, *got)


def _f32_offset(a):
    """A float32 device view of a that starts one element (4 bytes) past an
    aligned address, so every 16-byte alignment check fails."""
    a = np.asarray(a, np.float32)
    flat = torch.empty(a.size + 1, dtype=torch.float32, device=G.DEV)
    view = flat[1:].view(a.shape)
    view.copy_(G.t(a))
    return view


@pytest.mark.parametrize("dv", [64, 80])
def test_attention_fused_misaligned_operands(dev, orc, dv):
    """The fp32 fused kernel with every value buffer one element off a
    16-byte boundary: the non-interleaved output tiles, element-aligned Q
    and mask windows, and K^T gathers through a descriptor whose base is
    only 4-byte aligned."""
    csr = _tile_structure_csr()
    d = 64
    rng = np.random.default_rng(dv)
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    G.say(f"fused attention misaligned operands dv={dv}")
    scores = _f32_offset(np.full(csr.nnz, np.nan, np.float32))
    rmax = _f32_offset(np.full(csr.rows, np.nan, np.float32))
    rsum = _f32_offset(np.full(csr.rows, np.nan, np.float32))
    out = _f32_offset(np.full((csr.rows, dv), np.nan, np.float32))
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        _f32_offset(csr.values), _f32_offset(q),
                        _f32_offset(kt), _f32_offset(v), scores, rmax, rsum,
                        out, 0.125, 0.5, options=FUSED)
    torch.cuda.synchronize()
    refs = orc.sparse_attention(csr.row_offsets, csr.column_indices,
                                csr.values, q, kt, v, 0.125, 0.5)
    _check_attention(orc, csr, scores, rmax, rsum, out, refs, v,
                     (csr.values, q, kt, 0.125, 0.5))


def _few_entries_csr(nnz):
    """Five rows holding nnz entries in all (one to six), rows of one, two
    and three entries and empty rows: with nnz >= 4 the fused kernel reads
    every 4-entry mask window from inside the buffer, shifting the windows
    that would pass its end; below 4 the options fall back to the op chain."""
    lengths = {1: [0, 1, 0, 0, 0], 2: [1, 0, 1, 0, 0], 3: [0, 2, 0, 1, 0],
               4: [1, 3, 0, 0, 0], 5: [0, 2, 0, 0, 3], 6: [3, 0, 1, 0, 2]}[nnz]
    rng = np.random.default_rng(nnz)
    ro = np.zeros(6, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate([np.sort(rng.choice(8, n, replace=False))
                          for n in lengths]).astype(np.int32)
    val = rng.uniform(-1, 1, nnz).astype(np.float32)
    return W.CSR(5, 8, ro, col, val)


def _empty_tile_csr():
    """40 rows: a prefix-structured 16-row tile, a tile of 16 empty rows
    (its last row is empty, so the structure check passes with no entries
    at all) and a partial tile of 8 rows."""
    rng = np.random.default_rng(17)
    cols = 96
    rows_cols = []
    for nt, width in ((16, 70), (16, 0), (8, 40)):
        base = np.sort(rng.choice(cols, max(width, 1), replace=False))
        lens = np.sort(rng.integers(1, width + 1, nt)) if width else \
            np.zeros(nt, np.int64)
        if width:
            lens[-1] = width
        rows_cols += [base[:n].copy() for n in lens]
    lengths = np.array([len(c) for c in rows_cols])
    ro = np.zeros(len(rows_cols) + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(rows_cols).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    return W.CSR(len(rows_cols), cols, ro, col, val)


@pytest.mark.parametrize("dv", [64, 80])
def test_attention_fused_empty_tile(dev, orc, dv):
    """A tile whose rows are all empty takes the fused path with no entry:
    its outputs are the identities (row maximum -inf, row sum 0, output 0)
    and the V rows it reads are valid ones."""
    csr = _empty_tile_csr()
    assert np.all(np.diff(csr.row_offsets)[16:32] == 0)
    G.say(f"fused attention empty tile dv={dv}")
    got = _attention_case(orc, csr, 64, dv, FUSED)
    _check_attention(orc, csr, *got)
    rmax, rsum, out = got[1].cpu().numpy(), got[2].cpu().numpy(), got[3]
    assert np.all(np.isneginf(rmax[16:32])) and np.all(rsum[16:32] == 0)
    assert np.all(out.cpu().numpy()[16:32] == 0)


@pytest.mark.parametrize("nnz", [1, 2, 3, 4, 5, 6])
def test_attention_few_entries(dev, orc, nnz):
    csr = _few_entries_csr(nnz)
    G.say(f"fused attention few entries nnz={nnz}")
    _check_attention(orc, csr, *_attention_case(orc, csr, 64, 64, FUSED))


@pytest.mark.parametrize("opts", [FUSED] + ATT_OPTS[:2])
def test_attention_masked_out_entries(dev, orc, opts):
    """Mask values of -inf with beta = 1 (entries masked out) follow IEEE
    arithmetic as the reference's ops do: a masked entry's probability is 0,
    and a row whose entries are all masked has row maximum -inf and NaN row
    sum, probabilities and output."""
    csr = _tile_structure_csr()
    rng = np.random.default_rng(77)
    mask = rng.uniform(-1, 1, csr.nnz).astype(np.float32)
    mask[rng.random(csr.nnz) < 0.2] = -np.inf
    lens = np.diff(csr.row_offsets)
    dead = int(np.flatnonzero(lens > 20)[1])       # a row of a shared tile
    mask[csr.row_offsets[dead]:csr.row_offsets[dead + 1]] = -np.inf
    d = dv = 64
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    alpha, beta = 0.125, 1.0
    G.say(f"attention with masked entries opts={opts!r}")
    nan = float("nan")
    scores = torch.full((csr.nnz,), nan, device=G.DEV)
    rmax = torch.full((csr.rows,), nan, device=G.DEV)
    rsum = torch.full((csr.rows,), nan, device=G.DEV)
    out = torch.full((csr.rows, dv), nan, device=G.DEV)
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        G.t(mask), G.t(q), G.t(kt), G.t(v), scores, rmax,
                        rsum, out, alpha, beta, options=opts)
    torch.cuda.synchronize()
    refs = orc.sparse_attention(
        csr.row_offsets, csr.column_indices, mask, q, kt, v, alpha, beta)
    s_ref, m_ref, sum_ref, ref = refs
    assert m_ref[dead] == -np.inf and np.isnan(sum_ref[dead])
    o = out.cpu().numpy()
    assert np.isnan(o[dead]).all() and np.isnan(ref[dead]).all()
    assert np.isnan(rsum.cpu().numpy()[dead])
    _check_attention(orc, csr, scores, rmax, rsum, out, refs, v,
                     (mask, q, kt, alpha, beta))


@pytest.mark.parametrize("opts", [FUSED] + ATT_OPTS[:2])
def test_attention_non_finite_value_rows(dev, orc, opts):
    """inf / NaN in V rows that a tile's last row includes but its shorter
    rows leave out: only the rows whose entries name them become non-finite,
    as in the reference (the fused kernel recomputes such a tile's output
    row by row)."""
    csr = _tile_structure_csr()
    rng = np.random.default_rng(78)
    d = dv = 64
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    last = csr.column_indices[csr.row_offsets[15]:csr.row_offsets[16]]
    v[last[150], 3] = np.inf           # rows 0..15: only those past 150
    v[last[120], 7] = np.nan
    v[last[190], :] = -np.inf
    alpha, beta = 0.125, 0.5
    G.say(f"attention with non-finite V rows opts={opts!r}")
    nan = float("nan")
    scores = torch.full((csr.nnz,), nan, device=G.DEV)
    rmax = torch.full((csr.rows,), nan, device=G.DEV)
    rsum = torch.full((csr.rows,), nan, device=G.DEV)
    out = torch.full((csr.rows, dv), nan, device=G.DEV)
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        G.t(csr.values), G.t(q), G.t(kt), G.t(v), scores,
                        rmax, rsum, out, alpha, beta, options=opts)
    torch.cuda.synchronize()
    s_ref, m_ref, sum_ref, ref = orc.sparse_attention(
        csr.row_offsets, csr.column_indices, csr.values, q, kt, v, alpha,
        beta)
    o = out.cpu().numpy()
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(o), cls(ref))
    fin = np.isfinite(ref)
    assert (~fin).any() and fin[:15].any()
    _check_attention(orc, csr, scores, rmax, rsum, out,
                     (s_ref, m_ref, sum_ref, ref), v,
                     (csr.values, q, kt, alpha, beta))


def _check_attention(orc, csr, scores, rmax, rsum, out, refs, v, inputs):
    """The chain's four outputs against the oracle with the bounds derived
    in tests/_attention_check.py; inputs = (mask values, q, kt, alpha,
    beta)."""
    mv, q, kt, alpha, beta = inputs
    check_attention_f32(orc, csr, mv, q, kt, v, alpha, beta,
                        scores.cpu().numpy(), rmax.cpu().numpy(),
                        rsum.cpu().numpy(), out.cpu().numpy(), refs)


@pytest.mark.parametrize("opts", ["sddmm-mapping=row-tile-mfma",
                                  # thread-per-row: 64-row wave tiles
                                  "", "sddmm-block-size=128",
                                  "sddmm-block-size=64"])
@pytest.mark.parametrize("in_place", [False, True])
@pytest.mark.parametrize("kdim", [64, 128, 32])
def test_sddmm_tile_mfma_block_mask(dev, orc, kdim, in_place, opts):
    """Block-structured masks take the 16-row MFMA tiles (row-tile-mfma) or
    the 64-row wave tiles (thread-per-row, fp32, kdim 64 or 128); with the
    output in place of the sample values the tiles read each entry's sample
    before writing it."""
    mask = W.attention_mask(seq=2048, block=64, window=4, random_blocks=2,
                            seed=3)
    rng = np.random.default_rng(kdim)
    lhs = rng.standard_normal((mask.rows, kdim)).astype(np.float32)
    rhs = rng.standard_normal((kdim, mask.cols)).astype(np.float32)
    vals = rng.uniform(-1, 1, mask.nnz).astype(np.float32)
    vt = G.t(vals)
    out = vt if in_place else torch.empty(mask.nnz, device=G.DEV)
    G.say(f"sddmm tile kdim={kdim} in_place={in_place} opts='{opts}'")
    sw.sddmm(G.t(mask.row_offsets), G.t(mask.column_indices), vt,
             G.t(lhs), G.t(rhs), out, sw.SDDMM_AFFINE, 0.125, 0.5,
             options=opts or None)
    torch.cuda.synchronize()
    ref = orc.sddmm(mask.row_offsets, mask.column_indices, vals, lhs, rhs,
                    sw.SDDMM_AFFINE, 0.125, 0.5)
    rows = np.repeat(np.arange(mask.rows), np.diff(mask.row_offsets))
    absd = np.abs(lhs.astype(np.float64)) @ np.abs(rhs.astype(np.float64))
    bound = 0.5 * np.abs(vals) + 0.125 * absd[rows, mask.column_indices]
    assert_within_bound(out.cpu().numpy(), ref, bound)
