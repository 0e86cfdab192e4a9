"""GPU parity of the bf16 entry points: SDDMM, row reduce / row-wise map,
SpMM, the sparse-attention chain (six-op schedules and the fused tile
kernel) and BSR SpMM with bf16 and fp32 outputs.

Every bf16 op computes in fp32 from its bf16 operands and rounds its stored
result once, so against the fp32 oracle run on the same (bf16-rounded)
inputs a result obeys the fp32 bound plus that rounding:
    |y - y_ref| <= 1e-5 * sum|terms| * (1 + 2^-8) + 2^-8 * |y_ref|.
Chains are checked against the oracle's bf16 chain (each op rounded as it
stores) -- most values bit-equal, the rest one rounding step away -- and
within rel-L2 <= 1e-2 of the fp32 chain on the unrounded inputs."""
import math

import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import BF16_REL_L2, rel_l2

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def b16(a):
    """Device bf16 tensor of a (round to nearest even)."""
    return G.t(np.asarray(a, np.float32), BF)


def host(t):
    return t.float().cpu().numpy()


def nan_b16(*shape):
    return torch.full(shape, float("nan"), dtype=BF, device=G.DEV)


def assert_bf16_within_bound(got, ref32, bound, rel=1e-5, what="output"):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref32, np.float64)
    bound = np.asarray(bound, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    tol = rel * bound * (1 + 2.0**-8) + 2.0**-8 * np.abs(ref) + 1e-37
    bad = np.abs(got - ref) > tol
    if bad.any():
        i = np.flatnonzero(bad.ravel())[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} beyond the bf16 bound; first "
            f"{i.tolist()}: got {got.ravel()[i].tolist()} want "
            f"{ref.ravel()[i].tolist()} tol {tol.ravel()[i].tolist()}")


def within_steps(got, want, steps=1):
    """|got - want| <= steps bf16 rounding steps of want (relative 2^-7)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return np.abs(got - want) <= steps * 2.0**-7 * np.abs(want) + 1e-30


# ---- SDDMM -------------------------------------------------------------------

ROW_OPTS = ["", "sddmm-lanes-per-row=64", "sddmm-mapping=row-tile-mfma",
            "sddmm-mapping=wave-per-row"]


def _sddmm(csr, vals, lhs, rhs, kind, alpha, beta, opts):
    out = nan_b16(csr.nnz)
    G.say(f"bf16 sddmm rows={csr.rows} nnz={csr.nnz} kdim={lhs.shape[1]} "
          f"kind={kind} opts='{opts}'")
    sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices), b16(vals),
             b16(lhs), b16(rhs), out, kind, alpha, beta, options=opts)
    torch.cuda.synchronize()
    return host(out)


def _sddmm_check(orc, csr, vals, lhs, rhs, kind, alpha, beta, got):
    vb, lb, rb = orc.as_bf16(vals), orc.as_bf16(lhs), orc.as_bf16(rhs)
    ref = orc.sddmm(csr.row_offsets, csr.column_indices, vb, lb, rb, kind,
                    alpha, beta)
    rows = np.repeat(np.arange(csr.rows), np.diff(csr.row_offsets))
    absd = (np.abs(lb.astype(np.float64)) @ np.abs(rb.astype(np.float64)))[
        rows, csr.column_indices]
    v = np.abs(vb.astype(np.float64))
    bound = {sw.SDDMM_MUL: v * absd,
             sw.SDDMM_AFFINE: abs(beta) * v + abs(alpha) * absd,
             sw.SDDMM_DOT: absd}[kind]
    assert_bf16_within_bound(got, ref, bound, what=f"sddmm kind {kind}")
    assert np.mean(got == orc.as_bf16(ref)) > 0.95


@pytest.mark.parametrize("opts", ROW_OPTS)
def test_bf16_sddmm(dev, orc, golden, opts):
    g = golden["sddmm"]
    csr = W.CSR(len(g["row_offsets"]) - 1, len(g["rhs"][0]),
                np.array(g["row_offsets"], np.int32),
                np.array(g["column_indices"], np.int32),
                np.array(g["values"], np.float32))
    got = _sddmm(csr, csr.values, np.array(g["lhs"], np.float32),
                 np.array(g["rhs"], np.float32), sw.SDDMM_MUL, 1.0, 0.0, opts)
    np.testing.assert_array_equal(got, g["expected"])  # exact in bf16
    csr = W.random_csr(500, 300, 40.0, 2, empty_fraction=0.2)
    rng = np.random.default_rng(2)
    for kdim in (1, 64, 100, 128):
        lhs = rng.standard_normal((500, kdim)).astype(np.float32)
        rhs = rng.standard_normal((kdim, 300)).astype(np.float32)
        for kind in (sw.SDDMM_MUL, sw.SDDMM_AFFINE, sw.SDDMM_DOT):
            got = _sddmm(csr, csr.values, lhs, rhs, kind, 0.3, 0.7, opts)
            _sddmm_check(orc, csr, csr.values, lhs, rhs, kind, 0.3, 0.7, got)


# the 16-row tiles (row-tile-mfma) and thread-per-row, whose waves take
# their 64 rows as one matrix-core tile at kdim 64 and 128
TILE_OPTS = ["sddmm-mapping=row-tile-mfma", "", "sddmm-block-size=128"]


@pytest.mark.parametrize("opts", TILE_OPTS)
@pytest.mark.parametrize("kdim", [64, 128, 256])
@pytest.mark.parametrize("shape", ["block", "structure", "long"])
def test_bf16_sddmm_tiles(dev, orc, kdim, shape, opts):
    """The bf16 matrix-core SDDMM tiles on a block mask, on tiles that take
    their row-by-row fallback, and on tiles whose last rows hold 512, 513 and
    700 entries, for each combine kind."""
    from tests.test_gpu_bsr_attention import (_long_prefix_csr,
                                              _tile_structure_csr)
    csr = (W.attention_mask(seq=2048, block=64, window=4, random_blocks=2,
                            seed=3) if shape == "block"
           else _tile_structure_csr() if shape == "structure"
           else _long_prefix_csr())
    rng = np.random.default_rng(kdim)
    lhs = rng.standard_normal((csr.rows, kdim)).astype(np.float32)
    rhs = rng.standard_normal((kdim, csr.cols)).astype(np.float32)
    vals = rng.uniform(-1, 1, csr.nnz).astype(np.float32)
    for kind, alpha, beta in ((sw.SDDMM_AFFINE, 0.125, 0.5),
                              (sw.SDDMM_MUL, 1.0, 0.0),
                              (sw.SDDMM_DOT, 0.3, 0.7)):
        got = _sddmm(csr, vals, lhs, rhs, kind, alpha, beta, opts)
        _sddmm_check(orc, csr, vals, lhs, rhs, kind, alpha, beta, got)


@pytest.mark.parametrize("opts", TILE_OPTS)
@pytest.mark.parametrize("kdim", [64, 128])
def test_bf16_sddmm_tiles_in_place(dev, orc, kdim, opts):
    """Output in place of the sample values: each entry's sample is read
    before it is written."""
    csr = W.attention_mask(seq=2048, block=64, window=4, random_blocks=2,
                           seed=3)
    rng = np.random.default_rng(kdim)
    lhs = rng.standard_normal((csr.rows, kdim)).astype(np.float32)
    rhs = rng.standard_normal((kdim, csr.cols)).astype(np.float32)
    vals = rng.uniform(-1, 1, csr.nnz).astype(np.float32)
    vt = b16(vals)
    G.say(f"bf16 sddmm in place kdim={kdim} opts='{opts}'")
    sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices), vt, b16(lhs),
             b16(rhs), vt, sw.SDDMM_AFFINE, 0.125, 0.5, options=opts or None)
    torch.cuda.synchronize()
    _sddmm_check(orc, csr, vals, lhs, rhs, sw.SDDMM_AFFINE, 0.125, 0.5,
                 host(vt))


# ---- row reduce / row-wise map ---------------------------------------------


@pytest.mark.parametrize("opts", ["", "sddmm-lanes-per-row=64"])
def test_bf16_row_reduce_and_map(dev, orc, golden, opts):
    g = golden["row_reduce"]
    ro = G.t(np.array(g["row_offsets"], np.int32))
    val = b16(g["values"])
    s, m = nan_b16(3), nan_b16(3)
    G.say(f"bf16 row reduce golden opts='{opts}'")
    sw.csr_row_reduce(ro, None, val, s, "sum", options=opts)
    sw.csr_row_reduce(ro, None, val, m, "max", options=opts)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(s), g["expected_sum"])
    np.testing.assert_array_equal(host(m),
                                  [float(v) for v in g["expected_max"]])
    gs = golden["softmax"]
    e = nan_b16(4)
    sw.csr_rowwise_map(ro, None, val, m, e, sw.MAP_EXP_SUB, options=opts)
    sw.csr_row_reduce(ro, None, e, s, "sum", options=opts)
    sw.csr_rowwise_map(ro, None, e, s, e, sw.MAP_DIV, options=opts)
    torch.cuda.synchronize()
    assert np.all(within_steps(host(e), gs["expected"], 2))
    csr = W.random_csr(2000, 500, 30.0, 7, empty_fraction=0.2,
                       lognormal=True, max_len=500)
    vb = orc.as_bf16(csr.values)
    out = nan_b16(csr.rows)
    for kind, okind in (("sum", orc.REDUCE_SUM), ("max", orc.REDUCE_MAX)):
        sw.csr_row_reduce(G.t(csr.row_offsets), None, b16(vb), out, kind,
                          options=opts)
        torch.cuda.synchronize()
        ref = orc.row_reduce(csr.row_offsets, vb, okind)
        got = host(out)
        if kind == "max":
            np.testing.assert_array_equal(got, ref)  # a maximum is exact
        else:
            absb = np.add.reduceat(np.abs(vb.astype(np.float64)),
                                   csr.row_offsets[:-1].clip(0, csr.nnz - 1))
            absb[np.diff(csr.row_offsets) == 0] = 0
            assert_bf16_within_bound(got, ref, absb, what="row sum")
    rowv = orc.as_bf16(np.random.default_rng(1).uniform(0.5, 2, csr.rows))
    for kind in (sw.MAP_EXP_SUB, sw.MAP_DIV, sw.MAP_SUB, sw.MAP_MUL):
        o = nan_b16(csr.nnz)
        sw.csr_rowwise_map(G.t(csr.row_offsets), None, b16(vb), b16(rowv), o,
                           kind, options=opts)
        torch.cuda.synchronize()
        ref = orc.rowwise_map(csr.row_offsets, vb, rowv, kind)
        got = host(o)
        assert np.all(within_steps(got, ref, 1)), kind
        assert np.mean(got == orc.as_bf16(ref)) > 0.99


# ---- SpMM --------------------------------------------------------------------

SPMM_OPTS = ["", "spmm-mapping=wave-per-row-tile spmm-tile-size=4 "
             "spmm-block-size=64",
             "spmm-mapping=wave-per-row-tile spmm-tile-size=32 "
             "spmm-lanes-per-row=16",
             "spmm-mapping=wave-per-row-balanced spmm-block-size=1024",
             "spmm-mapping=row-tile-mfma"]


def _spmm_bf16(csr, vals, rhs, opts):
    out = nan_b16(csr.rows, rhs.shape[1])
    G.say(f"bf16 spmm rows={csr.rows} nnz={csr.nnz} k={rhs.shape[1]} "
          f"opts='{opts}'")
    sw.spmm(G.t(csr.row_offsets), G.t(csr.column_indices), b16(vals),
            b16(rhs), out, options=opts)
    torch.cuda.synchronize()
    return host(out)


@pytest.mark.parametrize("opts", SPMM_OPTS)
@pytest.mark.parametrize("k", [4, 64, 30])
@pytest.mark.parametrize("shape", ["random", "structure"])
def test_bf16_spmm(dev, orc, opts, k, shape):
    from tests.test_gpu_bsr_attention import _tile_structure_csr
    csr = (W.random_csr(700, 400, 25.0, k, empty_fraction=0.2, lognormal=True,
                        max_len=400) if shape == "random"
           else _tile_structure_csr())
    rhs = np.random.default_rng(k).standard_normal((csr.cols, k)).astype(
        np.float32)
    got = _spmm_bf16(csr, csr.values, rhs, opts)
    vb, rb = orc.as_bf16(csr.values), orc.as_bf16(rhs)
    ref = orc.spmm(csr.row_offsets, csr.column_indices, vb, rb)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices, vb, rb)
    assert_bf16_within_bound(got, ref, bound)
    ref32 = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    assert rel_l2(got, ref32) <= BF16_REL_L2


def test_bf16_spmm_rejects_output_accumulation(dev):
    csr = W.random_csr(64, 64, 4.0, 1)
    for mapping in ("wave-per-position", "thread-per-position"):
        with pytest.raises(sw.SparseWaveError, match="bf16 output cannot"):
            _spmm_bf16(csr, csr.values, np.ones((64, 4), np.float32),
                       f"spmm-mapping={mapping} spmm-block-size=64")


# ---- attention ---------------------------------------------------------------

FUSED = ("sddmm-mapping=row-tile-mfma sddmm-lanes-per-row=64 "
         "spmm-mapping=row-tile-mfma")
ATT_OPTS = ["", "sddmm-lanes-per-row=64 spmm-mapping=wave-per-row-tile "
            "spmm-tile-size=32 spmm-lanes-per-row=16", FUSED]


def _attention_bf16(csr, mask_vals, q, kt, v, alpha, beta, opts):
    G.say(f"bf16 attention rows={csr.rows} nnz={csr.nnz} d={q.shape[1]} "
          f"dv={v.shape[1]} opts='{opts}'")
    scores, rmax, rsum = nan_b16(csr.nnz), nan_b16(csr.rows), nan_b16(
        csr.rows)
    out = nan_b16(csr.rows, v.shape[1])
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        b16(mask_vals), b16(q), b16(kt), b16(v), scores, rmax,
                        rsum, out, alpha, beta, options=opts)
    torch.cuda.synchronize()
    return host(scores), host(rmax), host(rsum), host(out)


def _check_attention_bf16(orc, csr, mask_vals, q, kt, v, alpha, beta, got,
                          exact_frac=0.95):
    scores, rmax, rsum, out = got
    s_b, m_b, r_b, o_b = orc.sparse_attention_bf16(
        csr.row_offsets, csr.column_indices, mask_vals, q, kt, v, alpha, beta)
    # the oracle's bf16 chain: most values bit-equal, all within rel-L2
    # (empty rows hold the identities -inf and 0 in both)
    for name, a, b in (("scores", scores, s_b), ("row max", rmax, m_b),
                       ("row sum", rsum, r_b), ("output", out, o_b)):
        fin = np.isfinite(b)
        assert np.array_equal(a[~fin], b[~fin]), name
        assert rel_l2(a[fin], b[fin]) <= BF16_REL_L2, name
        assert np.mean(a == b) >= exact_frac, (name, np.mean(a == b))
    # the last op against the GPU's own (bf16) probabilities: the SpMM's
    # fp32 bar 1e-5 sum|P V| on the fp32 accumulation, then one bf16
    # rounding of the result (assert_bf16_within_bound adds 2^-8 |ref|)
    vb = orc.as_bf16(v)
    ref = orc.spmm(csr.row_offsets, csr.column_indices, scores, vb)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices, scores,
                               vb)
    assert_bf16_within_bound(out, ref, bound, what="output SpMM")
    # the fp32 chain on the unrounded inputs
    s32, m32, r32, o32 = orc.sparse_attention(
        csr.row_offsets, csr.column_indices, mask_vals, q, kt, v, alpha, beta)
    assert rel_l2(out, o32) <= BF16_REL_L2
    assert rel_l2(scores, s32) <= BF16_REL_L2
    assert rel_l2(rsum, r32) <= BF16_REL_L2


@pytest.mark.parametrize("opts", ATT_OPTS)
def test_bf16_attention_golden(dev, orc, golden, opts):
    g = golden["attention"]
    csr = W.CSR(2, 3, np.array(g["row_offsets"], np.int32),
                np.array(g["column_indices"], np.int32),
                np.array(g["mask_values"], np.float32))
    _, _, _, out = _attention_bf16(
        csr, csr.values, np.array(g["query"], np.float32),
        np.array(g["transposed_key"], np.float32),
        np.array(g["value"], np.float32), g["alpha"], g["beta"], opts)
    want = np.array(g["expected"], np.float64)
    assert np.all(np.abs(out - want) <= 2.0**-7 * np.abs(want) + 1e-4)


@pytest.mark.parametrize("opts", ATT_OPTS)
@pytest.mark.parametrize("seq", [1024, 8192])
def test_bf16_attention_config5(dev, orc, opts, seq):
    """Configuration 5 (seq 8192, d 64, 64 x 64 block mask) with the bf16
    option, against the oracle."""
    mask, q, kt, v, alpha = W.config5(seed=0, seq=seq)
    got = _attention_bf16(mask, mask.values, q, kt, v, alpha, 0.0, opts)
    _check_attention_bf16(orc, mask, mask.values, q, kt, v, alpha, 0.0, got)
    assert math.isfinite(float(got[3].sum()))


@pytest.mark.parametrize("shape", ["structure", "long"])
@pytest.mark.parametrize("d,dv", [(64, 64), (128, 128), (64, 80), (128, 16)])
def test_bf16_attention_fused_paths(dev, orc, shape, d, dv):
    """The bf16 fused kernel's register tiles and row-by-row fallbacks (dv a
    multiple of 64), and the bf16 six-op chain the same options select for
    other dv."""
    from tests.test_gpu_bsr_attention import (_long_prefix_csr,
                                              _tile_structure_csr)
    csr = _tile_structure_csr() if shape == "structure" else _long_prefix_csr()
    rng = np.random.default_rng(d + dv)
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    got = _attention_bf16(csr, csr.values, q, kt, v, 0.125, 0.5, FUSED)
    _check_attention_bf16(orc, csr, csr.values, q, kt, v, 0.125, 0.5, got,
                          exact_frac=0.9)


@pytest.mark.parametrize("nnz", [1, 2, 3, 4, 5, 6])
def test_bf16_attention_few_entries(dev, orc, nnz):
    """Matrices of one to six entries under the fused options: the bf16
    kernel's 4-entry mask windows near the buffer's end (nnz >= 4) and the
    op chain below that."""
    from tests.test_gpu_bsr_attention import _few_entries_csr
    csr = _few_entries_csr(nnz)
    rng = np.random.default_rng(nnz)
    q = rng.standard_normal((csr.rows, 64)).astype(np.float32)
    kt = rng.standard_normal((64, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, 64)).astype(np.float32)
    got = _attention_bf16(csr, csr.values, q, kt, v, 0.125, 0.5, FUSED)
    _check_attention_bf16(orc, csr, csr.values, q, kt, v, 0.125, 0.5, got,
                          exact_frac=0.9)


def test_bf16_attention_fused_empty_tile(dev, orc):
    """A tile of 16 empty rows between populated tiles under the fused
    options: the identities in its rows (row maximum -inf, row sum 0,
    output 0)."""
    from tests.test_gpu_bsr_attention import _empty_tile_csr
    csr = _empty_tile_csr()
    rng = np.random.default_rng(5)
    q = rng.standard_normal((csr.rows, 64)).astype(np.float32)
    kt = rng.standard_normal((64, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, 64)).astype(np.float32)
    got = _attention_bf16(csr, csr.values, q, kt, v, 0.125, 0.5, FUSED)
    _check_attention_bf16(orc, csr, csr.values, q, kt, v, 0.125, 0.5, got)
    _, rmax, rsum, out = got
    assert np.all(np.isneginf(rmax[16:32])) and np.all(rsum[16:32] == 0)
    assert np.all(out[16:32] == 0)


@pytest.mark.parametrize("opts", [FUSED] + ATT_OPTS[:2])
def test_bf16_attention_non_finite_value_rows(dev, orc, opts):
    """inf / NaN in V rows that a tile's last row includes and its shorter
    rows leave out reach exactly the rows whose entries name them."""
    from tests.test_gpu_bsr_attention import _tile_structure_csr
    csr = _tile_structure_csr()
    rng = np.random.default_rng(78)
    d = dv = 64
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    last = csr.column_indices[csr.row_offsets[15]:csr.row_offsets[16]]
    v[last[150], 3] = np.inf
    v[last[120], 7] = np.nan
    v[last[190], :] = -np.inf
    _, _, _, out = _attention_bf16(csr, csr.values, q, kt, v, 0.125, 0.5,
                                   opts)
    _, _, _, ref = orc.sparse_attention_bf16(
        csr.row_offsets, csr.column_indices, csr.values, q, kt, v, 0.125, 0.5)
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(out), cls(ref))
    fin = np.isfinite(ref)
    assert (~fin).any() and fin[:15].any()
    assert rel_l2(out[fin], ref[fin]) <= BF16_REL_L2


# ---- BSR SpMM ----------------------------------------------------------------


def _bsr_bf16(bsr, rhs, opts, out_dtype):
    G.say(f"bf16 bsr rows={bsr.rows} nnzb={bsr.nnzb} k={rhs.shape[1]} "
          f"out={out_dtype} opts='{opts}'")
    out = torch.full((bsr.rows, rhs.shape[1]), float("nan"), dtype=out_dtype,
                     device=G.DEV)
    sw.bsr_spmm(G.t(bsr.block_row_offsets), G.t(bsr.block_column_indices),
                b16(bsr.block_values), b16(rhs), out, bsr.block_size,
                options=opts)
    torch.cuda.synchronize()
    return host(out)


@pytest.mark.parametrize("opts", ["bsr-use-mfma=1", "bsr-use-mfma=0"])
@pytest.mark.parametrize("k", [128, 40, 200, 8, 30])
@pytest.mark.parametrize("out_dtype", [BF, torch.float32])
def test_bf16_bsr(dev, orc, opts, k, out_dtype):
    """k % 8 == 0 takes the column-interleaved kernel (partial strips at 40
    and 200); other k the scalar-load kernel."""
    bsr = W.bsr_banded(seed=k, rows=16 * 96, block_size=16, blocks_per_row=6,
                       band=3, band_blocks=3, value_std=0.5)
    rhs = np.random.default_rng(k).standard_normal((bsr.cols, k)).astype(
        np.float32)
    got = _bsr_bf16(bsr, rhs, opts, out_dtype)
    vb, rb = orc.as_bf16(bsr.block_values), orc.as_bf16(rhs)
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices, vb,
                       rb, 16)
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              vb, rb, 16)
    if out_dtype == BF:
        assert_bf16_within_bound(got, ref, bound)
    else:
        from tests._check import assert_within_bound
        assert_within_bound(got, ref, bound)
    ref32 = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                         bsr.block_values, rhs, 16)
    assert rel_l2(got, ref32) <= BF16_REL_L2


@pytest.mark.parametrize("out_dtype", [BF, torch.float32])
@pytest.mark.parametrize("k", [128, 64, 200, 40])
def test_bf16_bsr_ragged_block_rows(dev, orc, k, out_dtype):
    """Block rows of 0 to 9 blocks through the bf16 MFMA kernels, which split
    a block row's blocks over several waves."""
    from tests._check import assert_within_bound
    from tests.test_gpu_bsr_attention import _ragged_bsr
    bsr = _ragged_bsr(k)
    rhs = np.random.default_rng(k + 1).standard_normal(
        (bsr.cols, k)).astype(np.float32)
    got = _bsr_bf16(bsr, rhs, "bsr-use-mfma=1", out_dtype)
    vb, rb = orc.as_bf16(bsr.block_values), orc.as_bf16(rhs)
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices, vb,
                       rb, 16)
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              vb, rb, 16)
    if out_dtype == BF:
        assert_bf16_within_bound(got, ref, bound)
    else:
        assert_within_bound(got, ref, bound)


@pytest.mark.parametrize("opts,out_dtype", [
    ("bsr-use-mfma=1", BF), ("bsr-use-mfma=1", torch.float32),
    # the reference's thread-per-output mapping, as bench.py times it
    ("bsr-use-mfma=0", BF)])
def test_bf16_bsr_config4_sample(dev, orc, opts, out_dtype):
    """Configuration 4 at full size (262,144 rows, 131,072 blocks, k = 128)
    in bf16; 400 block rows (first, last, random) checked against the
    oracle on the bf16-rounded inputs."""
    bsr, rhs = W.config4(seed=0)
    got = _bsr_bf16(bsr, rhs, opts, out_dtype)
    brs = np.unique(np.concatenate([
        [0, 1, bsr.rows // 16 - 1],
        np.random.default_rng(1).choice(bsr.rows // 16, 400, replace=False)]))
    bro = bsr.block_row_offsets
    counts = bro[brs + 1] - bro[brs]
    sub_ro = np.zeros(brs.size + 1, np.int64)
    np.cumsum(counts, out=sub_ro[1:])
    idx = np.concatenate([np.arange(bro[b], bro[b + 1]) for b in brs])
    sub_vals = bsr.block_values.reshape(-1, 256)[idx].ravel()
    sub_ro = sub_ro.astype(np.int32)
    vb, rb = orc.as_bf16(sub_vals), orc.as_bf16(rhs)
    ref = orc.bsr_spmm(sub_ro, bsr.block_column_indices[idx], vb, rb, 16)
    bound = orc.bsr_abs_bound(sub_ro, bsr.block_column_indices[idx], vb, rb,
                              16)
    rows = (brs[:, None] * 16 + np.arange(16)[None, :]).ravel()
    if out_dtype == BF:
        assert_bf16_within_bound(got[rows], ref, bound)
    else:
        from tests._check import assert_within_bound
        assert_within_bound(got[rows], ref, bound)
    ref32 = orc.bsr_spmm(sub_ro, bsr.block_column_indices[idx], sub_vals, rhs,
                         16)
    assert rel_l2(got[rows], ref32) <= BF16_REL_L2
    assert np.all(np.isfinite(got))


# ---- misaligned operands: the vector fallbacks ---------------------------


def _b16_misaligned(a):
    """A bf16 device view of a that starts 2 bytes past an aligned address,
    so every 8- and 16-byte alignment check fails."""
    a = np.asarray(a, np.float32)
    flat = torch.empty(a.size + 1, dtype=BF, device=G.DEV)
    view = flat[1:].view(a.shape)
    view.copy_(b16(a))
    return view


def test_bf16_misaligned_operands(dev, orc):
    """bf16 SDDMM, SpMM, BSR and the fused attention options with operands
    that miss the matrix-core paths' alignment: the vector kernels run and
    keep the same results."""
    from tests.test_gpu_bsr_attention import _tile_structure_csr
    csr = _tile_structure_csr()
    rng = np.random.default_rng(11)
    d = dv = 64
    q = rng.standard_normal((csr.rows, d)).astype(np.float32)
    kt = rng.standard_normal((d, csr.cols)).astype(np.float32)
    v = rng.standard_normal((csr.cols, dv)).astype(np.float32)
    G.say("bf16 misaligned sddmm / spmm / attention")
    out = nan_b16(csr.nnz)
    sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices),
             b16(csr.values), _b16_misaligned(q), b16(kt), out,
             sw.SDDMM_AFFINE, 0.125, 0.5,
             options="sddmm-mapping=row-tile-mfma")
    torch.cuda.synchronize()
    _sddmm_check(orc, csr, csr.values, q, kt, sw.SDDMM_AFFINE, 0.125, 0.5,
                 host(out))
    o = nan_b16(csr.rows, dv)
    sw.spmm(G.t(csr.row_offsets), G.t(csr.column_indices), b16(csr.values),
            _b16_misaligned(v), o, options="spmm-mapping=row-tile-mfma")
    torch.cuda.synchronize()
    vb, rb = orc.as_bf16(csr.values), orc.as_bf16(v)
    ref = orc.spmm(csr.row_offsets, csr.column_indices, vb, rb)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices, vb, rb)
    assert_bf16_within_bound(host(o), ref, bound)
    scores, rmax, rsum = nan_b16(csr.nnz), nan_b16(csr.rows), nan_b16(
        csr.rows)
    att = nan_b16(csr.rows, dv)
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        b16(csr.values), _b16_misaligned(q), b16(kt),
                        _b16_misaligned(v), scores, rmax, rsum, att, 0.125,
                        0.5, options=FUSED)
    torch.cuda.synchronize()
    _check_attention_bf16(orc, csr, csr.values, q, kt, v, 0.125, 0.5,
                          (host(scores), host(rmax), host(rsum), host(att)),
                          exact_frac=0.9)
    bsr = W.bsr_banded(seed=5, rows=16 * 64, block_size=16, blocks_per_row=6,
                       band=3, band_blocks=3, value_std=0.5)
    rhs = rng.standard_normal((bsr.cols, 128)).astype(np.float32)
    ob = nan_b16(bsr.rows, 128)
    G.say("bf16 misaligned bsr")
    sw.bsr_spmm(G.t(bsr.block_row_offsets), G.t(bsr.block_column_indices),
                b16(bsr.block_values), _b16_misaligned(rhs), ob, 16,
                options="bsr-use-mfma=1")
    torch.cuda.synchronize()
    vb, rb = orc.as_bf16(bsr.block_values), orc.as_bf16(rhs)
    ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices, vb,
                       rb, 16)
    bound = orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                              vb, rb, 16)
    assert_bf16_within_bound(host(ob), ref, bound)
