"""Pins of the CPU oracle (oracle/sw_oracle.c).

Each oracle function is checked against (a) the golden vectors of the
reference's own runtime tests, (b) an independent computation (scipy.sparse,
dense numpy in float64, numpy.searchsorted, brute force), and (c) mutation
cases showing that a plausible mistake -- a dropped term, a transposed
operand, a wrong index -- fails the same check.
"""
import math

import numpy as np
import pytest
import scipy.sparse as sp

from sparsewavecomp_amd import workloads as W
from tests._check import assert_within_bound, rel_l2


def _csr(g):
    return (np.array(g["row_offsets"], np.int32),
            np.array(g["column_indices"], np.int32),
            np.array(g["values"], np.float32))


def _scipy(csr):
    return sp.csr_matrix((csr.values.astype(np.float64),
                          csr.column_indices, csr.row_offsets),
                         shape=(csr.rows, csr.cols))


# ---- golden vectors ------------------------------------------------------


@pytest.mark.parametrize("case", ["spmv", "spmv_sparse_tensor"])
def test_golden_spmv(orc, golden, case):
    g = golden[case]
    ro, col, val = _csr(g)
    y = orc.spmv(ro, col, val, np.array(g["vector"], np.float32))
    np.testing.assert_array_equal(y, np.array(g["expected"], np.float32))
    y = orc.spmv_wave_position(ro, col, val, np.array(g["vector"], np.float32))
    np.testing.assert_array_equal(y, np.array(g["expected"], np.float32))


def test_golden_coo_spmv(orc, golden):
    g = golden["coo_spmv"]
    y, bound = orc.spmv_coo(g["rows"], g["row_indices"], g["column_indices"],
                            g["values"], np.array(g["vector"], np.float32))
    np.testing.assert_array_equal(y, np.array(g["expected"], np.float32))
    # all products are positive here, so the magnitude bound is the sum
    np.testing.assert_array_equal(bound, np.array(g["expected"]))


def _random_coo(rng, rows, cols, nnz, sort):
    ri = rng.integers(0, rows, nnz).astype(np.int32)
    ci = rng.integers(0, cols, nnz).astype(np.int32)
    if sort:
        o = np.lexsort((ci, ri))
        ri, ci = ri[o], ci[o]
    val = rng.uniform(-1, 1, nnz).astype(np.float32)
    return ri, ci, val


@pytest.mark.parametrize("sort", [True, False])
def test_coo_spmv_matches_scipy(orc, sort):
    """scipy's coo_matrix adds repeated coordinates, as the op does."""
    rng = np.random.default_rng(11)
    rows, cols = 300, 200
    ri, ci, val = _random_coo(rng, rows, cols, 4000, sort)
    ri[:50] = ri[50]  # a run of one row with repeated coordinates
    ci[:50] = 7
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    y, bound = orc.spmv_coo(rows, ri, ci, val, x)
    a = sp.coo_matrix((val.astype(np.float64), (ri, ci)), shape=(rows, cols))
    ref = a @ x.astype(np.float64)
    assert_within_bound(y, ref, bound)
    # mutation: dropping repeated coordinates (keeping the first) fails
    _, first = np.unique(np.stack([ri, ci], 1), axis=0, return_index=True)
    keep = np.sort(first)
    y_bad, _ = orc.spmv_coo(rows, ri[keep], ci[keep], val[keep], x)
    with pytest.raises(AssertionError):
        assert_within_bound(y_bad, ref, bound)


def _run_segmented_emulation(rows, ri, ci, val, x, P, wave=64):
    """Lane-by-lane emulation of the run-segmented COO kernel's emission
    rule (runs in a lane, a scan over the lanes' last runs keyed on run
    numbers, head/tail hand-off between neighbours); products in float64 so
    the comparison isolates the emission logic."""
    y = np.zeros(rows)
    nnz = ri.size
    lanes = -(-nnz // P)
    for w0 in range(0, lanes, wave):
        L = []
        for u in range(w0, min(w0 + wave, lanes)):
            seg = list(range(u * P, min(u * P + P, nnz)))
            runs = []
            for p in seg:
                pr = float(val[p]) * float(x[ci[p]])
                if runs and runs[-1][0] == ri[p]:
                    runs[-1][1] += pr
                else:
                    runs.append([int(ri[p]), pr])
            L.append(runs)
        L += [None] * (wave - len(L))
        tails, keys = [], []
        for i, runs in enumerate(L):
            if runs is None:
                keys.append(None)
                tails.append(0.0)
                continue
            prev = L[i - 1][-1][0] if i and L[i - 1] else None
            cont = len(runs) == 1 and runs[0][0] == prev
            tails.append(runs[-1][1] + (tails[i - 1] if cont else 0.0))
            keys.append(runs[-1][0])
        for i, runs in enumerate(L):
            if runs is None:
                continue
            prev_t = keys[i - 1] if i else None
            if len(runs) > 1:
                h = runs[0][1] + (tails[i - 1] if prev_t == runs[0][0] else 0)
                y[runs[0][0]] += h
                for r, s in runs[1:-1]:
                    y[r] += s
            nxt = L[i + 1][0][0] if i + 1 < wave and L[i + 1] else None
            if nxt != runs[-1][0]:
                y[runs[-1][0]] += tails[i]
    return y


@pytest.mark.parametrize("sort", [True, False])
@pytest.mark.parametrize("P", [1, 4, 16])
def test_run_segmented_emission_rule(orc, sort, P):
    """The emission rule of the run-segmented COO kernel delivers every
    entry exactly once, for sorted and unsorted entries, runs that cross
    lanes and waves, and ragged final lanes."""
    rng = np.random.default_rng(P + 2 * sort)
    rows, cols = 40, 30
    ri, ci, val = _random_coo(rng, rows, cols, 64 * P * 2 + 37, sort)
    ri[100:100 + 3 * P * 64 // 2] = 5  # one row spanning lanes and waves
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    y = _run_segmented_emulation(rows, ri, ci, val, x, P)
    _, bound = orc.spmv_coo(rows, ri, ci, val, x)
    ref = np.zeros(rows)
    np.add.at(ref, ri, val.astype(np.float64) * x[ci])
    np.testing.assert_allclose(y, ref, rtol=0, atol=1e-9 * (1 + bound.max()))


@pytest.mark.parametrize("case", ["spmm", "spmm_torch_example"])
def test_golden_spmm(orc, golden, case):
    g = golden[case]
    ro, col, val = _csr(g)
    out = orc.spmm(ro, col, val, np.array(g["rhs"], np.float32))
    np.testing.assert_array_equal(out, np.array(g["expected"], np.float32))


def test_golden_bsr(orc, golden):
    g = golden["bsr_spmm"]
    out = orc.bsr_spmm(np.array(g["block_row_offsets"], np.int32),
                       np.array(g["block_column_indices"], np.int32),
                       np.array(g["block_values"], np.float32),
                       np.array(g["rhs"], np.float32), g["block_size"])
    np.testing.assert_array_equal(out, np.array(g["expected"], np.float32))


def test_golden_sddmm(orc, golden):
    g = golden["sddmm"]
    ro, col, val = _csr(g)
    out = orc.sddmm(ro, col, val, np.array(g["lhs"], np.float32),
                    np.array(g["rhs"], np.float32), orc.SDDMM_MUL)
    np.testing.assert_array_equal(out, np.array(g["expected"], np.float32))


def test_golden_row_reduce(orc, golden):
    g = golden["row_reduce"]
    ro, _, val = _csr(g)
    np.testing.assert_array_equal(orc.row_reduce(ro, val, orc.REDUCE_SUM),
                                  np.array(g["expected_sum"], np.float32))
    want = np.array([float(v) for v in g["expected_max"]], np.float32)
    np.testing.assert_array_equal(orc.row_reduce(ro, val, orc.REDUCE_MAX),
                                  want)


def test_golden_softmax(orc, golden):
    g = golden["softmax"]
    ro, _, val = _csr(g)
    m = orc.row_reduce(ro, val, orc.REDUCE_MAX)
    e = orc.rowwise_map(ro, val, m, orc.MAP_EXP_SUB)
    s = orc.row_reduce(ro, e, orc.REDUCE_SUM)
    p = orc.rowwise_map(ro, e, s, orc.MAP_DIV)
    # the reference prints 6 significant digits
    np.testing.assert_allclose(p, g["expected"], rtol=0, atol=5e-7)


def test_golden_attention(orc, golden):
    g = golden["attention"]
    ro = np.array(g["row_offsets"], np.int32)
    col = np.array(g["column_indices"], np.int32)
    _, _, _, out = orc.sparse_attention(
        ro, col, np.array(g["mask_values"], np.float32),
        np.array(g["query"], np.float32),
        np.array(g["transposed_key"], np.float32),
        np.array(g["value"], np.float32), g["alpha"], g["beta"])
    want = np.array(g["expected"], np.float64)
    # CHECK matches 4.2177..., 5.2177..., 3, 4: compare the printed prefix
    np.testing.assert_allclose(
        np.floor(out.astype(np.float64) * 1e4) / 1e4, want, rtol=0, atol=1e-9)


# ---- independent computations on random inputs ----------------------------


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_spmv_matches_scipy(orc, seed):
    csr = W.random_csr(300, 200, 12.0, seed, empty_fraction=0.2)
    x = np.random.default_rng(seed).uniform(-1, 1, 200).astype(np.float32)
    y = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    exact = _scipy(csr) @ x.astype(np.float64)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    assert_within_bound(y, exact, bound)
    # bound is sum|a*x| computed independently
    np.testing.assert_allclose(bound, abs(_scipy(csr)) @ np.abs(x), rtol=1e-12)


def test_spmv_mutations_fail(orc):
    csr = W.random_csr(200, 150, 10.0, 5, empty_fraction=0.1)
    x = np.random.default_rng(5).uniform(-1, 1, 150).astype(np.float32)
    exact = _scipy(csr) @ x.astype(np.float64)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    mutants = {
        "reversed vector": orc.spmv(csr.row_offsets, csr.column_indices,
                                    csr.values, x[::-1].copy()),
        "dropped last term": orc.spmv(
            csr.row_offsets, csr.column_indices,
            np.where(np.isin(np.arange(csr.nnz), csr.row_offsets[1:] - 1),
                     0, csr.values).astype(np.float32), x),
        "shifted row offsets": orc.spmv(
            np.minimum(csr.row_offsets + 1, csr.nnz).astype(np.int32),
            csr.column_indices, csr.values, x),
    }
    for name, y in mutants.items():
        with pytest.raises(AssertionError):
            assert_within_bound(y, exact, bound, what=name)


@pytest.mark.parametrize("k", [1, 4, 7])
def test_spmm_matches_scipy(orc, k):
    csr = W.random_csr(120, 90, 8.0, 11, empty_fraction=0.2)
    rhs = np.random.default_rng(3).uniform(-1, 1, (90, k)).astype(np.float32)
    out = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    exact = _scipy(csr) @ rhs.astype(np.float64)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, rhs)
    assert_within_bound(out, exact, bound)
    if k > 1:  # transposed-operand mutation: reversing rhs columns must fail
        with pytest.raises(AssertionError):
            assert_within_bound(out[:, ::-1], exact, bound)


def _bsr_dense(bsr):
    b = bsr.block_size
    dense = np.zeros((bsr.rows, bsr.cols), np.float64)
    blocks = bsr.block_values.reshape(-1, b, b)
    for br in range(bsr.rows // b):
        for bp in range(bsr.block_row_offsets[br],
                        bsr.block_row_offsets[br + 1]):
            bc = bsr.block_column_indices[bp]
            dense[br * b:(br + 1) * b, bc * b:(bc + 1) * b] = blocks[bp]
    return dense


@pytest.mark.parametrize("b", [2, 4, 16])
def test_bsr_matches_dense(orc, b):
    bsr = W.bsr_banded(seed=b, rows=b * 24, block_size=b, blocks_per_row=5,
                       band=2, band_blocks=2, value_std=1.0)
    rhs = np.random.default_rng(b).standard_normal((bsr.cols, 6)).astype(
        np.float32)
    out = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                       bsr.block_values, rhs, b)
    dense = _bsr_dense(bsr)
    exact = dense @ rhs.astype(np.float64)
    bound = np.abs(dense) @ np.abs(rhs.astype(np.float64))
    assert_within_bound(out, exact, bound)
    np.testing.assert_allclose(
        orc.bsr_abs_bound(bsr.block_row_offsets, bsr.block_column_indices,
                          bsr.block_values, rhs, b), bound, rtol=1e-12)
    # transposed blocks must fail
    tb = bsr.block_values.reshape(-1, b, b).transpose(0, 2, 1).ravel()
    bad = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices, tb,
                       rhs, b)
    with pytest.raises(AssertionError):
        assert_within_bound(bad, exact, bound)


def test_sddmm_matches_dense(orc):
    csr = W.random_csr(50, 40, 9.0, 21, empty_fraction=0.2)
    rng = np.random.default_rng(21)
    lhs = rng.standard_normal((50, 16)).astype(np.float32)
    rhs = rng.standard_normal((16, 40)).astype(np.float32)
    dense = lhs.astype(np.float64) @ rhs.astype(np.float64)
    absd = np.abs(lhs.astype(np.float64)) @ np.abs(rhs.astype(np.float64))
    rows = np.repeat(np.arange(50), np.diff(csr.row_offsets))
    dot = dense[rows, csr.column_indices]
    bound = absd[rows, csr.column_indices]
    v = csr.values.astype(np.float64)
    for kind, want, scale in [
            (orc.SDDMM_MUL, v * dot, np.abs(v) * bound),
            (orc.SDDMM_DOT, dot, bound),
            (orc.SDDMM_AFFINE, 0.5 * v + 0.25 * dot,
             0.5 * np.abs(v) + 0.25 * bound)]:
        out = orc.sddmm(csr.row_offsets, csr.column_indices, csr.values, lhs,
                        rhs, kind, 0.25, 0.5)
        assert_within_bound(out, want, scale + 1e-30)
    # using lhs rows of the wrong row (index mistake) must fail
    out = orc.sddmm(csr.row_offsets, csr.column_indices, csr.values,
                    lhs[::-1].copy(), rhs, orc.SDDMM_DOT)
    with pytest.raises(AssertionError):
        assert_within_bound(out, dot, bound)


def test_row_reduce_and_map_match_numpy(orc):
    csr = W.random_csr(80, 60, 6.0, 31, empty_fraction=0.3)
    ro, v = csr.row_offsets, csr.values
    s = orc.row_reduce(ro, v, orc.REDUCE_SUM)
    m = orc.row_reduce(ro, v, orc.REDUCE_MAX)
    for r in range(csr.rows):
        seg = v[ro[r]:ro[r + 1]].astype(np.float64)
        assert abs(s[r] - seg.sum()) <= 1e-6 * max(1.0, np.abs(seg).sum())
        assert m[r] == (seg.max() if seg.size else -np.inf)
    # NaN propagates through max (arith.maximumf)
    v2 = v.copy()
    if csr.nnz:
        v2[ro[np.argmax(np.diff(ro) > 0)]] = np.nan
        assert np.isnan(orc.row_reduce(ro, v2, orc.REDUCE_MAX)).any()
    rowv = np.random.default_rng(1).uniform(0.5, 2, csr.rows).astype(
        np.float32)
    rows = np.repeat(np.arange(csr.rows), np.diff(ro))
    for kind, fn in [(orc.MAP_EXP_SUB, lambda a, b: np.exp(a - b)),
                     (orc.MAP_DIV, lambda a, b: a / b),
                     (orc.MAP_SUB, lambda a, b: a - b),
                     (orc.MAP_MUL, lambda a, b: a * b)]:
        out = orc.rowwise_map(ro, v, rowv, kind)
        want = fn(v.astype(np.float64), rowv[rows].astype(np.float64))
        np.testing.assert_allclose(out, want, rtol=2e-6, atol=1e-7)


def _dense_attention(mask, q, kt, v, alpha):
    rows = np.repeat(np.arange(mask.rows), np.diff(mask.row_offsets))
    s = alpha * (q.astype(np.float64) @ kt.astype(np.float64))
    dense = np.full((mask.rows, mask.cols), -np.inf)
    dense[rows, mask.column_indices] = s[rows, mask.column_indices]
    mx = dense.max(axis=1, keepdims=True)
    mx[~np.isfinite(mx)] = 0
    e = np.exp(dense - mx)
    den = e.sum(axis=1, keepdims=True)
    den[den == 0] = 1
    p = e / den
    return p @ v.astype(np.float64), np.abs(p) @ np.abs(v.astype(np.float64))


def test_attention_matches_dense_softmax(orc):
    mask = W.attention_mask(seq=256, block=16, window=3, random_blocks=2,
                            seed=4)
    rng = np.random.default_rng(4)
    q = rng.standard_normal((256, 8)).astype(np.float32)
    k = rng.standard_normal((256, 8)).astype(np.float32)
    v = rng.standard_normal((256, 8)).astype(np.float32)
    kt = np.ascontiguousarray(k.T)
    alpha = 1 / math.sqrt(8)
    _, _, _, out = orc.sparse_attention(mask.row_offsets, mask.column_indices,
                                        mask.values, q, kt, v, alpha)
    want, bound = _dense_attention(mask, q, kt, v, alpha)
    tol = _fp32_chain_vs_exact_tolerance(orc, mask, q, kt, v, alpha)
    assert np.all(np.abs(out - want) <= tol)
    # the bound is not vacuous: at most 1e-4 of sum |P V| on every output
    assert np.all(tol <= 1e-4 * bound)
    # a non-transposed key (operand mistake) must fail
    _, _, _, bad = orc.sparse_attention(mask.row_offsets, mask.column_indices,
                                        mask.values, q, np.ascontiguousarray(
                                            kt.reshape(256, 8).T), v, alpha)
    assert not np.all(np.abs(bad - want) <= tol)


def _fp32_chain_vs_exact_tolerance(orc, mask, q, kt, v, alpha):
    """|out_fp32 - out_exact| for the oracle's fp32 chain: each score is a
    d-term fp32 dot product and one scaling, so |s - s_exact| <= (d + 2) u
    B_p (u = 2^-24, B_p = |alpha| sum_k |q_rk kt_kc|); the probabilities
    then obey the softmax bound of tests/_attention_check.py with that E_r,
    and the output SpMM adds its sequential-sum rounding (n_r + 2) u
    sum_p |P_p V_pc| to sum_p tolP_p |V_pc|."""
    from tests._attention_check import (U, row_error, score_bounds,
                                        tolerances)
    d = q.shape[1]
    s_ref, m_ref, _, _ = orc.sparse_attention(
        mask.row_offsets, mask.column_indices, mask.values, q, kt, v, alpha)
    raw = orc.sddmm(mask.row_offsets, mask.column_indices, mask.values, q, kt,
                    orc.SDDMM_AFFINE, alpha, 0.0).astype(np.float64)
    rows = np.repeat(np.arange(mask.rows), np.diff(mask.row_offsets))
    e_row = row_error(mask, (d + 2) * U * score_bounds(orc, 
        mask, mask.values, q, kt, alpha, 0.0), raw)
    tol_p, _ = tolerances(mask, s_ref, raw - m_ref[rows], e_row)
    n = np.diff(mask.row_offsets).astype(np.float64)
    pv = orc.spmm_abs_bound(mask.row_offsets, mask.column_indices, s_ref, v)
    carried = orc.spmm_abs_bound(mask.row_offsets, mask.column_indices,
                                 tol_p.astype(np.float32), v)
    return carried + (n[:, None] + 2) * U * pv


def test_attention_checker_accepts_oracle_and_rejects_mistakes(orc):
    """tests/_attention_check.check_attention_f32 (the GPU tests' checker)
    passes the oracle's own chain and fails planted mistakes: one
    probability moved by 1e-3 of itself, a row maximum off by 1e-3, a
    wrong alpha, and an output element moved by 1e-4 of sum |P V|."""
    from tests._attention_check import check_attention_f32
    mask = W.attention_mask(seq=256, block=16, window=3, random_blocks=2,
                            seed=7)
    rng = np.random.default_rng(7)
    q = rng.standard_normal((256, 16)).astype(np.float32)
    kt = rng.standard_normal((16, 256)).astype(np.float32)
    v = rng.standard_normal((256, 16)).astype(np.float32)
    mv = rng.uniform(-1, 1, mask.nnz).astype(np.float32)
    mv[rng.random(mask.nnz) < 0.1] = -np.inf
    alpha, beta = 0.25, 0.5
    refs = orc.sparse_attention(mask.row_offsets, mask.column_indices, mv, q,
                                kt, v, alpha, beta)
    s, m, r, o = refs
    check_attention_f32(orc, mask, mv, q, kt, v, alpha, beta, s, m, r, o)
    p = int(np.argmax(s))
    for what in ("p", "m", "alpha", "o"):
        s2, m2, r2, o2 = (a.copy() for a in refs)
        if what == "p":
            s2[p] *= 1 + 1e-3
        elif what == "m":
            m2[3] += 1e-3 * max(1.0, abs(m2[3]))
        elif what == "alpha":
            s2, m2, r2, o2 = orc.sparse_attention(
                mask.row_offsets, mask.column_indices, mv, q, kt, v,
                alpha * 1.01, beta)
        else:
            pv = orc.spmm_abs_bound(mask.row_offsets, mask.column_indices,
                                    s, v)
            o2[5, 2] += 1e-4 * pv[5, 2]
        with pytest.raises(AssertionError):
            check_attention_f32(orc, mask, mv, q, kt, v, alpha, beta, s2, m2,
                                r2, o2)


# ---- index work: bit-exact ------------------------------------------------


@pytest.mark.parametrize("seed", [0, 1])
def test_row_search_matches_searchsorted(orc, seed):
    csr = W.random_csr(500, 100, 3.0, seed, empty_fraction=0.4)
    pos = np.arange(csr.nnz, dtype=np.int64)
    rows = orc.rows_at_positions(csr.row_offsets, pos)
    want = np.searchsorted(csr.row_offsets[1:], pos, side="right")
    np.testing.assert_array_equal(rows, want)
    # brute force: ro[r] <= p < ro[r+1]
    ro = csr.row_offsets
    assert np.all(ro[rows] <= pos) and np.all(pos < ro[rows + 1])


def test_row_search_tiny_bruteforce(orc):
    ro = np.array([0, 0, 3, 3, 3, 4, 8, 8], np.int32)
    for p in range(8):
        want = [r for r in range(7) if ro[r] <= p < ro[r + 1]][0]
        assert orc.rows_at_positions(ro, [p])[0] == want


@pytest.mark.parametrize("span,workers", [(0, 3), (10, 3), (64, 64),
                                          (1000, 37), (7, 10)])
def test_position_space_partition(orc, span, workers):
    lo = 5
    parts = [orc.position_space(lo, lo + span, w, workers)
             for w in range(workers)]
    assert parts[0][0] == lo and parts[-1][1] == lo + span
    for (b0, e0), (b1, _) in zip(parts, parts[1:]):
        assert e0 == b1
    sizes = [e - b for b, e in parts]
    assert max(sizes) - min(sizes) <= 1
    assert sizes == sorted(sizes, reverse=True)


def test_wave_segmented_scan_bruteforce(orc):
    rng = np.random.default_rng(9)
    for wave in (32, 64):
        for _ in range(20):
            n_active = int(rng.integers(0, wave + 1))
            keys = np.sort(rng.integers(0, 6, wave)).astype(np.int64)
            vals = rng.integers(-4, 5, wave).astype(np.float32)
            act = np.arange(wave) < n_active
            out, seg = orc.wave_segmented_scan(keys, vals, act)
            for l in range(wave):
                if not act[l]:
                    assert not seg[l]
                    continue
                start = l
                while start > 0 and keys[start - 1] == keys[l]:
                    start -= 1
                assert out[l] == vals[start:l + 1].sum()
            # each segment emitted exactly once
            ends = [l for l in range(n_active) if seg[l]]
            assert len(ends) == len(np.unique(keys[:n_active]))


@pytest.mark.parametrize("block", [64, 256])
def test_wave_position_schedule_equals_row_sum(orc, block):
    csr = W.random_csr(400, 300, 20.0, 8, empty_fraction=0.2, lognormal=True)
    x = np.random.default_rng(8).uniform(-1, 1, 300).astype(np.float32)
    ref = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    y = orc.spmv_wave_position(csr.row_offsets, csr.column_indices,
                               csr.values, x, block=block, wave=64)
    assert_within_bound(y, ref, bound)


def test_bf16_tolerance_helper():
    a = np.ones(100)
    assert rel_l2(a, a) == 0.0
    assert abs(rel_l2(a * 1.01, a) - 0.01) < 1e-12


def test_multithreaded_spmv_equals_scalar(orc):
    """The all-cores CPU extra computes the same rows in the same order."""
    csr = W.random_csr(5000, 3000, 20.0, 12, empty_fraction=0.1)
    x = np.random.default_rng(12).uniform(-1, 1, 3000).astype(np.float32)
    a = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    b = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x,
                 threads=True)
    np.testing.assert_array_equal(a, b)


def test_spmm_abs_bound_matches_scipy(orc):
    """oracle_spmm_abs_bound is |A| @ |B| computed independently (scipy in
    float64); a bound that drops a term or takes the wrong rhs column must
    differ."""
    for k in (1, 3, 8):
        csr = W.random_csr(150, 110, 9.0, 31 + k, empty_fraction=0.25)
        rhs = np.random.default_rng(k).uniform(-2, 2, (110, k)).astype(
            np.float32)
        bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                                   csr.values, rhs)
        want = abs(_scipy(csr)) @ np.abs(rhs.astype(np.float64))
        np.testing.assert_allclose(bound, want, rtol=1e-12, atol=0)
        # mutation: the signed sum instead of the sum of magnitudes
        signed = _scipy(csr) @ rhs.astype(np.float64)
        assert not np.allclose(np.abs(signed), want, rtol=1e-6)
        if k > 1:  # columns swapped must not match
            assert not np.allclose(bound[:, ::-1], want, rtol=1e-6)


# ---- bf16 ----------------------------------------------------------------


def _torch_bf16_bits(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(
        torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)


def test_round_bf16_matches_torch(orc):
    """oracle_round_bf16 against torch's float32 -> bfloat16 conversion
    (round to nearest even) over random bit patterns of every exponent,
    exact ties, subnormals, overflow and non-finite values."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2**16, 20000, dtype=np.uint64).astype(np.uint32)
            << 16) | 0x8000
    special = np.array([0, 0x80000000, 0x00000001, 0x807FFFFF, 0x7F7FFFFF,
                        0x7F7F8000, 0x7F7F7FFF, 0xFF7FFFFF, 0x7F800000,
                        0xFF800000, 0x7FC00000, 0x7F800001, 0xFFFFFFFF,
                        0x3F808000, 0x3F818000], np.uint32)
    x = np.concatenate([bits, ties, special]).view(np.float32)
    got = orc.round_bf16(x)
    want = _torch_bf16_bits(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(orc.bf16_to_f32(got[nan])))
    # widening is exact: the pattern shifted into the upper half
    h = rng.integers(0, 2**16, 1000, dtype=np.uint64).astype(np.uint16)
    w = orc.bf16_to_f32(h)
    np.testing.assert_array_equal(w.view(np.uint32), h.astype(np.uint32) << 16)


def test_round_bf16_hand_cases(orc):
    one = np.float32(1.0)
    cases = {1 + 2.0**-8: 1.0,             # tie -> even (fraction 0)
             1 + 3 * 2.0**-8: 1 + 2.0**-6,  # tie -> even (fraction 2)
             1 + 2.0**-8 + 2.0**-20: 1 + 2.0**-7,  # above the tie
             -(1 + 2.0**-7): -(1 + 2.0**-7),       # exact
             3.4e38: float("inf")}                 # overflow
    for x, want in cases.items():
        got = orc.as_bf16(np.array([x], np.float32))[0]
        assert got == np.float32(want), (x, got, want)
    assert orc.as_bf16(np.array([one]))[0] == one


def _dense_attention_bf16_staged(mask, q, kt, v, alpha):
    """The six ops on bf16 buffers as dense torch algebra: each op's result
    rounded with torch's bfloat16 conversion (an implementation independent
    of the oracle's CSR loops, expf and rounding)."""
    import torch
    r = lambda t: t.to(torch.bfloat16).to(torch.float32)
    rows = np.repeat(np.arange(mask.rows), np.diff(mask.row_offsets))
    cols = mask.column_indices
    Q = r(torch.from_numpy(q))
    KT = r(torch.from_numpy(kt))
    V = r(torch.from_numpy(v))
    s = r((Q.double() @ KT.double()).float()[rows, cols] * np.float32(alpha))
    n = mask.rows
    dense = torch.full((n, mask.cols), -float("inf"))
    dense[rows, cols] = s
    mx = dense.max(dim=1).values
    e = r(torch.exp(s - mx[rows]))
    rsum = r(torch.zeros(n).index_add_(0, torch.from_numpy(rows), e))
    p = r(e / rsum[rows])
    P = torch.zeros(n, mask.cols, dtype=torch.float64)
    P[rows, cols] = p.double()
    out = r((P @ V.double()).float())
    bound = (P.abs() @ V.double().abs()).numpy()
    return (s.numpy(), mx.numpy(), rsum.numpy(), p.numpy(), out.numpy(),
            bound)


def test_attention_bf16_matches_dense_staged(orc):
    mask = W.attention_mask(seq=256, block=16, window=3, random_blocks=2,
                            seed=5)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((256, 16)).astype(np.float32)
    kt = rng.standard_normal((16, 256)).astype(np.float32)
    v = rng.standard_normal((256, 16)).astype(np.float32)
    alpha = 0.25
    sc, mx, rs, out = orc.sparse_attention_bf16(
        mask.row_offsets, mask.column_indices, mask.values, q, kt, v, alpha)
    _, wmx, wrs, wp, wout, bound = _dense_attention_bf16_staged(
        mask, q, kt, v, alpha)
    # every stored value is a bf16 value
    for a in (sc, mx, rs, out):
        np.testing.assert_array_equal(orc.as_bf16(a), a)
    # results agree up to one bf16 step where fp32 summation order or exp
    # differ by an ulp across a rounding boundary
    ulp = lambda a: np.abs(np.asarray(a, np.float64)) * 2.0**-7 + 1e-30
    assert np.all(np.abs(mx - wmx) <= ulp(wmx))
    assert np.all(np.abs(rs - wrs) <= ulp(wrs))
    assert np.all(np.abs(sc - wp) <= 2 * ulp(wp) + 1e-7)
    assert np.all(np.abs(out - wout) <= 2 * ulp(wout) + 1e-3 * bound)
    assert np.mean(sc == wp) > 0.95 and np.mean(out == wout) > 0.95
    # and within the bf16 tolerance of the fp32 chain
    _, _, _, out32 = orc.sparse_attention(
        mask.row_offsets, mask.column_indices, mask.values, q, kt, v, alpha)
    assert rel_l2(out, out32) <= 1e-2
    # mutation: the same chain with the row sums left unrounded agrees with
    # the staged dense computation far less often
    ro, col = mask.row_offsets, mask.column_indices
    s1 = orc.as_bf16(orc.sddmm(ro, col, mask.values, orc.as_bf16(q),
                               orc.as_bf16(kt), orc.SDDMM_AFFINE, alpha, 0.0))
    m1 = orc.row_reduce(ro, s1, orc.REDUCE_MAX)
    e1 = orc.as_bf16(orc.rowwise_map(ro, s1, m1, orc.MAP_EXP_SUB))
    r1 = orc.row_reduce(ro, e1, orc.REDUCE_SUM)
    p1 = orc.as_bf16(orc.rowwise_map(ro, e1, r1, orc.MAP_DIV))
    assert np.mean(p1 == wp) < 0.9


def test_golden_attention_bf16(orc, golden):
    """The reference's attention golden vector, within bf16 accuracy."""
    g = golden["attention"]
    _, _, _, out = orc.sparse_attention_bf16(
        np.array(g["row_offsets"], np.int32),
        np.array(g["column_indices"], np.int32),
        np.array(g["mask_values"], np.float32),
        np.array(g["query"], np.float32),
        np.array(g["transposed_key"], np.float32),
        np.array(g["value"], np.float32), g["alpha"], g["beta"])
    want = np.array(g["expected"], np.float64)
    assert np.all(np.abs(out - want) <= 2.0**-7 * np.abs(want) + 1e-4)
