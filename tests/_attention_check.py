"""Parity bounds for the fp32 sparse-attention chain, derived from the
per-op bars (examples/pytorch/integration/SparseAttentionToSparseWave.cpp:
230-315 is the chain: scores = sddmm, row max, exp(s - max), row sum,
s / sum, output = P V).

Inputs to the derivation, with u = 2^-24 (fp32 unit roundoff):

* SDDMM (the op's stated bar): |s_p - s_ref_p| <= 1e-5 * B_p with
  B_p = |beta * mask_p| + |alpha| * sum_k |q_rk kt_kc|.  Per row r let
  E_r = max over the row's finite scores of 1e-5 * B_p.
* Row max is 1-Lipschitz in the max-norm: |m_r - m_ref_r| <= E_r.
* Softmax: with P = softmax(s) over the row, P(s) / P(s_ref) lies in
  [e^{-2 E_r}, e^{2 E_r}] (numerator and denominator each move by at most
  e^{E_r}), so the exact-arithmetic difference is at most
  P_ref * (e^{2 E_r} - 1).  Rounding, on each side (GPU and oracle):
  exp(x) with x = s - m rounded and, in the fused kernels, scaled by
  log2(e) before v_exp_f32: relative (|x| + 4) u; the row sum of n_r
  positive terms: relative n_r u (sequential; the GPU's tree sum is
  smaller); the division: u.  Both sides together:
      |P_p - P_ref_p| <= P_ref_p * ((e^{2 E_r} - 1)(1 + 1e-3)
                                    + (2 |x_p| + 2 n_r + 16) u) + 2^-126
  where x_p = s_ref_p - m_ref_r.  The absolute 2^-126 covers
  probabilities below the smallest normal, which v_exp_f32 flushes to
  zero (exp of x < -87.3 is subnormal or zero; P_ref <= e^x since the row
  sum is >= 1).
* Row sum: the same argument with the largest |x| of the row.
* Output: two checks.  (1) The SpMM op's own bar on the GPU's
  probabilities: |out - spmm(P, V)| <= 1e-5 * sum_p |P_p V_pc|.
  (2) End to end against the oracle chain:
      |out - out_ref| <= 1e-5 * (sum_p |P_p V_pc| + sum_p |P_ref_p V_pc|)
                         + sum_p tolP_p |V_pc|
  i.e. each side's SpMM within its bar plus the probabilities' bound
  carried through the product.
"""
import numpy as np

from tests._check import FP32_REL, assert_within_bound

U = 2.0 ** -24
TINY = 2.0 ** -126


def score_bounds(orc, csr, mask_vals, q, kt, alpha, beta):
    """B_p = |beta mask_p| + |alpha| sum_k |q_rk kt_kc| per stored entry
    (non-finite mask values contribute 0: their scores are exact).  The
    sum of non-negative products comes from the oracle's SDDMM (dot form)
    on |q| and |kt|; its fp32 rounding is at most d u relative, which the
    factor (1 + 2 d u) covers."""
    d = np.asarray(q).shape[1]
    aq = np.abs(np.asarray(q, np.float32))
    ak = np.abs(np.asarray(kt, np.float32))
    b = orc.sddmm(csr.row_offsets, csr.column_indices,
                  np.zeros(len(csr.column_indices), np.float32), aq, ak,
                  orc.SDDMM_DOT).astype(np.float64) * (1 + 2 * d * U)
    mv = np.asarray(mask_vals, np.float64)
    mb = np.where(np.isfinite(mv), np.abs(beta * mv), 0.0)
    return abs(alpha) * b + mb


def row_error(csr, per_entry, s_ref):
    """E_r = max over row r's finite reference scores of per_entry."""
    ro = np.asarray(csr.row_offsets, np.int64)
    vals = np.where(np.isfinite(s_ref), per_entry, 0.0)
    e = np.zeros(csr.rows)
    nz = np.flatnonzero(np.diff(ro) > 0)
    if nz.size:
        e[nz] = np.maximum.reduceat(vals, ro[nz])
    return e


def tolerances(csr, p_ref, x_ref, e_row):
    """(tolP per entry, tol_sum_rel per row) for P_ref = p_ref and
    x_ref = s_ref - m_ref (the oracle's exponent arguments, -inf where the
    score is masked)."""
    ro = np.asarray(csr.row_offsets, np.int64)
    n = np.diff(ro).astype(np.float64)
    rows = np.repeat(np.arange(csr.rows), np.diff(ro))
    p = np.asarray(p_ref, np.float64)
    x = np.asarray(x_ref, np.float64)
    fin = np.isfinite(x)
    ax = np.where(fin, np.abs(x), 0.0)
    shift = np.expm1(2.0 * e_row) * (1 + 1e-3)
    rel = shift[rows] + (2.0 * ax + 2.0 * n[rows] + 16.0) * U
    tol_p = np.where(fin & np.isfinite(p), np.abs(p) * rel, 0.0) + TINY
    axmax = np.zeros(csr.rows)
    nz = np.flatnonzero(n > 0)
    if nz.size:
        axmax[nz] = np.maximum.reduceat(ax, ro[nz])
    tol_sum = shift + (2.0 * axmax + 2.0 * n + 16.0) * U
    return tol_p, tol_sum


def check_attention_f32(orc, csr, mask_vals, q, kt, v, alpha, beta, scores,
                        rmax, rsum, out, refs=None):
    """Checks the four outputs of the fp32 chain against the oracle with
    the bounds derived above.  Rows whose reference maximum is -inf (every
    entry masked) must match the reference's non-finite pattern; outputs
    where the reference is non-finite (inf / NaN in V) must match its
    class."""
    if refs is None:
        refs = orc.sparse_attention(csr.row_offsets, csr.column_indices,
                                    mask_vals, q, kt, v, alpha, beta)
    s_ref, m_ref, sum_ref, ref = refs
    scores, rmax, rsum, out = (np.asarray(a, np.float64)
                               for a in (scores, rmax, rsum, out))
    ro = np.asarray(csr.row_offsets, np.int64)
    rows = np.repeat(np.arange(csr.rows), np.diff(ro))
    # the oracle's raw scores (before exp / division) give x = s - m
    raw = orc.sddmm(csr.row_offsets, csr.column_indices, mask_vals, q, kt,
                    orc.SDDMM_AFFINE, alpha, beta).astype(np.float64)
    live_row = np.isfinite(m_ref)
    live = live_row[rows]
    e_row = row_error(csr, FP32_REL * score_bounds(orc, csr, mask_vals, q, kt,
                                                   alpha, beta), raw)
    with np.errstate(invalid="ignore"):
        x = np.where(live, raw - m_ref[rows], -np.inf)
    tol_p, tol_sum = tolerances(csr, s_ref, x, e_row)

    # rows with no entries hold the identities: -inf, 0, and a zero output
    empty = np.diff(ro) == 0
    assert np.all(np.isneginf(rmax[empty])) and np.all(rsum[empty] == 0)
    assert np.all(out[empty] == 0)
    # row maxima
    mr = np.asarray(m_ref, np.float64)
    assert np.array_equal(np.isfinite(rmax), np.isfinite(mr)), "row max class"
    d = np.abs(rmax[live_row] - mr[live_row])
    assert np.all(d <= e_row[live_row] + TINY), ("row max", d.max())
    # probabilities
    sp = np.asarray(s_ref, np.float64)
    assert np.array_equal(np.isnan(scores[~live]), np.isnan(sp[~live]))
    dp = np.abs(scores[live] - sp[live])
    bad = dp > tol_p[live]
    assert not bad.any(), ("probabilities", int(bad.sum()),
                           float((dp / tol_p[live]).max()))
    # row sums
    sr = np.asarray(sum_ref, np.float64)
    ds = np.abs(rsum[live_row] - sr[live_row])
    assert np.all(ds <= sr[live_row] * tol_sum[live_row]), (
        "row sum", float((ds / (sr[live_row] * tol_sum[live_row])).max()))
    # output: (1) the SpMM bar on the GPU's own probabilities
    pg = np.where(np.isfinite(scores), scores, 0.0).astype(np.float32)
    vf = np.nan_to_num(np.asarray(v, np.float32), posinf=0, neginf=0)
    fin = np.isfinite(ref) & live_row[:, None]
    own = orc.spmm(csr.row_offsets, csr.column_indices, pg, v)
    own_b = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices, pg, vf)
    assert_within_bound(out[fin], own[fin], own_b[fin], what="output SpMM")
    # (2) end to end against the oracle chain
    pr = np.where(np.isfinite(sp), sp, 0.0).astype(np.float32)
    ref_b = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices, pr, vf)
    carried = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                                 tol_p.astype(np.float32), vf)
    tol = FP32_REL * (own_b + ref_b) + carried
    err = np.abs(out[fin] - np.asarray(ref, np.float64)[fin])
    bad = err > tol[fin]
    assert not bad.any(), ("output vs oracle chain", int(bad.sum()),
                           float((err / tol[fin]).max()))
