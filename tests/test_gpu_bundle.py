"""Bundles run on the GPU through a stand-in of lrrt's launch(n, args) and
match the CPU oracle (fp32 bound |y - y_ref| <= 1e-5 sum|a*b|)."""
import math

import numpy as np
import pytest
import torch

from sparsewavecomp_amd import bundle as B
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._attention_check import check_attention_f32
from tests._check import assert_within_bound
from sparsewavecomp_amd.bundle.runtime import Bundle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tile", [4, 1, 8])
def test_spmm_bundle_matches_oracle(dev, orc, tmp_path, tile):
    csr = W.random_csr(3000, 2000, 20.0, tile, empty_fraction=0.2,
                       lognormal=True, max_len=2000)
    rhs = np.random.default_rng(1).uniform(-1, 1, (2000, tile)).astype(
        np.float32)
    B.build_spmm_bundle(tmp_path / "b", rows=csr.rows, rhs_columns=tile,
                        tile_size=tile)
    B.verify_bundle(tmp_path / "b")
    bun = Bundle(tmp_path / "b")
    ro, col, val, b = (G.t(csr.row_offsets), G.t(csr.column_indices),
                       G.t(csr.values), G.t(rhs))
    out = torch.full((csr.rows, tile), float("nan"), device=G.DEV)
    G.say(f"bundle spmm tile={tile}")
    bun.launch("spmm", csr.rows, {"rowOffsets": ro.data_ptr(),
                                  "columnIndices": col.data_ptr(),
                                  "values": val.data_ptr(),
                                  "rhs": b.data_ptr(),
                                  "output": out.data_ptr()})
    torch.cuda.synchronize()
    bun.close()
    ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, rhs)
    bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, rhs)
    assert_within_bound(out.cpu().numpy(), ref, bound)


def _attention_case(case):
    """(mask, q, kt, v, alpha) for the attention bundle tests: block masks
    whose 64-row tiles hold the prefix column structure (the scores kernel's
    matrix-core tiles), a partial last tile, 32-row blocks that straddle
    the 64-row tiles and ragged masks (its row-by-row path), and head dims
    of 64, 128 and 32 (no tiles at 32).  The "_dv64" / "_dv128" cases give V
    64 or 128 columns, which the output kernel computes as 16-row
    matrix-core tiles (prefix tiles) or row by row (the ragged masks);
    "inf_dv64" puts an inf in a V row that only the last row of a 16-row
    tile reads, so that the tile's other rows meet 0 * inf and the tile is
    recomputed row by row.  "masked" sets a fifth of the mask values, and
    one row's whole, to -inf.  "wide" spreads the scores over 100 below their
    row maxima, so that the exponential kernel's v_exp_f32 runs over a wide
    range of arguments and flushes the results below 2^-126 that expf
    gives as subnormals (the checker's absolute 2^-126 per probability)."""
    if case.endswith("_dv64") or case.endswith("_dv128"):
        base, wide = case.rsplit("_dv", 1)
        mask, q, kt, v, alpha = _attention_case(base)
        rng = np.random.default_rng(len(case) + 100)
        v = rng.standard_normal((mask.cols, int(wide))).astype(np.float32)
        if base == "inf":
            v[31, 5] = np.inf  # column 31: row 31, the last of rows 16-31
        return mask, q, kt, v, alpha
    if case == "inf":
        mask, q, kt, v, alpha = W.config5(seed=1, seq=256, d=64)
        return mask, q, kt, v, alpha
    if case == "wide":
        # scores spread over 100 below their row maxima (alpha = 1.6)
        mask, q, kt, v, _ = W.config5(seed=0, seq=1024)
        return mask, q, kt, v, 1.6
    if case == "masked":
        # a fifth of the mask values -inf (entries masked out) and one row
        # masked whole: probability 0, and -inf maximum with NaN sum,
        # probabilities and output for the dead row
        mask, q, kt, v, _ = W.config5(seed=2, seq=512)
        rng = np.random.default_rng(78)
        vals = rng.uniform(-1, 1, mask.nnz).astype(np.float32)
        vals[rng.random(mask.nnz) < 0.2] = -np.inf
        dead = int(np.flatnonzero(np.diff(mask.row_offsets) > 20)[3])
        vals[mask.row_offsets[dead]:mask.row_offsets[dead + 1]] = -np.inf
        mask = W.CSR(mask.rows, mask.cols, mask.row_offsets,
                     mask.column_indices, vals)
        return mask, q, kt, v, 0.125
    if case in ("config5", "d128", "d32"):
        d = {"config5": 64, "d128": 128, "d32": 32}[case]
        mask, q, kt, v, alpha = W.config5(seed=0, seq=512, d=d)
        return mask, q, kt, np.ascontiguousarray(v[:, :32]), alpha
    if case == "partial":
        mask = W.attention_mask(seq=300, block=64, window=3,
                                random_blocks=1, seed=4)
    elif case == "block32":
        mask = W.attention_mask(seq=448, block=32, window=4,
                                random_blocks=2, seed=5)
    else:
        from tests.test_gpu_fuzz_attention import _mask
        mask, _ = _mask({"ragged0": 0, "ragged2": 2}[case])
    rng = np.random.default_rng(len(case))
    q = rng.standard_normal((mask.rows, 64)).astype(np.float32)
    kt = rng.standard_normal((64, mask.cols)).astype(np.float32)
    v = rng.standard_normal((mask.cols, 48)).astype(np.float32)
    mask = W.CSR(mask.rows, mask.cols, mask.row_offsets, mask.column_indices,
                 rng.uniform(-1, 1, mask.nnz).astype(np.float32))
    return mask, q, kt, v, 0.125


@pytest.mark.parametrize("case", ["config5", "partial", "block32", "ragged0",
                                  "ragged2", "d128", "d32", "config5_dv64",
                                  "partial_dv64", "block32_dv128",
                                  "ragged0_dv64", "ragged2_dv64", "d128_dv64",
                                  "inf_dv64", "wide", "masked"])
def test_attention_bundle_matches_oracle(dev, orc, tmp_path, case):
    mask, q, kt, v, alpha = _attention_case(case)
    rows, d, dv = mask.rows, q.shape[1], v.shape[1]
    beta = 0.0 if case.split("_dv")[0] in ("config5", "d128", "d32",
                                           "inf", "wide") else 0.5
    B.build_attention_bundle(tmp_path / "b", rows=rows, key_rows=mask.cols,
                             head_dim=d, value_cols=dv, alpha=alpha,
                             beta=beta)
    B.verify_bundle(tmp_path / "b")
    bun = Bundle(tmp_path / "b")
    nan = float("nan")
    bufs = {"rowOffsets": G.t(mask.row_offsets),
            "columnIndices": G.t(mask.column_indices),
            "maskValues": G.t(mask.values), "query": G.t(q),
            "transposedKey": G.t(kt), "value": G.t(v),
            "scores": torch.full((mask.nnz,), nan, device=G.DEV),
            "rowMaximum": torch.full((rows,), nan, device=G.DEV),
            "rowSum": torch.full((rows,), nan, device=G.DEV),
            "output": torch.full((rows, dv), nan, device=G.DEV)}
    ptrs = {k: t.data_ptr() for k, t in bufs.items()}
    # the runtime executor's order (the manifest deliberately has none)
    G.say(f"bundle attention {case} rows={rows} nnz={mask.nnz} d={d}")
    for name in B.ATTENTION_ORDER:
        bun.launch(name, rows * dv if name == "sparse_attention_output"
                   else rows, ptrs)
    torch.cuda.synchronize()
    bun.close()
    # the chain's bounds derived from the per-op bars
    refs = orc.sparse_attention(mask.row_offsets, mask.column_indices,
                                mask.values, q, kt, v, alpha, beta)
    out = bufs["output"].cpu().numpy()
    check_attention_f32(orc, mask, mask.values, q, kt, v, alpha, beta,
                        *(bufs[k].cpu().numpy() for k in (
                            "scores", "rowMaximum", "rowSum")), out, refs)
    # non-finite outputs in the reference's places and classes
    ref = np.asarray(refs[3])
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(out), cls(ref)), cls.__name__
    if case == "inf_dv64":
        assert np.isposinf(ref).any() and np.isfinite(ref[16:31]).all()
    if case == "masked":
        m_ref, sum_ref = np.asarray(refs[1]), np.asarray(refs[2])
        dead = np.flatnonzero(np.isneginf(m_ref))
        assert dead.size >= 1 and np.isnan(sum_ref[dead]).all()
        assert np.isnan(bufs["rowSum"].cpu().numpy()[dead]).all()
        assert np.isnan(out[dead]).all()
    if case == "wide":
        p_ref = np.asarray(refs[0])
        assert float(np.log(p_ref[p_ref > 0]).min()) < -95.0


def test_config3_bundle_at_full_size(dev, orc):
    """The in-tree bundle of configuration 3 at K = 4 (1,048,576 rows, the
    configuration-2 matrix times 4 RHS columns), launched as lrrt does with
    n = rows: 20,000 random rows and the 50 longest checked against the
    oracle within the fp32 bound, every row written."""
    from tests.test_gpu_spmm import _row_subset
    if not (B.CONFIG3_BUNDLE / "manifest.json").exists():
        pytest.fail("the configuration-3 bundle is not built "
                    "(__graft_entry__.build() writes it)")
    B.verify_bundle(B.CONFIG3_BUNDLE)
    csr, _ = W.config2(seed=0)
    assert csr.rows == B.CONFIG3_ROWS
    rhs = W.config3_rhs(csr.cols, 4, seed=0)
    bun = Bundle(B.CONFIG3_BUNDLE)
    ro, col, val, b = (G.t(csr.row_offsets), G.t(csr.column_indices),
                       G.t(csr.values), G.t(rhs))
    out = torch.full((csr.rows, 4), float("nan"), device=G.DEV)
    G.say("configuration-3 bundle, 1,048,576 rows, K = 4")
    bun.launch("spmm", csr.rows, {"rowOffsets": ro.data_ptr(),
                                  "columnIndices": col.data_ptr(),
                                  "values": val.data_ptr(),
                                  "rhs": b.data_ptr(),
                                  "output": out.data_ptr()})
    torch.cuda.synchronize()
    bun.close()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    rows = np.sort(np.random.default_rng(3).choice(csr.rows, 20000,
                                                   replace=False))
    rows = np.concatenate([rows, np.argsort(np.diff(csr.row_offsets))[-50:]])
    sub = _row_subset(csr, rows)
    ref = orc.spmm(sub.row_offsets, sub.column_indices, sub.values, rhs)
    bound = orc.spmm_abs_bound(sub.row_offsets, sub.column_indices,
                               sub.values, rhs)
    assert_within_bound(got[rows], ref, bound)



def test_config5_bundle_at_full_size(dev, orc):
    """The in-tree attention bundle of configuration 5 (seq 8192, d = dv =
    64, alpha = 1/8), its six kernels launched in order as a runtime does,
    n = rows (output elements for the output kernel): every output of the
    chain against the oracle with the bounds derived from the per-op bars."""
    if not (B.CONFIG5_BUNDLE / "manifest.json").exists():
        pytest.fail("the configuration-5 bundle is not built "
                    "(__graft_entry__.build() writes it)")
    B.verify_bundle(B.CONFIG5_BUNDLE)
    mask, q, kt, v, alpha = W.config5(seed=0)
    assert mask.rows == B.CONFIG5_SEQ and q.shape[1] == B.CONFIG5_HEAD_DIM
    assert alpha == 1.0 / math.sqrt(B.CONFIG5_HEAD_DIM)
    rows, dv = mask.rows, v.shape[1]
    nan = float("nan")
    bufs = {"rowOffsets": G.t(mask.row_offsets),
            "columnIndices": G.t(mask.column_indices),
            "maskValues": G.t(mask.values), "query": G.t(q),
            "transposedKey": G.t(kt), "value": G.t(v),
            "scores": torch.full((mask.nnz,), nan, device=G.DEV),
            "rowMaximum": torch.full((rows,), nan, device=G.DEV),
            "rowSum": torch.full((rows,), nan, device=G.DEV),
            "output": torch.full((rows, dv), nan, device=G.DEV)}
    ptrs = {k: t.data_ptr() for k, t in bufs.items()}
    bun = Bundle(B.CONFIG5_BUNDLE)
    G.say("configuration-5 attention bundle, seq 8192")
    for name in B.ATTENTION_ORDER:
        bun.launch(name, rows * dv if name == "sparse_attention_output"
                   else rows, ptrs)
    torch.cuda.synchronize()
    bun.close()
    check_attention_f32(orc, mask, mask.values, q, kt, v, alpha, 0.0,
                        *(bufs[k].cpu().numpy() for k in (
                            "scores", "rowMaximum", "rowSum", "output")))
