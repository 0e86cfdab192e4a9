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


def test_attention_bundle_matches_oracle(dev, orc, tmp_path):
    mask, q, kt, v, alpha = W.config5(seed=0, seq=512, d=64)
    v = v[:, :32].copy()
    B.build_attention_bundle(tmp_path / "b", rows=512, key_rows=512,
                             head_dim=64, value_cols=32, alpha=alpha)
    B.verify_bundle(tmp_path / "b")
    bun = Bundle(tmp_path / "b")
    bufs = {"rowOffsets": G.t(mask.row_offsets),
            "columnIndices": G.t(mask.column_indices),
            "maskValues": G.t(mask.values), "query": G.t(q),
            "transposedKey": G.t(kt), "value": G.t(v),
            "scores": torch.empty(mask.nnz, device=G.DEV),
            "rowMaximum": torch.empty(512, device=G.DEV),
            "rowSum": torch.empty(512, device=G.DEV),
            "output": torch.full((512, 32), float("nan"), device=G.DEV)}
    ptrs = {k: t.data_ptr() for k, t in bufs.items()}
    # the runtime executor's order (the manifest deliberately has none)
    order = ["sparse_attention_scores", "sparse_attention_row_max",
             "sparse_attention_exp", "sparse_attention_row_sum",
             "sparse_attention_normalize", "sparse_attention_output"]
    G.say("bundle attention")
    for name in order:
        n = 512 * 32 if name == "sparse_attention_output" else 512
        bun.launch(name, n, ptrs)
    torch.cuda.synchronize()
    bun.close()
    # the chain's bounds derived from the per-op bars
    check_attention_f32(orc, mask, mask.values, q, kt, v, alpha, 0.0,
                        *(bufs[k].cpu().numpy() for k in (
                            "scores", "rowMaximum", "rowSum", "output")))
    assert math.isfinite(float(bufs["rowSum"].sum()))


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

