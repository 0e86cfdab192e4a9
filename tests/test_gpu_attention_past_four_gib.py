"""SDDMM and the attention chain with K^T and V past 4 GiB (fp32 and bf16).

The matrix-core SDDMM tiles and the fused attention kernels address K^T and
V with 32-bit byte offsets, and the launchers take them only when every
offset fits (4 * cols * d and 4 * cols * dv below 2^32).  Here cols is
2^24 + 32, so d = dv = 64 puts K^T and V past 4 GiB (fp32; 2 GiB+ in bf16,
the same bound): each op must take the kernels that address them with 64-bit
offsets and still match the oracle.  Only 64 columns are used (16 low, 48 at
the far end), so the oracle runs on the problem with those columns compacted,
which holds the same values in the same order.
"""
import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._check import assert_within_bound
from tests.test_gpu_bf16 import (_check_attention_bf16, _sddmm_check, host,
                                 nan_b16)
from tests.test_gpu_bsr_attention import _check_attention

pytestmark = pytest.mark.gpu

COLS = (1 << 24) + 32
D = DV = 64
FUSED = ("sddmm-mapping=row-tile-mfma sddmm-lanes-per-row=64 "
         "spmm-mapping=row-tile-mfma")


def _wide_case():
    """53 rows over a pool of 64 columns: two 16-row tiles whose rows are
    prefixes of their last row (the matrix-core paths), one tile of unrelated
    rows (the row paths), and a partial tile of 5 prefix rows."""
    rng = np.random.default_rng(77)
    pool = np.sort(np.concatenate([rng.choice(1 << 16, 16, replace=False),
                                   COLS - 48 + np.arange(48)]))
    rows_cols = []
    for tile, nt in enumerate((16, 16, 16, 5)):
        if tile == 2:
            for _ in range(nt):
                n = int(rng.integers(0, 41))
                rows_cols.append(np.sort(rng.choice(pool, n, replace=False)))
            continue
        base = np.sort(rng.choice(pool, 40, replace=False))
        lens = np.sort(rng.integers(1, 41, nt))
        lens[-1] = 40
        rows_cols += [base[:n].copy() for n in lens]
    lengths = np.array([len(c) for c in rows_cols])
    ro = np.zeros(len(rows_cols) + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(rows_cols).astype(np.int32)
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    wide = W.CSR(len(rows_cols), COLS, ro, col, vals)
    compact = W.CSR(len(rows_cols), pool.size, ro,
                    np.searchsorted(pool, col).astype(np.int32), vals)
    q = rng.standard_normal((wide.rows, D)).astype(np.float32)
    kp = rng.standard_normal((D, pool.size)).astype(np.float32)
    vp = rng.standard_normal((pool.size, DV)).astype(np.float32)
    return wide, compact, pool, q, kp, vp


@pytest.fixture(scope="module")
def wide():
    return _wide_case()


def _device_operands(pool, kp, vp, dtype):
    """K^T [D, COLS] and V [COLS, DV] on the device, zero but for the pool's
    columns / rows."""
    idx = torch.from_numpy(pool.astype(np.int64)).to(G.DEV)
    kt = torch.zeros((D, COLS), dtype=dtype, device=G.DEV)
    kt[:, idx] = torch.from_numpy(kp).to(G.DEV).to(dtype)
    v = torch.zeros((COLS, DV), dtype=dtype, device=G.DEV)
    v[idx] = torch.from_numpy(vp).to(G.DEV).to(dtype)
    return kt, v


@pytest.mark.parametrize("opts", ["", "sddmm-mapping=row-tile-mfma",
                                  "sddmm-lanes-per-row=64"])
def test_sddmm_kt_past_four_gib(dev, orc, wide, opts):
    csr, compact, pool, q, kp, vp = wide
    kt, v = _device_operands(pool, kp, vp, torch.float32)
    del v
    for kind in (sw.SDDMM_AFFINE, sw.SDDMM_MUL, sw.SDDMM_DOT):
        G.say(f"fp32 sddmm K^T of {D} x {COLS} kind={kind} opts='{opts}'")
        out = torch.full((csr.nnz,), float("nan"), device=G.DEV)
        sw.sddmm(G.t(csr.row_offsets), G.t(csr.column_indices),
                 G.t(csr.values), G.t(q), kt, out, kind, 0.125, 0.5,
                 options=opts)
        torch.cuda.synchronize()
        ref = orc.sddmm(compact.row_offsets, compact.column_indices,
                        compact.values, q, kp, kind, 0.125, 0.5)
        rows = np.repeat(np.arange(csr.rows), np.diff(csr.row_offsets))
        absd = (np.abs(q.astype(np.float64)) @ np.abs(kp.astype(np.float64)))[
            rows, compact.column_indices]
        vv = np.abs(csr.values.astype(np.float64))
        bound = {sw.SDDMM_AFFINE: 0.5 * vv + 0.125 * absd,
                 sw.SDDMM_MUL: vv * absd, sw.SDDMM_DOT: absd}[kind]
        assert_within_bound(out.cpu().numpy(), ref, bound + 1e-30)
    del kt
    torch.cuda.empty_cache()


@pytest.mark.parametrize("opts", ["", FUSED])
def test_attention_kt_v_past_four_gib(dev, orc, wide, opts):
    csr, compact, pool, q, kp, vp = wide
    kt, v = _device_operands(pool, kp, vp, torch.float32)
    G.say(f"fp32 attention K^T and V past 4 GiB opts='{opts}'")
    nan = float("nan")
    scores = torch.full((csr.nnz,), nan, device=G.DEV)
    rmax = torch.full((csr.rows,), nan, device=G.DEV)
    rsum = torch.full((csr.rows,), nan, device=G.DEV)
    out = torch.full((csr.rows, DV), nan, device=G.DEV)
    sw.sparse_attention(G.t(csr.row_offsets), G.t(csr.column_indices),
                        G.t(csr.values), G.t(q), kt, v, scores, rmax, rsum,
                        out, 0.125, 0.5, options=opts)
    torch.cuda.synchronize()
    refs = orc.sparse_attention(compact.row_offsets, compact.column_indices,
                                compact.values, q, kp, vp, 0.125, 0.5)
    _check_attention(orc, compact, scores, rmax, rsum, out, refs, vp,
                     (compact.values, q, kp, 0.125, 0.5))
    del kt, v
    torch.cuda.empty_cache()


def test_bf16_sddmm_and_attention_past_four_gib(dev, orc, wide):
    """bf16: K^T and V of 2 GiB+, past the same 32-bit offset bound."""
    csr, compact, pool, q, kp, vp = wide
    kt, v = _device_operands(pool, kp, vp, torch.bfloat16)
    ro, col = G.t(csr.row_offsets), G.t(csr.column_indices)
    vals = torch.from_numpy(csr.values).to(G.DEV).to(torch.bfloat16)
    qb = torch.from_numpy(q).to(G.DEV).to(torch.bfloat16)
    for opts in ("", "sddmm-mapping=row-tile-mfma"):
        G.say(f"bf16 sddmm K^T past the offset bound opts='{opts}'")
        out = nan_b16(csr.nnz)
        sw.sddmm(ro, col, vals, qb, kt, out, sw.SDDMM_AFFINE, 0.125, 0.5,
                 options=opts)
        torch.cuda.synchronize()
        _sddmm_check(orc, compact, compact.values, q, kp, sw.SDDMM_AFFINE,
                     0.125, 0.5, host(out))
    for opts in ("", FUSED):
        G.say(f"bf16 attention K^T and V past the offset bound opts='{opts}'")
        scores, rmax, rsum = nan_b16(csr.nnz), nan_b16(csr.rows), nan_b16(
            csr.rows)
        out = nan_b16(csr.rows, DV)
        sw.sparse_attention(ro, col, vals, qb, kt, v, scores, rmax, rsum, out,
                            0.125, 0.5, options=opts)
        torch.cuda.synchronize()
        _check_attention_bf16(orc, compact, compact.values, q, kp, vp, 0.125,
                              0.5, (host(scores), host(rmax), host(rsum),
                                    host(out)))
    del kt, v
    torch.cuda.empty_cache()
