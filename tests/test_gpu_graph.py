"""The hot entry points captured into a HIP graph (torch.cuda.CUDAGraph,
which records hipStreamBeginCapture on ROCm) and replayed.

Every launch path of the library enqueues kernels only -- the position
mappings zero their output with a fill kernel, not hipMemsetAsync, and no
path allocates, copies or synchronizes -- so a caller can capture a call
once and replay it.  Each test captures one call, then replays the graph
several times with eager launches and synchronizations between the replays,
and checks every replay: bit-equal to the eager call for the kernels whose
sums have a fixed order, within the fp32 bar of the oracle for the atomic
position mappings.  The input is rewritten in place between replays, as a
serving loop would, and the replay must follow it."""
import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G
from tests._attention_check import check_attention_f32
from tests._check import assert_within_bound
from tests.test_gpu_bf16 import assert_bf16_within_bound

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _capture(fn):
    """Warm fn up on a side stream, then capture one call into a graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _replays(g, outs, inputs, expect, eager_between):
    """Replay g REPLAYS times.  Before replay j, inputs(j) rewrites the
    captured input buffers in place and every tensor of outs is filled with
    NaN; expect(j) checks the replay's outputs; eager_between() runs
    uncaptured work and synchronizes."""
    for j in range(REPLAYS):
        inputs(j)
        for t in outs:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        expect(j)
        eager_between()


def _eager_equal(call, tensors):
    """The replay's outputs (host copies) equal an eager call's."""
    got = [t.float().cpu().numpy() for t in tensors]
    call()
    torch.cuda.synchronize()
    for a, t in zip(got, tensors):
        np.testing.assert_array_equal(a, t.float().cpu().numpy())
    return got


SPMV_CASES = [
    # the headline mapping (fill kernel + atomic segment emissions)
    ("spmv-mapping=wave-per-position spmv-positions-per-lane=4 "
     "spmv-block-size=64", False),
    # fixed-order mappings: every replay bit-equal to the eager call
    ("spmv-mapping=wave-per-row-balanced spmv-positions-per-lane=4 "
     "spmv-block-size=64", True),
    ("spmv-mapping=wave-per-row spmv-lanes-per-row=16", True),
    ("", True),  # the reference's default, thread-per-row
]


@pytest.mark.parametrize("opts,exact", SPMV_CASES)
def test_graph_spmv(dev, orc, opts, exact):
    csr = W.random_csr(30000, 20000, 24.0, 11, empty_fraction=0.1,
                       lognormal=True, max_len=3000)
    rng = np.random.default_rng(5)
    xs = [rng.uniform(-1, 1, csr.cols).astype(np.float32)
          for _ in range(REPLAYS)]
    ro, col, val = (G.t(a) for a in (csr.row_offsets, csr.column_indices,
                                     csr.values))
    x = G.t(xs[0])
    y = torch.empty(csr.rows, device=G.DEV)
    G.say(f"graph spmv rows={csr.rows} nnz={csr.nnz} opts='{opts}'")
    call = lambda: sw.spmv(ro, col, val, x, y, options=opts or None)
    g = _capture(call)
    other = torch.empty_like(y)
    refs = [orc.spmv(csr.row_offsets, csr.column_indices, csr.values, xi)
            for xi in xs]
    bounds = [orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                                 csr.values, xi) for xi in xs]

    def expect(j):
        got = y.cpu().numpy()
        assert_within_bound(got, refs[j], bounds[j], what=f"replay {j}")
        if exact:  # the same call eagerly on the same input
            _eager_equal(call, [y])

    def eager_between():
        sw.spmv(ro, col, val, x, other,
                options="spmv-mapping=wave-per-position")
        torch.cuda.synchronize()

    _replays(g, [y], lambda j: x.copy_(G.t(xs[j])), expect, eager_between)


@pytest.mark.parametrize("k,opts", [
    (4, "spmm-mapping=wave-per-row-tile spmm-tile-size=4 "
        "spmm-block-size=64"),
    (64, "spmm-mapping=wave-per-row-tile spmm-tile-size=32 "
         "spmm-lanes-per-row=64 spmm-block-size=64"),
    (4, "spmm-mapping=wave-per-position spmm-positions-per-lane=4 "
        "spmm-block-size=64"),
])
def test_graph_spmm(dev, orc, k, opts):
    csr = W.random_csr(8000, 6000, 20.0, 12, empty_fraction=0.1,
                       lognormal=True, max_len=1000)
    rng = np.random.default_rng(k)
    bs = [rng.uniform(-1, 1, (csr.cols, k)).astype(np.float32)
          for _ in range(REPLAYS)]
    ro, col, val = (G.t(a) for a in (csr.row_offsets, csr.column_indices,
                                     csr.values))
    b = G.t(bs[0])
    out = torch.empty((csr.rows, k), device=G.DEV)
    G.say(f"graph spmm rows={csr.rows} k={k} opts='{opts}'")
    call = lambda: sw.spmm(ro, col, val, b, out, options=opts)
    g = _capture(call)
    exact = "position" not in opts

    def expect(j):
        ref = orc.spmm(csr.row_offsets, csr.column_indices, csr.values, bs[j])
        bound = orc.spmm_abs_bound(csr.row_offsets, csr.column_indices,
                                   csr.values, bs[j])
        assert_within_bound(out.cpu().numpy(), ref, bound,
                            what=f"replay {j}")
        if exact:
            _eager_equal(call, [out])

    def eager_between():
        sw.spmv(ro, col, val, b[:, 0].contiguous(),
                torch.empty(csr.rows, device=G.DEV))
        torch.cuda.synchronize()

    _replays(g, [out], lambda j: b.copy_(G.t(bs[j])), expect, eager_between)


@pytest.mark.parametrize("bf16", [False, True])
def test_graph_bsr(dev, orc, bf16):
    bsr = W.bsr_banded(seed=3, rows=16 * 300, block_size=16,
                       blocks_per_row=6, band=3, band_blocks=3,
                       value_std=0.5)
    k = 128
    rng = np.random.default_rng(9)
    rs = [rng.standard_normal((bsr.cols, k)).astype(np.float32)
          for _ in range(REPLAYS)]
    dt = torch.bfloat16 if bf16 else torch.float32
    bro, bcol = G.t(bsr.block_row_offsets), G.t(bsr.block_column_indices)
    vals = G.t(bsr.block_values, dt)
    rhs = G.t(rs[0], dt)
    out = torch.empty((bsr.rows, k), dtype=dt, device=G.DEV)
    G.say(f"graph bsr rows={bsr.rows} k={k} bf16={bf16}")
    call = lambda: sw.bsr_spmm(bro, bcol, vals, rhs, out, 16,
                               options="bsr-use-mfma=1")
    g = _capture(call)
    vref = orc.as_bf16(bsr.block_values) if bf16 else bsr.block_values

    def expect(j):
        # the MFMA tiles' sums have a fixed order: bit-equal to eager
        (got,) = _eager_equal(call, [out])
        rref = orc.as_bf16(rs[j]) if bf16 else rs[j]
        ref = orc.bsr_spmm(bsr.block_row_offsets, bsr.block_column_indices,
                           vref, rref, 16)
        bound = orc.bsr_abs_bound(bsr.block_row_offsets,
                                  bsr.block_column_indices, vref, rref, 16)
        if bf16:
            assert_bf16_within_bound(got, ref, bound, what=f"replay {j}")
        else:
            assert_within_bound(got, ref, bound, what=f"replay {j}")

    def eager_between():
        torch.cuda.synchronize()

    _replays(g, [out], lambda j: rhs.copy_(G.t(rs[j], dt)), expect,
             eager_between)


@pytest.mark.parametrize("opts", [
    "sddmm-mapping=row-tile-mfma sddmm-lanes-per-row=64 "
    "spmm-mapping=row-tile-mfma",   # the fused one-kernel chain
    "",                             # the reference's six-kernel schedule
])
def test_graph_attention(dev, orc, opts):
    mask, q, kt, v, alpha = W.config5(seed=0, seq=1024)
    rng = np.random.default_rng(4)
    qs = [q] + [rng.standard_normal(q.shape).astype(np.float32)
                for _ in range(REPLAYS - 1)]
    ro, col, mv = (G.t(a) for a in (mask.row_offsets, mask.column_indices,
                                    mask.values))
    qd, ktd, vd = G.t(qs[0]), G.t(kt), G.t(v)
    scores = torch.empty(mask.nnz, device=G.DEV)
    rmax = torch.empty(mask.rows, device=G.DEV)
    rsum = torch.empty(mask.rows, device=G.DEV)
    out = torch.empty((mask.rows, v.shape[1]), device=G.DEV)
    G.say(f"graph attention seq={mask.rows} opts='{opts}'")
    call = lambda: sw.sparse_attention(ro, col, mv, qd, ktd, vd, scores,
                                       rmax, rsum, out, alpha, 0.0,
                                       options=opts or None)
    g = _capture(call)

    def expect(j):
        # every output of the chain bit-equal to an eager call on the same
        # input (the chain's sums have a fixed order), and within the
        # attention bounds of the oracle
        s_, m_, r_, o_ = _eager_equal(call, [scores, rmax, rsum, out])
        check_attention_f32(orc, mask, mask.values, qs[j], kt, v, alpha, 0.0,
                            s_, m_, r_, o_)

    def eager_between():
        torch.cuda.synchronize()

    _replays(g, [scores, rmax, rsum, out], lambda j: qd.copy_(G.t(qs[j])),
             expect, eager_between)
