"""The BSR slab-floor diagnostic (sw_bsr_slab_floor): the matrix-core BSR
SpMM launch with its block products replaced by an XOR of the 32-bit words
each lane loads.  The XOR is order-free, so a numpy reference that follows
the kernels' lane layout gives every output bit exactly; a kernel that
skipped a load or read a wrong slab would differ.

Lane layout (sparsewavecomp_amd/csrc/sw_bsr.hip):
* fp32 (bsr16_mfma_f32_x4): the lane computing output columns c .. c + 3
  (c % 4 == 0) of rows 16 br + 4 g .. + 3 loads, per block b of block row
  br, A row (c % 64) / 4, elements 4 g .. 4 g + 3, and RHS rows
  16 bcol[b] + 4 g + st (st < 4), columns c .. c + 3;
* bf16 (bsr16_mfma_bf16_x8): columns c .. c + 7 (c % 8 == 0), A row
  (c % 128) / 8, elements 4 g .. 4 g + 3 (two words), RHS rows as above,
  columns c .. c + 7 (four words).
Every element of the lane's 4 x 4 (fp32) or 4 x 8 (bf16) output region
holds the XOR over the block row's blocks (its low 16 bits for a bf16
output).

It is not a reference op: bench.py times it beside the BSR SpMM as the
floor of the kernels' memory trips."""
import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G

pytestmark = pytest.mark.gpu


def _expected(bro, bcol, bval_words, rhs_words, k, bf16, block_rows=None):
    """uint32 [len(block_rows) * 16, k] of the floor's output bits."""
    nbr = len(bro) - 1
    if block_rows is None:
        block_rows = np.arange(nbr)
    lane_cols = 8 if bf16 else 4
    wpc = 2 if bf16 else 1           # elements per 32-bit word
    out = np.zeros((len(block_rows) * 16, k), np.uint32)
    idx = np.concatenate([np.arange(bro[b], bro[b + 1]) for b in block_rows]
                         ).astype(np.int64)
    counts = (bro[block_rows + 1] - bro[block_rows]).astype(np.int64)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    bc = bcol[idx].astype(np.int64)
    for c0 in range(0, k, lane_cols):
        a_row = (c0 % 128) // 8 if bf16 else (c0 % 64) // 4
        w0, nw = c0 // wpc, lane_cols // wpc
        for g in range(4):
            if bf16:
                aw = (bval_words[idx, a_row, 2 * g] ^
                      bval_words[idx, a_row, 2 * g + 1])
            else:
                aw = np.bitwise_xor.reduce(
                    bval_words[idx, a_row, 4 * g:4 * g + 4], axis=1)
            rr = 16 * bc[:, None] + 4 * g + np.arange(4)[None, :]
            rw = np.bitwise_xor.reduce(
                rhs_words[rr][:, :, w0:w0 + nw].reshape(len(idx), -1), axis=1)
            per_block = aw ^ rw
            x = np.zeros(len(block_rows), np.uint32)
            ne = counts > 0
            if per_block.size:
                red = np.bitwise_xor.reduceat(per_block, starts[ne])
                x[ne] = red
            for v in range(4):
                out[16 * np.arange(len(block_rows)) + 4 * g + v,
                    c0:c0 + lane_cols] = x[:, None]
    return out


def _run(bsr, rhs, bf16, out_dtype):
    dt = torch.bfloat16 if bf16 else torch.float32
    vals = G.t(bsr.block_values, dt)
    b = G.t(rhs, dt)
    out = torch.full((bsr.rows, rhs.shape[1]), float("nan"), dtype=out_dtype,
                     device=G.DEV)
    G.say(f"bsr slab floor rows={bsr.rows} k={rhs.shape[1]} bf16={bf16} "
          f"out={out_dtype}")
    sw.bsr_slab_floor(G.t(bsr.block_row_offsets),
                      G.t(bsr.block_column_indices), vals, b, out)
    torch.cuda.synchronize()
    words = lambda t: t.cpu().view(torch.int32).numpy().view(np.uint32)
    bw = words(vals.reshape(-1)).reshape(bsr.nnzb, 16, 8 if bf16 else 16)
    rw = words(b.reshape(-1)).reshape(bsr.cols, -1)
    got = out.cpu()
    got = (got.view(torch.int16).numpy().view(np.uint16).astype(np.uint32)
           if out_dtype == torch.bfloat16 else
           got.view(torch.int32).numpy().view(np.uint32))
    return got, bw, rw


@pytest.mark.parametrize("bf16,out_dtype", [
    (False, torch.float32), (True, torch.bfloat16), (True, torch.float32)])
@pytest.mark.parametrize("k", [128, 64, 40, 200])
def test_slab_floor_bits(dev, bf16, out_dtype, k):
    from tests.test_gpu_bsr_attention import _ragged_bsr
    if bf16 and k % 8:
        pytest.skip("bf16 floor needs k % 8 == 0")
    bsr = _ragged_bsr(k)
    rhs = np.random.default_rng(k).standard_normal((bsr.cols, k)).astype(
        np.float32)
    got, bw, rw = _run(bsr, rhs, bf16, out_dtype)
    want = _expected(bsr.block_row_offsets, bsr.block_column_indices, bw, rw,
                     k, bf16)
    if out_dtype == torch.bfloat16:
        want = want & 0xFFFF
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("bf16,out_dtype", [
    (False, torch.float32), (True, torch.bfloat16)])
def test_slab_floor_config4_sample(dev, bf16, out_dtype):
    """Configuration 4 at full size; 300 block rows (first, last, random)
    checked bit for bit."""
    bsr, rhs = W.config4(seed=0)
    got, bw, rw = _run(bsr, rhs, bf16, out_dtype)
    nbr = bsr.rows // 16
    brs = np.unique(np.concatenate([
        [0, nbr - 1], np.random.default_rng(2).choice(nbr, 300,
                                                      replace=False)]))
    want = _expected(bsr.block_row_offsets, bsr.block_column_indices, bw, rw,
                     128, bf16, brs)
    if out_dtype == torch.bfloat16:
        want = want & 0xFFFF
    rows = (brs[:, None] * 16 + np.arange(16)[None, :]).ravel()
    np.testing.assert_array_equal(got[rows], want)
