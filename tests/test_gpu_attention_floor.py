"""The attention tile-floor diagnostic (sw_attention_tile_floor): the fused
attention tile kernel with every product, exponential and division replaced
by an XOR of the words each lane loads.  Its outputs are bit patterns with
no reference value; the test checks that the launch covers every score, row
and output element (two runs over buffers pre-filled with different bit
patterns must agree bit for bit: an element the kernel did not write would
keep its fill) and that it is deterministic.

It is not a reference op: bench.py times it beside the fused attention as
the floor of the tile's chain of memory trips."""
import numpy as np
import pytest
import torch

import sparsewavecomp_amd as sw
from sparsewavecomp_amd import workloads as W
from tests import gpu_util as G

pytestmark = pytest.mark.gpu


def _run(mask, q, kt, v, dt, fill):
    bufs = [torch.empty(n, dtype=dt, device=G.DEV)
            for n in (mask.nnz, mask.rows, mask.rows)]
    out = torch.empty((mask.rows, v.shape[1]), dtype=dt, device=G.DEV)
    for b in bufs + [out]:
        (b.view(torch.int16) if dt == torch.bfloat16 else
         b.view(torch.int32)).fill_(fill)
    sw.attention_tile_floor(G.t(mask.row_offsets), G.t(mask.column_indices),
                            G.t(mask.values, dt), G.t(q, dt), G.t(kt, dt),
                            G.t(v, dt), *bufs, out)
    torch.cuda.synchronize()
    iv = torch.int16 if dt == torch.bfloat16 else torch.int32
    return [b.view(iv).cpu().numpy() for b in bufs + [out]]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seq,d", [(8192, 64), (1024, 128)])
def test_tile_floor_covers_every_output(dev, dt, seq, d):
    mask, q, kt, v, _ = W.config5(seed=0, seq=seq, d=d)
    G.say(f"attention tile floor seq={seq} d={d} dtype={dt}")
    a = _run(mask, q, kt, v, dt, 0x1357)
    b = _run(mask, q, kt, v, dt, 0x2468)
    for name, x, y in zip(("scores", "row max", "row sum", "output"), a, b):
        assert np.array_equal(x, y), name


def test_tile_floor_rejects_other_shapes(dev):
    mask, q, kt, v, _ = W.config5(seed=0, seq=256, d=64)
    dt = torch.float32
    args = [G.t(mask.row_offsets), G.t(mask.column_indices),
            G.t(mask.values), G.t(q[:, :32].copy()), G.t(kt[:32].copy()),
            G.t(v)]
    outs = [torch.empty(mask.nnz, device=G.DEV),
            torch.empty(mask.rows, device=G.DEV),
            torch.empty(mask.rows, device=G.DEV),
            torch.empty((mask.rows, v.shape[1]), dtype=dt, device=G.DEV)]
    with pytest.raises(sw.SparseWaveError, match="fused kernel's shapes"):
        sw.attention_tile_floor(*args, *outs)  # d = 32
