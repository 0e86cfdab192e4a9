"""CPU emulation of the row-owner SpMV kernel (spmv_row_owner in
sparsewavecomp_amd/csrc/sw_spmv.hip, spmv-mapping=wave-per-row-balanced),
lane by lane and step by step, on small matrices: every row offset, column,
value and output index it touches stays in range, every output row is
written by exactly one wave (rows with no entries may get a second zero
from the same wave), and the result matches the oracle's SpMV within the
fp32 bound.  It checks the kernel's ownership, window, walk, scan, carry
and emission rules before they run on a GPU; a planted mistake (a dropped
carry) must fail."""
import numpy as np
import pytest

from sparsewavecomp_amd import workloads as W
from tests._check import assert_within_bound

WAVE = 64
INT32_MAX = 2 ** 31 - 1


def _upper(ro, lo, hi, pos, touched):
    """(first j in [lo, hi) with ro[j] > pos) - 1, or hi - 1 (the kernel's
    row searches; the probes are recorded)."""
    while lo < hi:
        mid = (lo + hi) // 2
        touched.append(mid)
        if ro[mid] <= pos:
            lo = mid + 1
        else:
            hi = mid
    return lo - 1


def emulate(ro, col, val, x, P, steps, vec, drop_carry=False):
    rows = ro.size - 1
    nnz = col.size
    chunk = WAVE * P * steps
    waves = max(-(-nnz // chunk), 1)
    y = np.full(rows, np.nan, np.float32)
    writer = np.full(rows, -1, np.int64)
    ro_idx = []

    def store(r, v, w):
        assert 0 <= r < rows
        assert writer[r] in (-1, w), f"row {r} written by {writer[r]} and {w}"
        writer[r] = w
        y[r] = v

    def pos_ok(p):
        assert 0 <= p < nnz

    for w in range(waves):
        r_lo = 0 if w == 0 else _upper(ro, 0, rows + 1, w * chunk - 1,
                                       ro_idx) + 1
        r_hi = rows if w == waves - 1 else _upper(
            ro, r_lo, rows + 1, (w + 1) * chunk - 1, ro_idx) + 1
        if r_lo >= r_hi:
            continue
        p_beg = min(max(int(ro[r_lo]), 0), nnz)
        p_end = min(max(int(ro[r_hi]), p_beg), nnz)
        k_step = WAVE * P
        a0 = (p_beg & ~3) if vec else p_beg
        r_cur, carry = r_lo, 0.0
        s0 = a0
        while s0 < p_end:
            win = np.array([ro[j] if j <= r_hi else INT32_MAX
                            for j in range(r_cur + 1, r_cur + 1 + WAVE)],
                           np.int64)
            ro_idx.extend(j for j in range(r_cur + 1, r_cur + 1 + WAVE)
                          if j <= r_hi)
            lrow = np.zeros(WAVE, np.int64)
            row = np.zeros(WAVE, np.int64)
            closed = np.zeros(WAVE, np.int64)
            head = np.zeros(WAVE, np.float32)
            acc = np.zeros(WAVE, np.float32)
            nxt = np.zeros(WAVE, np.int64)
            active = np.zeros(WAVE, bool)
            for lane in range(WAVE):
                q0 = s0 + lane * P
                lb, le = max(q0, p_beg), min(q0 + P, p_end)
                if lb >= le:
                    continue
                active[lane] = True
                prods = {}
                for q in range(P):
                    p = q0 + q
                    if vec and P >= 4 and q0 + P <= nnz:
                        pos_ok(p)  # the vector load reads all P
                    if lb <= p < le:
                        pos_ok(p)
                        prods[p] = np.float32(val[p]) * np.float32(
                            x[col[p]])
                cnt = int(np.searchsorted(win, lb, side="right"))
                if cnt < WAVE:
                    lr = min(r_cur + cnt, r_hi - 1)
                    nx = int(win[lr - r_cur])
                else:
                    lr = min(_upper(ro, r_cur + WAVE + 1, r_hi + 1, lb,
                                    ro_idx), r_hi - 1)
                    ro_idx.append(lr + 1)
                    nx = int(ro[lr + 1])
                r = lr
                a = np.float32(carry if lane == 0 and not drop_carry
                               else 0.0)
                c, h = 0, np.float32(0)
                for q in range(P):
                    p = q0 + q
                    if lb <= p < le:
                        while p >= nx and r < r_hi - 1:
                            if c == 0:
                                h = a
                            else:
                                store(r, a, w)
                            c += 1
                            a = np.float32(0)
                            r += 1
                            if r - r_cur < WAVE:
                                nx = int(win[r - r_cur])
                            else:
                                ro_idx.append(r + 1)
                                nx = int(ro[r + 1])
                        a = np.float32(a + prods[p])
                lrow[lane], row[lane], closed[lane] = lr, r, c
                head[lane], acc[lane], nxt[lane] = h, a, nx
            key = np.where(active, row, -1)
            vals = np.where(active, acc, np.float32(0))
            scanned = np.zeros(WAVE, np.float32)
            for lane in range(WAVE):  # inclusive segmented scan
                scanned[lane] = vals[lane] + (
                    scanned[lane - 1] if lane and key[lane - 1] == key[lane]
                    else np.float32(0))
            step_end = min(s0 + k_step, p_end)
            for lane in range(WAVE):
                if not active[lane]:
                    continue
                prev_key = key[lane - 1] if lane else -(2 ** 31)
                prev_sc = scanned[lane - 1] if lane else np.float32(0)
                next_lrow = (lrow[lane + 1] if lane < WAVE - 1 and
                             active[lane + 1] else -2)
                if closed[lane] > 0:
                    store(lrow[lane], head[lane] + (
                        prev_sc if prev_key == lrow[lane] else 0), w)
                if next_lrow != row[lane] and nxt[lane] <= step_end:
                    store(row[lane], scanned[lane], w)
            is_open = s0 + k_step < p_end and nxt[WAVE - 1] > s0 + k_step
            carry = float(scanned[WAVE - 1]) if is_open else 0.0
            if s0 + k_step < p_end:
                if is_open:
                    r_cur = int(row[WAVE - 1])
                else:
                    r_cur = min(_upper(ro, int(row[WAVE - 1]) + 1, r_hi + 1,
                                       s0 + k_step, ro_idx), r_hi - 1)
            s0 += k_step
        for r in range(r_lo, r_hi):
            ro_idx.extend((r, r + 1))
            if ro[r] == ro[r + 1]:
                store(r, np.float32(0), w)
    assert all(0 <= j <= rows for j in ro_idx)
    assert np.all(writer >= 0), "rows never written"
    return y


def _ragged(rows, cols, seed, mean=12.0, empty=0.3, max_len=900):
    return W.random_csr(rows, cols, mean, seed, empty_fraction=empty,
                        max_len=max_len, lognormal=True)


@pytest.mark.parametrize("P,steps,vec", [(4, 1, True), (4, 2, True),
                                         (1, 1, False), (8, 1, True),
                                         (16, 1, False), (2, 3, False)])
@pytest.mark.parametrize("seed", [0, 1])
def test_row_owner_emulation_matches_oracle(orc, P, steps, vec, seed):
    csr = _ragged(700, 500, seed)
    x = np.random.default_rng(seed).uniform(-1, 1, 500).astype(np.float32)
    y = emulate(csr.row_offsets, csr.column_indices, csr.values, x, P, steps,
                vec)
    ref = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    assert_within_bound(y, ref, bound)


@pytest.mark.parametrize("lengths", [
    [0, 0, 0, 5, 0],                 # empty rows at both ends
    [300],                           # one row over several steps
    [1] * 300,                       # more rows than a window
    [0] * 70 + [3] * 70 + [0] * 70,  # long runs of empty rows
    [255, 1, 256, 0, 257, 64, 0, 0],  # rows ending at step edges
    [1000, 2, 0, 1000],
])
@pytest.mark.parametrize("P,steps,vec", [(4, 1, True), (1, 2, False),
                                         (4, 3, True)])
def test_row_owner_emulation_edges(orc, lengths, P, steps, vec):
    rng = np.random.default_rng(len(lengths))
    ro = np.zeros(len(lengths) + 1, np.int32)
    np.cumsum(lengths, out=ro[1:])
    cols = 1200
    col = np.concatenate([np.sort(rng.choice(cols, n, replace=False))
                          for n in lengths]).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    y = emulate(ro, col, val, x, P, steps, vec)
    ref = orc.spmv(ro, col, val, x)
    bound = orc.spmv_abs_bound(ro, col, val, x)
    assert_within_bound(y, ref, bound)


def test_row_owner_emulation_catches_a_dropped_carry(orc):
    """A planted mistake in the rule (lane 0 not picking up the carried
    partial) fails the comparison: rows longer than a step lose a part."""
    csr = _ragged(300, 400, 5, mean=40.0, empty=0.0, max_len=900)
    x = np.random.default_rng(5).uniform(-1, 1, 400).astype(np.float32)
    ref = orc.spmv(csr.row_offsets, csr.column_indices, csr.values, x)
    bound = orc.spmv_abs_bound(csr.row_offsets, csr.column_indices,
                               csr.values, x)
    y = emulate(csr.row_offsets, csr.column_indices, csr.values, x, 4, 1,
                True, drop_carry=True)
    with pytest.raises(AssertionError):
        assert_within_bound(y, ref, bound)


def test_row_owner_emulation_random_shapes(orc):
    """Property check over random ragged matrices: row lengths from a mix of
    empty, short and step-spanning rows, every positions-per-lane value and
    1-3 steps per chunk; the emulation must stay in range, write each row
    once and match the oracle."""
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=60, deadline=None, derandomize=True)
    @given(lengths=st.lists(st.one_of(st.just(0), st.integers(1, 6),
                                      st.integers(60, 700)),
                            min_size=1, max_size=40),
           P=st.sampled_from([1, 2, 4, 8, 16]),
           steps=st.integers(1, 3), seed=st.integers(0, 2 ** 16))
    def check(lengths, P, steps, seed):
        rng = np.random.default_rng(seed)
        cols = 800
        ro = np.zeros(len(lengths) + 1, np.int32)
        np.cumsum(lengths, out=ro[1:])
        col = (np.concatenate([np.sort(rng.choice(cols, n, replace=False))
                               for n in lengths]).astype(np.int32)
               if ro[-1] else np.zeros(0, np.int32))
        val = rng.uniform(-1, 1, col.size).astype(np.float32)
        x = rng.uniform(-1, 1, cols).astype(np.float32)
        if col.size == 0:
            return  # the launcher fills the output instead (nnz == 0)
        y = emulate(ro, col, val, x, P, steps, vec=P >= 4)
        ref = orc.spmv(ro, col, val, x)
        bound = orc.spmv_abs_bound(ro, col, val, x)
        assert_within_bound(y, ref, bound)

    check()
