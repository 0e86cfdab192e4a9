"""Seeded synthetic inputs for the five benchmark configurations.

Every generator uses ``numpy.random.default_rng(seed)`` and draws in a fixed
order, so the same seed gives the same matrix on every machine.  Shapes and
distributions follow the configuration list of the benchmark contract:

1. CSR SpMV 4096 x 4096, exactly 16 distinct sorted columns per row.
2. CSR SpMV 1,048,576 x 1,048,576, row lengths
   ``clip(rint(lognormal(mu, 1.5)), 1, 4096)`` with ``E[len] = 32``
   (``mu = ln 32 - 1.5**2 / 2``), distinct sorted uniform columns.
3. The config-2 pattern times a row-major dense RHS with 4 or 64 columns.
4. BSR 262,144 x 262,144 in 16 x 16 blocks, 8 blocks per block row: the
   diagonal, 4 distinct band offsets from +-1..+-4, 3 distinct random blocks
   off the band; values N(0, 0.02), RHS 262,144 x 128 N(0, 1).
5. Sparse attention, seq 8192, d 64, 64 x 64 block mask: blocks b-3..b
   (clipped at 0) plus 2 distinct random blocks before the window, the
   diagonal block causal (column <= row); Q, K, V ~ N(0, 1).

Distinct sorted columns are drawn as ``sort(u_i) + i`` with
``u_i ~ U{0, .., m-k}``: a strictly increasing k-subset of ``[0, m)``.  This
is the synthetic-workload layer only.  One generator follows the reference:
``reference_sweep_matrix`` restates the formulas of the reference harness's
synthetic SpMV inputs, so that its published mapping sweep can be rerun on
the same shapes.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass
class CSR:
    rows: int
    cols: int
    row_offsets: np.ndarray      # int32 [rows + 1]
    column_indices: np.ndarray   # int32 [nnz]
    values: np.ndarray           # float32 [nnz]

    @property
    def nnz(self) -> int:
        return int(self.column_indices.size)


@dataclass
class BSR:
    rows: int
    cols: int
    block_size: int
    block_row_offsets: np.ndarray     # int32 [rows / b + 1]
    block_column_indices: np.ndarray  # int32 [nnzb]
    block_values: np.ndarray          # float32 [nnzb * b * b], row-major blocks

    @property
    def nnzb(self) -> int:
        return int(self.block_column_indices.size)


def _distinct_sorted_columns(rng, lengths: np.ndarray, cols: int) -> np.ndarray:
    lengths = lengths.astype(np.int64)
    rows = lengths.size
    nnz = int(lengths.sum())
    row_id = np.repeat(np.arange(rows, dtype=np.int64), lengths)
    hi = np.repeat(cols - lengths + 1, lengths)
    u = rng.integers(0, hi, dtype=np.int64)
    keys = row_id * cols + u
    keys.sort(kind="stable")
    u = keys - row_id * cols
    starts = np.zeros(rows + 1, np.int64)
    np.cumsum(lengths, out=starts[1:])
    local = np.arange(nnz, dtype=np.int64) - np.repeat(starts[:-1], lengths)
    return (u + local).astype(np.int32)


def csr_from_lengths(rng, lengths: np.ndarray, cols: int) -> CSR:
    lengths = np.asarray(lengths, np.int64)
    ro = np.zeros(lengths.size + 1, np.int64)
    np.cumsum(lengths, out=ro[1:])
    if ro[-1] > np.iinfo(np.int32).max:
        raise ValueError("nnz exceeds the i32 index range")
    col = _distinct_sorted_columns(rng, lengths, cols)
    val = rng.uniform(-1.0, 1.0, size=col.size).astype(np.float32)
    return CSR(int(lengths.size), int(cols), ro.astype(np.int32), col, val)


def lognormal_lengths(rng, rows: int, mean: float = 32.0, sigma: float = 1.5,
                      lo: int = 1, hi: int = 4096) -> np.ndarray:
    mu = math.log(mean) - sigma * sigma / 2.0
    raw = rng.lognormal(mu, sigma, size=rows)
    return np.clip(np.rint(raw), lo, hi).astype(np.int64)


def config1(seed: int = 0):
    """4096 x 4096, 16 nnz per row; returns (csr, x)."""
    rng = np.random.default_rng(seed)
    n = 4096
    csr = csr_from_lengths(rng, np.full(n, 16, np.int64), n)
    x = rng.uniform(-1.0, 1.0, size=n).astype(np.float32)
    return csr, x


def config2(seed: int = 0, rows: int = 1 << 20):
    """Lognormal row lengths (E=32, sigma=1.5, clip [1, 4096]); (csr, x)."""
    rng = np.random.default_rng(seed)
    lengths = lognormal_lengths(rng, rows, hi=min(4096, rows))
    csr = csr_from_lengths(rng, lengths, rows)
    x = rng.uniform(-1.0, 1.0, size=rows).astype(np.float32)
    return csr, x


def config3_rhs(cols: int, k: int, seed: int = 0) -> np.ndarray:
    """Row-major dense RHS [cols][k] ~ U(-1, 1)."""
    rng = np.random.default_rng(seed + 1000 + k)
    return rng.uniform(-1.0, 1.0, size=(cols, k)).astype(np.float32)


def bsr_banded(seed: int = 0, rows: int = 262144, block_size: int = 16,
               blocks_per_row: int = 8, band: int = 4, band_blocks: int = 4,
               value_std: float = 0.02) -> BSR:
    """Config-4 BSR: diagonal + band_blocks offsets in +-1..+-band + random
    off-band blocks, sorted per block row."""
    rng = np.random.default_rng(seed)
    nbr = rows // block_size
    offsets = np.array([o for o in range(-band, band + 1) if o != 0])
    cols_per_row = []
    for br in range(nbr):
        chosen = {br}
        valid = [br + o for o in offsets if 0 <= br + o < nbr]
        take = min(band_blocks, len(valid))
        if take:
            chosen.update(int(c) for c in rng.choice(valid, size=take,
                                                     replace=False))
        want = min(blocks_per_row, nbr) - len(chosen)
        while want > 0:
            cand = rng.integers(0, nbr, size=want * 2 + 4)
            for c in cand:
                c = int(c)
                if abs(c - br) > band and c not in chosen:
                    chosen.add(c)
                    want -= 1
                    if want == 0:
                        break
            if nbr <= 2 * band + 1 and want > 0:
                # tiny matrices: fill from whatever is left
                rest = [c for c in range(nbr) if c not in chosen]
                chosen.update(rest[:want])
                want = 0
        cols_per_row.append(sorted(chosen))
    counts = np.array([len(c) for c in cols_per_row], np.int64)
    bro = np.zeros(nbr + 1, np.int64)
    np.cumsum(counts, out=bro[1:])
    bcol = np.concatenate([np.asarray(c, np.int32) for c in cols_per_row])
    nnzb = int(bro[-1])
    bval = rng.normal(0.0, value_std,
                      size=nnzb * block_size * block_size).astype(np.float32)
    return BSR(rows, rows, block_size, bro.astype(np.int32), bcol, bval)


def config4(seed: int = 0, rows: int = 262144, k: int = 128):
    bsr = bsr_banded(seed, rows)
    rng = np.random.default_rng(seed + 7)
    rhs = rng.standard_normal(size=(rows, k), dtype=np.float32)
    return bsr, rhs


def attention_mask(seq: int = 8192, block: int = 64, window: int = 4,
                   random_blocks: int = 2, seed: int = 0) -> CSR:
    """Block-sparse causal mask as an element CSR (values 0.0)."""
    rng = np.random.default_rng(seed)
    nb = seq // block
    block_cols = []
    for b in range(nb):
        local = list(range(max(0, b - window + 1), b + 1))
        before = max(0, b - window + 1)
        extra = []
        if before > 0:
            take = min(random_blocks, before)
            extra = sorted(int(c) for c in rng.choice(before, size=take,
                                                      replace=False))
        block_cols.append(sorted(extra + local))
    lengths = np.zeros(seq, np.int64)
    cols_list = []
    for b in range(nb):
        for i in range(block):
            r = b * block + i
            parts = []
            for cb in block_cols[b]:
                if cb < b:
                    parts.append(np.arange(cb * block, cb * block + block))
                else:
                    parts.append(np.arange(cb * block, r + 1))
            c = np.concatenate(parts)
            lengths[r] = c.size
            cols_list.append(c)
    ro = np.zeros(seq + 1, np.int64)
    np.cumsum(lengths, out=ro[1:])
    col = np.concatenate(cols_list).astype(np.int32)
    return CSR(seq, seq, ro.astype(np.int32), col,
               np.zeros(col.size, np.float32))


def config5(seed: int = 0, seq: int = 8192, d: int = 64):
    """(mask csr, query [S,d], transposed_key [d,S], value [S,d], alpha)."""
    mask = attention_mask(seq, seed=seed)
    rng = np.random.default_rng(seed + 5)
    q = rng.standard_normal(size=(seq, d), dtype=np.float32)
    k = rng.standard_normal(size=(seq, d), dtype=np.float32)
    v = rng.standard_normal(size=(seq, d), dtype=np.float32)
    kt = np.ascontiguousarray(k.T)
    return mask, q, kt, v, 1.0 / math.sqrt(d)


def reference_sweep_matrix(distribution: str, nnz_per_row: int,
                           rows: int = 65536, cols: int = 65536) -> CSR:
    """The reference harness's synthetic SpMV input, restated
    (benchmark/run_spmv_benchmark.py:225-259): row lengths ``uniform`` (every
    row nnz_per_row), ``alternating`` (1 and 2 nnz_per_row - 1) or
    ``skewed`` (seven of every eight rows 1, the eighth 8 nnz_per_row - 7);
    the column of position p is p mod cols and every value is 1.0.  The
    harness multiplies it by a vector of ones (benchmark/spmv.mlir.in)."""
    r = np.arange(rows, dtype=np.int64)
    if distribution == "uniform":
        lengths = np.full(rows, nnz_per_row, dtype=np.int64)
    elif distribution == "alternating":
        lengths = np.where(r % 2 == 0, 1, 2 * nnz_per_row - 1)
    elif distribution == "skewed":
        lengths = np.where(r % 8 == 7, 8 * nnz_per_row - 7, 1)
    else:
        raise ValueError(f"unknown distribution: {distribution}")
    ro = np.zeros(rows + 1, dtype=np.int32)
    np.cumsum(lengths, out=ro[1:])
    nnz = int(ro[-1])
    col = (np.arange(nnz, dtype=np.int64) % cols).astype(np.int32)
    return CSR(rows, cols, ro, col, np.ones(nnz, dtype=np.float32))


def random_csr(rows: int, cols: int, mean_len: float, seed: int,
               empty_fraction: float = 0.1, max_len: int | None = None,
               lognormal: bool = False) -> CSR:
    """Small ragged CSR for parity tests, including empty rows."""
    rng = np.random.default_rng(seed)
    max_len = cols if max_len is None else min(max_len, cols)
    if lognormal:
        lengths = lognormal_lengths(rng, rows, mean=max(mean_len, 1.0),
                                    hi=max_len)
    else:
        lengths = rng.poisson(mean_len, size=rows).astype(np.int64)
    lengths = np.clip(lengths, 0, max_len)
    if empty_fraction > 0:
        lengths[rng.random(rows) < empty_fraction] = 0
    return csr_from_lengths(rng, lengths, cols)


def algorithmic_bytes_spmv(rows: int, cols: int, nnz: int) -> int:
    """4(n+1) row offsets + 4 nnz columns + 4 nnz values + 4 m x + 4 n y."""
    return 4 * (rows + 1) + 8 * nnz + 4 * cols + 4 * rows


def algorithmic_bytes_spmm(rows: int, cols: int, nnz: int, k: int) -> int:
    """CSR arrays once, each RHS row once, each output element once."""
    return 8 * nnz + 4 * (rows + 1) + 4 * cols * k + 4 * rows * k


def algorithmic_bytes_bsr(rows: int, cols: int, nnzb: int, b: int, k: int,
                          value_bytes: int = 4, out_bytes: int = 4) -> int:
    """Block-row offsets, block columns, blocks and RHS once, output once."""
    nbr = rows // b
    return (4 * (nbr + 1) + 4 * nnzb + value_bytes * nnzb * b * b
            + value_bytes * cols * k + out_bytes * rows * k)
