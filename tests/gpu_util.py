"""Helpers for the GPU parity tests: move seeded numpy inputs to the device,
call the C ABI through the Python mirror, bring results back."""
import sys

import numpy as np
import torch

import sparsewavecomp_amd as sw

DEV = torch.device("cuda:0")


def say(msg: str):
    """Name the case before its GPU step (flushed)."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def t(a, dtype=None):
    a = np.ascontiguousarray(a)
    x = torch.from_numpy(a)
    if dtype is not None:
        x = x.to(dtype)
    return x.to(DEV)


def spmv(csr, x, options, out_fill=float("nan")):
    say(f"spmv rows={csr.rows} nnz={csr.nnz} opts='{options}'")
    ro, col, val = t(csr.row_offsets), t(csr.column_indices), t(csr.values)
    xv = t(x)
    y = torch.full((csr.rows,), out_fill, dtype=torch.float32, device=DEV)
    sw.spmv(ro, col, val, xv, y, options=options)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def spmm(csr, rhs, options, out_fill=float("nan")):
    say(f"spmm rows={csr.rows} nnz={csr.nnz} k={rhs.shape[1]} opts='{options}'")
    ro, col, val = t(csr.row_offsets), t(csr.column_indices), t(csr.values)
    b = t(rhs)
    out = torch.full((csr.rows, rhs.shape[1]), out_fill, dtype=torch.float32,
                     device=DEV)
    sw.spmm(ro, col, val, b, out, options=options)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest even) and back, as torch does."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(
        torch.bfloat16).to(torch.float32).numpy()
