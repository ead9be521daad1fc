"""CPU restatement of the quantised head's candidate select + exact rescore -- TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).  Restates engine/src/head_q.cu:124-302 (k_chunkmax, k_extract, k_rank, k_rescore) and
engine/include/head_q.h:21-36 as a definition:

  key(v) = ord32(v) << 32 | (2^32 - 1 - index), ord32 the order-preserving map of fp32 bits (-0 below +0);
           NaN logits are never candidates (head_q.cu:113-117, 175).
  candidates of row t = the R largest keys of the approximate logits, in descending key order (rank 0 first;
           a row with fewer than R non-NaN logits leaves -1 after them).
  exact logit of a candidate = sum_k bf16(w[id][k]) * bf16(x[t][k]), here in float64 (the GPU accumulates the exact
           bf16 products in fp32 in its own order: tests compare within that accumulation's error bound).
  out_tok[t] = the candidate with the largest exact logit, the lowest token id on ties (head_q.cu:284-298).
"""
from typing import Optional

import numpy as np
import torch


def ord32(v: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def keys(v: np.ndarray) -> np.ndarray:
    """uint64 keys of a logits row (0 for NaN: never a candidate)."""
    idx = np.arange(v.size, dtype=np.uint64)
    k = (ord32(v) << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)
    return np.where(np.isnan(v), np.uint64(0), k)


def candidates(v: np.ndarray, R: int) -> np.ndarray:
    """Row indices of the R largest keys, rank order; -1 past the non-NaN ones."""
    k = keys(v)
    order = np.argsort(k)[::-1]
    out = np.full(R, -1, dtype=np.int64)
    n = min(R, int((k > 0).sum()))
    out[:n] = order[:n]
    return out


def exact_logits(w_rows: torch.Tensor, x_row: torch.Tensor) -> np.ndarray:
    """float64 dot products of bf16 rows [R][K] with a bf16 vector [K], and the fp32 accumulation error bound of
    each (K * 2^-23 * sum |w x|, with room)."""
    a = w_rows.to(torch.float64)
    b = x_row.to(torch.float64)
    return (a @ b).numpy(), ((a * b).abs().sum(1) * (w_rows.shape[1] * 2.0 ** -23)).numpy()


def select_rescore(logits: np.ndarray, w: torch.Tensor, x: torch.Tensor, R: int, ids: Optional[np.ndarray] = None):
    """logits [T][N] fp32, w [rows][K] bf16 (CPU), x [T][K] bf16.  Returns per row (candidate ids in rank order,
    -1 past them; their exact logits (float64); their error bounds)."""
    out = []
    for t in range(logits.shape[0]):
        c = candidates(logits[t], R)
        rows = c[c >= 0]
        tok = ids[rows] if ids is not None else rows
        ex, tol = exact_logits(w[torch.as_tensor(tok, dtype=torch.long)], x[t]) if len(rows) else (np.zeros(0), np.zeros(0))
        out.append((np.where(c >= 0, (ids[np.maximum(c, 0)] if ids is not None else c), -1), ex, tol))
    return out
