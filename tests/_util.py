"""Shared test helpers: textbook references (double precision), chi-square, seeded case generators."""
import json
import math
from pathlib import Path

import numpy as np
import torch
from scipy import stats

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "reference_vectors.json").read_text())
V = 248320


def chi2_sf(x, dof):
    return float(stats.chi2.sf(x, dof))


def chi_square(counts, probs, n):
    """Pearson chi-square of observed counts against expected probabilities (cells with expected < 5 pooled),
    as tests/test_spec_procs.py:111-119."""
    counts = np.asarray(counts, dtype=np.float64)
    exp = np.asarray(probs, dtype=np.float64) * n
    small = exp < 5.0
    obs_p = np.concatenate([counts[~small], [counts[small].sum()]])
    exp_p = np.concatenate([exp[~small], [exp[small].sum()]])
    keep = exp_p > 0
    stat = float(((obs_p[keep] - exp_p[keep]) ** 2 / exp_p[keep]).sum())
    dof = int(keep.sum()) - 1
    return stat, dof, chi2_sf(stat, dof)


def textbook_dist(x, temperature, top_k=0, top_p=1.0, min_p=0.0):
    """The textbook definition in float64 (vLLM order: temperature -> min_p -> top-k -> top-p; ties in rank
    broken by lower index, exactly K kept), independent of the oracle's fixed-point arithmetic.
    Returns {token: probability}."""
    x = x.double()
    finite = torch.isfinite(x) | (x == math.inf)
    ids = torch.nonzero(x > -math.inf).flatten()
    xv = x[ids]
    order = np.lexsort((ids.numpy(), -xv.numpy()))
    ids, xv = ids[order], xv[order]
    z = (xv - xv[0]) / float(np.float32(temperature))
    e = torch.exp(z)
    if min_p > 0:
        keep = e >= float(np.float32(min_p))
        ids, e = ids[keep], e[keep]
    if top_k > 0:
        ids, e = ids[:top_k], e[:top_k]
    p = e / e.sum()
    if top_p < 1.0:
        before = torch.cumsum(p, 0) - p
        keep = before < float(np.float32(top_p))
        keep[0] = True
        ids, p = ids[keep], p[keep]
        p = p / p.sum()
    del finite
    return {int(i): float(v) for i, v in zip(ids, p)}


def zipf_ids(g: torch.Generator, n: int, s: float, vocab: int, perm: torch.Tensor):
    """n ids from a bounded Zipf(s) over ranks 1..vocab mapped through a permutation (config 2)."""
    ranks = torch.arange(1, vocab + 1, dtype=torch.float64)
    w = ranks ** (-s)
    r = torch.multinomial(w / w.sum(), n, replacement=True, generator=g)
    return perm[r]
