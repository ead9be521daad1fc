"""Synthetic workloads of the five benchmark configurations (BASELINE.json `configs`): seeded logits, per-row
sampling parameters and token histories, and each one's algorithmic byte count.  Used by bench.py, the
parity tests and the smoke check; data is synthetic (no checkpoint, no network)."""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .sampling import RowSpec

V = 248320
STOP_EOS = (248044, 248046)  # the reference tests' EOS pair (tests/test_logit_procs.py:112)
STOP_FIXED = 248045


@dataclass
class Workload:
    name: str
    logits: torch.Tensor            # CPU [B, V] fp32 or bf16
    rows: list
    algo_bytes: int
    note: str = ""
    extra: dict = field(default_factory=dict)


def _gen(cfg: int) -> torch.Generator:
    return torch.Generator().manual_seed(1000 + cfg)


def _bytes(logits: torch.Tensor, rows) -> int:
    b = logits.numel() * logits.element_size()
    for r in rows:
        b += 4 * (len(r.gen) + len(r.prompt)) + 4 * len(r.stop) + 8 * len(r.bias or {})
        if r.banned is not None:
            b += logits.shape[1] // 8
    return b


def c1(greedy: bool = False, B: int = 1) -> Workload:
    """B=1, fp32 N(0,3) with 32 random ids boosted +8; T 0.7, top-k 20, top-p 0.8, repetition 1.05 over a
    2,048-token uniform history, Philox seed 0 (greedy variant: T = 0, same processors)."""
    g = _gen(1)
    x = torch.randn(B, V, generator=g) * 3.0
    for b in range(B):
        boost = torch.randperm(V, generator=g)[:32]
        x[b, boost] += 8.0
    rows = []
    for b in range(B):
        hist = torch.randint(0, V, (2048,), generator=g).tolist()
        rows.append(RowSpec(temperature=0.0 if greedy else 0.7, top_k=20, top_p=0.8, min_p=0.0, repetition=1.05, gen=hist, seed=0, row_key=b))
    return Workload("c1_greedy" if greedy else "c1", x, rows, _bytes(x, rows))


def zipf_ids(g, n, vocab, perm, s=1.1):
    ranks = torch.arange(1, vocab + 1, dtype=torch.float64)
    w = ranks ** (-s)
    r = torch.multinomial(w / w.sum(), n, replacement=True, generator=g)
    return perm[r]


def c2(B: int = 8) -> Workload:
    """B=8 bf16 N(0,2.5); per row T ~ U[0.3,1.2], top-k in {0,20,50,1000}, top-p ~ U[0.5,1], min-p ~ U[0,0.1],
    presence / frequency ~ U[0,1.5]; per-row Zipf(1.1) histories of 512 .. 32,768 tokens."""
    g = _gen(2)
    x = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
    perm = torch.randperm(V, generator=g)
    lens = [512, 1024, 2048, 4096, 8192, 16384, 24576, 32768]
    ks = [0, 20, 50, 1000]
    rows = []
    for b in range(B):
        u = torch.rand(5, generator=g).tolist()
        k = ks[int(torch.randint(0, 4, (1,), generator=g))]
        hist = zipf_ids(g, lens[b % len(lens)], V, perm).tolist()
        rows.append(RowSpec(temperature=0.3 + 0.9 * u[0], top_k=k, top_p=0.5 + 0.5 * u[1], min_p=0.1 * u[2], presence=1.5 * u[3],
                            frequency=1.5 * u[4], gen=hist, seed=2000 + b, row_key=b))
    return Workload("c2", x, rows, _bytes(x, rows))


def c3(B: int = 4, K: int = 8, Vd: int = 64000, aligned: bool = False) -> Workload:
    """Speculative verify: target fp32 [B][K+1][V] ~ N(0,3); draft probs fp32 [B][K][Vd] = softmax of N(0,3) rows over
    a reduced vocabulary of Vd ids (a random injective table, randperm(V)[:Vd]); draft tokens sampled from the draft
    probs (torch.multinomial on the CPU); T 1.0, top-p 0.95, top-k 0.  aligned=True: the drafter's logits follow the
    target's at its ids plus N(0,1) noise instead (more drafts accepted).  extra: idmap [Vd], draft_probs,
    drafts [B][K] (all CPU).  Algorithmic bytes: target logits + draft probs + id table + draft tokens."""
    g = _gen(3)
    tl = torch.randn(B, K + 1, V, generator=g) * 3.0
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32)
    if aligned:
        dl = tl[:, :K, :][:, :, idmap.long()] + torch.randn(B, K, Vd, generator=g)
    else:
        dl = torch.randn(B, K, Vd, generator=g) * 3.0
    q = torch.softmax(dl, dim=2).float()
    j = torch.multinomial(q.reshape(B * K, Vd).double(), 1, generator=g).reshape(B, K)
    drafts = idmap[j].to(torch.int32)
    rows = [RowSpec(temperature=1.0, top_k=0, top_p=0.95, seed=3000 + b, row_key=b, position=7) for b in range(B)]
    nbytes = tl.numel() * 4 + q.numel() * 4 + idmap.numel() * 4 + drafts.numel() * 4
    return Workload("c3_aligned" if aligned else "c3", tl, rows, nbytes, extra=dict(idmap=idmap, draft_probs=q, drafts=drafts, K=K))


def c4(B: int = 64) -> Workload:
    """B=64 fp32 N(0,0.5) (near-flat): T 1.0, top-k 0, top-p 0.95, repetition 1.1 over 4,096-token uniform histories."""
    g = _gen(4)
    x = torch.randn(B, V, generator=g) * 0.5
    rows = []
    for b in range(B):
        hist = torch.randint(0, V, (4096,), generator=g).tolist()
        rows.append(RowSpec(temperature=1.0, top_k=0, top_p=0.95, repetition=1.1, gen=hist, seed=4000, row_key=b))
    return Workload("c4", x, rows, _bytes(x, rows))


def c5(B: int = 32) -> Workload:
    """B=32 bf16 N(0,3): 300 distinct (id, U[-100,100]) bias pairs, min_tokens=1 with nothing generated on 3 stop
    ids, a banned bitmask uint32[B][7760] at 1% density; top-k 50, T 0.6, seeded."""
    g = _gen(5)
    x = (torch.randn(B, V, generator=g) * 3.0).to(torch.bfloat16)
    W = V // 32
    rows = []
    for b in range(B):
        ids = torch.randperm(V, generator=g)[:300].tolist()
        vals = ((torch.rand(300, generator=g) * 200.0) - 100.0).tolist()
        bits = (torch.rand(V, generator=g) < 0.01).numpy()
        m = np.zeros(W, dtype=np.uint32)
        nz = np.nonzero(bits)[0]
        np.bitwise_or.at(m, nz >> 5, (np.uint32(1) << (nz & 31).astype(np.uint32)))
        rows.append(RowSpec(temperature=0.6, top_k=50, top_p=1.0, bias=dict(zip(ids, vals)), min_tokens=1, ngen=0,
                            stop=[STOP_EOS[0], STOP_EOS[1], STOP_FIXED], banned=m, seed=5000 + b, row_key=b))
    return Workload("c5", x, rows, _bytes(x, rows))


ALL = {"c1": c1, "c1_greedy": lambda **k: c1(greedy=True, **k), "c2": c2, "c3": c3, "c3_aligned": lambda **k: c3(aligned=True, **k), "c4": c4, "c5": c5}
