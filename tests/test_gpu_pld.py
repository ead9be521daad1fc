"""The device PLD proposer (qws_pld_* through the C ABI) against the CPU oracle (oracle/pld.py, itself equal to
the reference's proposer built from source: tests/test_pld_oracle.py): tails, lengths and agreement lengths
bit-exact for many sequences per call, across configurations, draft counts, appends with -1 padding, long
histories, and the overflow rule."""
import random

import numpy as np
import pytest
import torch

from oracle.pld import Pld, PldCfg
from qwen_warp_amd import _lib
from qwen_warp_amd.pld import DevicePld

pytestmark = pytest.mark.gpu

CFGS = [PldCfg(), PldCfg(n=1, min_len=1, max_tail=7), PldCfg(n=3, min_len=3, max_tail=2, cap=5, back=9), PldCfg(n=4, min_len=4, cap=2, back=4),
        PldCfg(longest=0, min_len=2), PldCfg(n=2, min_len=0, max_tail=7, cap=1000, back=200)]


def _cfg(c: PldCfg):
    return _lib.PldCfg(c.n, c.min_len, c.max_tail, c.cap, c.back, c.longest)


def _check(dev, refs, seqs, drafts, mt, ml, label):
    d = torch.tensor(drafts, dtype=torch.int32, device="cuda") if drafts and len(drafts[0]) else None
    out, n, l = dev.propose(seqs, d, mt, ml)
    out, n, l = out.cpu().numpy(), n.cpu().numpy(), l.cpu().numpy()
    for b, s in enumerate(seqs):
        want, wl = refs[s].propose(drafts[b] if drafts else [], mt, ml)
        got = out[b, : n[b]].tolist()
        assert (got, int(l[b])) == (want, wl), f"{label} row {b} (seq {s}): {got}, l={int(l[b])} != {want}, l={wl}"
        assert (out[b, n[b]:] == -1).all()


@pytest.mark.parametrize("ci", range(len(CFGS)))
def test_propose_matches_oracle(ci):
    cfg = CFGS[ci]
    rng = random.Random(99 + ci)
    S = 12
    dev = DevicePld(S, 4096, _cfg(cfg))
    refs = [Pld(cfg) for _ in range(S)]
    for s in range(S):
        alpha = rng.choice([3, 5, 12, 60])
        ctx = [rng.randrange(alpha) for _ in range(rng.randrange(0, 700))]
        dev.reset(s, ctx)
        refs[s].reset(ctx)
    for step in range(25):
        seqs = rng.sample(range(S), rng.randrange(1, S + 1))
        nd = rng.randrange(0, 8)
        drafts = [[rng.randrange(12) for _ in range(nd)] for _ in seqs]
        _check(dev, refs, seqs, drafts if nd else None, rng.randrange(0, 9), rng.randrange(0, 7), f"cfg {ci} step {step}")
        # append: per row 1..T tokens, then -1 padding
        T = rng.randrange(1, 10)
        arr = np.full((len(seqs), T), -1, dtype=np.int32)
        for b, s in enumerate(seqs):
            k = rng.randrange(1, T + 1)
            toks = [rng.randrange(12) for _ in range(k)]
            arr[b, :k] = toks
            refs[s].append(toks)
        dev.append(seqs, torch.from_numpy(arr).cuda())


def test_long_history_and_repeats():
    """A 60,000-token history with a repeating block (many candidates, the cap decides), and a rare key."""
    rng = random.Random(5)
    base = [rng.randrange(1000) for _ in range(300)]
    hist = (base * 200)[:60000] + [77777, 88888]
    dev = DevicePld(2, 1 << 16)
    refs = [Pld(), Pld()]
    for s, ctx in enumerate([hist, hist[:-2]]):
        dev.reset(s, ctx)
        refs[s].reset(ctx)
    for nd in (0, 1, 3, 7):
        drafts = [[base[i % 300] for i in range(5, 5 + nd)], [77777, 88888, 5][:nd] + [1] * max(0, nd - 3)]
        _check(dev, refs, [0, 1], drafts if nd else None, 4, 3, f"nd {nd}")


def test_overflow_and_bad_rows():
    dev = DevicePld(3, 16)
    ref = Pld()
    ctx = [1, 2, 3, 1, 2, 3, 1, 2]
    dev.reset(0, ctx)
    ref.reset(ctx)
    dev.reset(1, ctx)
    # sequence 1 overflows (8 + 9 > 16): its proposals are empty until a reset
    dev.append([1], torch.tensor([[3, 1, 2, 3, 1, 2, 3, 1, 2]], dtype=torch.int32, device="cuda"))
    out, n, l = dev.propose([0, 1, -1, 7])
    assert n.tolist()[1:] == [0, 0, 0] and l.tolist()[1:] == [0, 0, 0]
    assert (out[0, : n[0]].cpu().tolist(), int(l[0])) == ref.propose([])
    dev.reset(1, ctx)
    out, n, l = dev.propose([1])
    assert (out[0, : n[0]].cpu().tolist(), int(l[0])) == ref.propose([])
