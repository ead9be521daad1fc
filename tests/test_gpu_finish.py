"""Device decode-step bookkeeping (qws_finish through the C ABI) against a host model of the reference's spec_finish
(engine/src/mtp_sample.h:65-92): output rings (with wraparound), positions, last tokens, cycle counters and the
accepted-length histogram; the same launch's processor-state note (slot contents decoded and compared with
counts kept on the host) and PLD append (proposals equal the oracle's after the same appends)."""
import random

import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from oracle.pld import Pld
from qwen_warp_amd.sampling import ProcState
from _util import V

pytestmark = pytest.mark.gpu
BLK = 8192


def decode_state(st: ProcState, slot: int) -> dict:
    """{token: (generated count, in prompt)} from a slot's entries (qws_block.h state layout)."""
    G = (st.V + BLK - 1) // BLK
    stride = 256 + G * BLK * 4
    raw = st.mem[slot * stride:(slot + 1) * stride].cpu().numpy().view(np.uint32)
    cnt = raw[:G]
    out = {}
    for g in range(G):
        ent = raw[64 + g * BLK: 64 + g * BLK + int(cnt[g])]
        for e in ent.tolist():
            out[g * BLK + (e & 0x1FFF)] = (e >> 16, (e >> 13) & 1)
    return out


def test_finish_matches_model():
    rng = random.Random(3)
    N, R, T = 6, 16, 9
    book = q.StepBook(N, R)
    st = ProcState(N, V, "cuda")
    pld = q.DevicePld(N, 4096)
    model = [dict(pos=0, last=0, outn=0, cycles=0, hist=[0] * 8, ring=[-1] * R) for _ in range(N)]
    counts = [dict() for _ in range(N)]
    prompts = []
    refs = [Pld() for _ in range(N)]
    for s in range(N):
        prompt = [rng.randrange(50) for _ in range(40)] + [rng.randrange(V) for _ in range(10)]
        prompts.append(set(prompt))
        st.begin(s, prompt, [])
        pld.reset(s, prompt)
        refs[s].reset(prompt)
        book.start(s, len(prompt), prompt[-1])
        model[s].update(pos=len(prompt), last=prompt[-1])
    for step in range(12):
        seqs = rng.sample(range(N), rng.randrange(1, N + 1))
        B = len(seqs)
        toks = np.full((B, T), -1, dtype=np.int32)
        use_counts = step % 2 == 0
        cnt = np.zeros(B, dtype=np.int32)
        for b in range(B):
            a = rng.randrange(0 if use_counts else 1, T + 1)
            toks[b, :a] = [rng.randrange(50) if rng.random() < 0.7 else rng.randrange(V) for _ in range(a)]
            cnt[b] = a
            if use_counts and a < T and rng.random() < 0.5:
                toks[b, a] = 123  # beyond the count: ignored
        book.finish(seqs, torch.from_numpy(toks).cuda(), torch.from_numpy(cnt).cuda() if use_counts else None, state=st, pld=pld)
        for b, s in enumerate(seqs):
            a = int(cnt[b])
            if a == 0:
                continue
            y = toks[b, :a].tolist()
            m = model[s]
            for i, t in enumerate(y):
                m["ring"][(m["outn"] + i) % R] = t
            m.update(outn=m["outn"] + a, pos=m["pos"] + a, last=y[-1], cycles=m["cycles"] + 1)
            m["hist"][min(a - 1, 7)] += 1
            for t in y:
                counts[s][t] = counts[s].get(t, 0) + 1
            refs[s].append(y)
    rings = book.rings.cpu().numpy()
    for s in range(N):
        got = book.read(s)
        m = model[s]
        assert got == {k: m[k] for k in ("pos", "last", "outn", "cycles", "hist")}, s
        assert rings[s].tolist() == m["ring"], s
        want = {t: (counts[s].get(t, 0), int(t in prompts[s])) for t in set(counts[s]) | prompts[s]}
        assert decode_state(st, s) == want, s
    out, n, l = pld.propose(list(range(N)))
    for s in range(N):
        assert (out[s, : n[s]].cpu().tolist(), int(l[s])) == refs[s].propose([]), s
