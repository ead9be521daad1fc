"""Device-resident processor state (ProcState over qws_state_begin / qws_state_note) through the C ABI: a row that
takes its prompt set and generated counts from a slot samples exactly like the same row with its history passed
per call (processed logits bit-identical, tokens and survivor probabilities equal), after begin and after any
sequence of notes; the processed logits also equal the CPU oracle's."""
import copy

import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from qwen_warp_amd import workloads
from oracle import sampler as S
from _util import V

pytestmark = pytest.mark.gpu


def _as_state(rows, slots):
    out = []
    for r, s in zip(rows, slots):
        t = copy.deepcopy(r)
        t.ngen = len(r.gen) if r.ngen is None else r.ngen
        t.state_slot = s
        out.append(t)
    return out


def _same(sampler, logits, rows, state_rows, state, label):
    lg = logits.cuda()
    a = torch.empty(logits.shape, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    ta = sampler.run(q.PackedBatch(rows, V, "cuda"), lg, out_logits=a)
    tb = sampler.run(q.PackedBatch(state_rows, V, "cuda", state), lg, out_logits=b)
    assert torch.equal(a, b), f"{label}: {int((a != b).sum())} processed logits differ"
    assert torch.equal(ta, tb), f"{label}: tokens {ta.tolist()} vs {tb.tolist()}"
    pa = sampler.probs(lg, rows)[1]
    pb = torch.zeros_like(pa)
    info = torch.empty(len(rows), dtype=torch.int32, device="cuda")
    sampler.run(q.PackedBatch(state_rows, V, "cuda", state), lg, out_probs=pb, out_info=info)
    assert torch.equal(pa, pb), f"{label}: probabilities differ"
    return a.cpu()


def test_begin_matches_history_c2(sampler):
    """The C2 rows (Zipf histories of 512 .. 32,768 tokens, penalties and per-row parameters), plus a prompt set."""
    w = workloads.c2()
    g = torch.Generator().manual_seed(77)
    rows = copy.deepcopy(w.rows)
    for i, r in enumerate(rows):
        r.prompt = torch.randint(0, V, (200 * i,), generator=g).tolist()
        r.repetition = 1.0 + 0.1 * i
    st = q.ProcState(len(rows) + 3, V, "cuda")
    slots = [len(rows) + 2 - i for i in range(len(rows))]
    for r, s in zip(rows, slots):
        st.begin(s, r.prompt, r.gen)
    got = _same(sampler, w.logits, rows, _as_state(rows, slots), st, "c2")
    for b in (0, 7):  # the oracle on the shortest and the longest history
        r = rows[b]
        pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, prompt=r.prompt, gen=r.gen)
        assert torch.equal(got[b], S.process(w.logits[b].float(), pr, []))


def test_notes_match_history(sampler):
    """begin with part of the history, then notes of one token per step, a multi-token step with repeats and -1
    padding, and tokens of a block that had no entry yet; each stage against the full CSR history."""
    g = torch.Generator().manual_seed(5)
    B = 6
    logits = torch.randn(B, V, generator=g) * 3.0
    pool = torch.randint(0, V, (40,), generator=g).tolist()
    rows = []
    for b in range(B):
        gen = [pool[int(i)] for i in torch.randint(0, 40, (30 + 7 * b,), generator=g)]
        rows.append(q.RowSpec(temperature=0.8, top_k=0, top_p=0.9, seed=b, row_key=b, presence=0.4, frequency=0.3, repetition=1.2,
                              prompt=torch.randint(0, V, (50,), generator=g).tolist(), gen=gen))
    st = q.ProcState(B, V, "cuda")
    n0 = 10
    for b, r in enumerate(rows):
        st.begin(b, r.prompt, r.gen[:n0])
    hist = [list(r.gen[:n0]) for r in rows]
    slots = list(range(B))

    def stage(label):
        now = copy.deepcopy(rows)
        for r, h in zip(now, hist):
            r.gen = list(h)
        _same(sampler, logits, now, _as_state(now, slots), st, label)

    stage("begin")
    for step in range(3):  # one token per row per step
        tok = [rows[b].gen[n0 + step] for b in range(B)]
        st.note(slots, torch.tensor(tok, dtype=torch.int32, device="cuda"))
        for b in range(B):
            hist[b].append(tok[b])
    stage("3 single-token notes")
    # a verify-like step: 9 tokens per row with repeats, -1 after the emitted ones, rows 1 and 4 skipped
    T = 9
    arr = np.full((B, T), -1, dtype=np.int32)
    for b in range(B):
        n = 1 + (b * 2) % T
        toks = [rows[b].gen[n0 + 3 + (k % 3)] for k in range(n)] + ([V - 1] if n < T else [])
        arr[b, : len(toks)] = toks
    use = [s if b not in (1, 4) else -1 for b, s in enumerate(slots)]
    st.note(use, torch.from_numpy(arr).cuda())
    for b in range(B):
        if b not in (1, 4):
            hist[b] += [int(v) for v in arr[b] if 0 <= v < V]
    stage("multi-token note")
    # the rest of each history, several tokens per call
    for b in range(B):
        rest = rows[b].gen[n0 + 3:]
        for k in range(0, len(rest), 4):
            chunk = rest[k:k + 4]
            t = np.full((1, 4), -1, dtype=np.int32)
            t[0, : len(chunk)] = chunk
            st.note([b], torch.from_numpy(t).cuda())
            hist[b] += chunk
    stage("full histories")


def test_full_block_and_saturation(sampler):
    """A slot whose entries cover every token of block 1 (a full bucket), notes that only update entries there, and
    the last (ragged) block."""
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(2, V, generator=g) * 2.0
    block1 = list(range(8192, 16384))
    tail = list(range(V - 40, V))
    r = q.RowSpec(temperature=1.0, top_p=0.95, seed=3, frequency=0.01, presence=0.2, repetition=1.05, gen=block1 + tail + block1[:100],
                  prompt=tail[:5])
    r2 = copy.deepcopy(r)
    r2.gen = tail * 3
    st = q.ProcState(2, V, "cuda")
    st.begin(0, r.prompt, r.gen)
    st.begin(1, r2.prompt, r2.gen)
    _same(sampler, logits, [r, r2], _as_state([r, r2], [0, 1]), st, "full block")
    extra = np.asarray([[8192, 16383, V - 1, 9000]], dtype=np.int32)
    st.note([0], torch.from_numpy(extra).cuda())
    r.gen = r.gen + extra[0].tolist()
    _same(sampler, logits, [r, r2], _as_state([r, r2], [0, 1]), st, "full block + note")


def test_verify_with_state(sampler):
    """qws_verify over rows whose history comes from the state equals the same call with CSR histories."""
    w = workloads.c3(B=3, K=5, Vd=4096)
    x = w.extra
    seqs = copy.deepcopy(w.rows)
    g = torch.Generator().manual_seed(11)
    for s in seqs:
        s.gen = torch.randint(0, V, (300,), generator=g).tolist() + x["drafts"][0].tolist()[:2]
        s.presence, s.repetition = 0.7, 1.3
    st = q.ProcState(4, V, "cuda")
    for i, s in enumerate(seqs):
        st.begin(i + 1, s.prompt, s.gen)
    tl, dp = w.logits.cuda(), x["draft_probs"].cuda()
    inv = sampler.verify_map(x["idmap"].cuda(), V)
    d = x["drafts"].cuda()
    oa, na = sampler.verify(tl, dp, inv, d, seqs)
    ob, nb = sampler.verify(tl, dp, inv, d, _as_state(seqs, [1, 2, 3]), state=st)
    assert torch.equal(oa, ob) and torch.equal(na, nb)


def test_state_validation(sampler):
    st = q.ProcState(2, V, "cuda")
    with pytest.raises(q.ValidationError):
        st.begin(2, [1], [2])
    with pytest.raises(q.ValidationError):
        st.begin(0, [V], [])
    with pytest.raises(q.ValidationError):
        q.PackedBatch([q.RowSpec(temperature=1.0, presence=1.0, state_slot=0)], V, "cuda")
    with pytest.raises(q.ValidationError):
        q.PackedBatch([q.RowSpec(temperature=1.0, presence=1.0, state_slot=2)], V, "cuda", st)
    with pytest.raises(q.ValidationError):
        st.note([0, 0], torch.zeros(2, dtype=torch.int32, device="cuda"))


def test_state_rows_at_benchmark_shape(sampler):
    """fp32 rows whose only list is a state slot take k_scan's in-place processing of the slot's entries: the 64 C4
    rows (512-thread workgroups) equal their per-call histories and, on two rows, the oracle's processed logits."""
    w = workloads.c4()
    st = q.ProcState(len(w.rows), V, "cuda")
    for b, r in enumerate(w.rows):
        st.begin(b, r.prompt, r.gen)
    got = _same(sampler, w.logits, w.rows, _as_state(w.rows, list(range(len(w.rows)))), st, "c4 state")
    for b in (0, 63):
        r = w.rows[b]
        assert torch.equal(got[b], S.process(w.logits[b].float(), S.RowProcs(repetition=r.repetition, gen=r.gen), []))


def test_state_rows_dense_blocks_masks_nan(sampler):
    """The in-place state form on blocks with more entries than a workgroup has threads (second load round) and more
    than the patches hold (the resolver rebuilds such a block), prompt-only tokens, a banned mask over touched
    tokens and NaN logits, in 512-thread workgroups (12 rows x 31 blocks)."""
    g = torch.Generator().manual_seed(21)
    B = 12
    logits = torch.randn(B, V, generator=g) * 1.5
    logits[:, 8192 + torch.randint(0, 8192, (50,), generator=g)] = float("nan")
    rows = []
    for b in range(B):
        dense = torch.randint(8192, 8192 + 8192, (600 + 150 * b,), generator=g).tolist()  # block 1: 600 .. 2,250 draws
        spread = torch.randint(0, V, (700,), generator=g).tolist()
        prompt = torch.randint(16384, 24576, (300,), generator=g).tolist()
        banned = None
        if b % 3 == 0:
            bits = np.zeros(V // 32, dtype=np.uint32)
            for t in dense[:40] + prompt[:10]:
                bits[t >> 5] |= np.uint32(1) << np.uint32(t & 31)
            banned = bits
        rows.append(q.RowSpec(temperature=0.9, top_k=0 if b % 2 else 40, top_p=0.9, seed=100 + b, row_key=b, presence=0.3, frequency=0.05,
                              repetition=1.15, prompt=prompt, gen=dense + spread, banned=banned))
    st = q.ProcState(B, V, "cuda")
    for b, r in enumerate(rows):
        st.begin(b, r.prompt, r.gen)
    got = _same(sampler, logits, rows, _as_state(rows, list(range(B))), st, "dense state")
    r = rows[3]
    pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, prompt=r.prompt, gen=r.gen, banned=r.banned)
    assert torch.equal(got[3], S.process(logits[3].float(), pr, []))
