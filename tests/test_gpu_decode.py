"""Decode steps that advance on the device (qws_finish_rows): each step samples B rows whose penalties come from a
ProcState slot, then one finish launch notes the emitted tokens into the state and advances every row's Philox
counter word 0 (+1 per cycle, the reference's ss[SS_NCYC]) and ngen (+a).  Six eager steps equal the oracle's
autoregressive decode; the same step captured once in a HIP graph and replayed six times (fresh logits copied in by
eager work between replays) emits the same tokens.  The same decode with qws_batch.advance instead of the finish
launch: the sampling call takes the step itself."""
import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from oracle import sampler as S

pytestmark = pytest.mark.gpu

V, B, STEPS = 65536, 4, 6


def _setup(g):
    prompts = [torch.randint(0, V, (30,), generator=g).tolist() for _ in range(B)]
    gens = [torch.randint(0, V, (20 + 5 * b,), generator=g).tolist() for b in range(B)]
    pos0 = [100 * b + 3 for b in range(B)]
    rows = [q.RowSpec(temperature=[0.9, 1.0, 0.7, 1.2][b], top_k=[0, 50, 0, 20][b], top_p=[0.9, 1.0, 0.8, 0.95][b], min_p=[0.0, 0.0, 0.02, 0.0][b],
                      presence=0.5, frequency=0.3, repetition=1.2, min_tokens=len(gens[b]) + 2, stop=[11, 12], seed=500 + b,
                      position=pos0[b], row_key=b, state_slot=b, ngen=len(gens[b])) for b in range(B)]
    return prompts, gens, pos0, rows


def _fresh(prompts, gens, rows):
    state = q.ProcState(B, V)
    for b in range(B):
        state.begin(b, prompts[b], gens[b])
    packed = q.PackedBatch(rows, V, "cuda", state)
    book = q.StepBook(B)
    for b in range(B):
        book.start(b, 0, -1)
    return state, packed, book


def test_decode_steps_advance_on_device_and_replay_from_a_graph():
    g = torch.Generator().manual_seed(81)
    L = torch.randn(STEPS, B, V, generator=g) * 2.5
    L[:, :, 11] = 9.0  # stop ids: masked while min_tokens is unmet (the first two steps), likely afterwards
    prompts, gens, pos0, rows = _setup(g)
    sm = q.Sampler("cuda")
    rs = torch.arange(B, dtype=torch.int32, device="cuda")
    lg = torch.empty(B, V, dtype=torch.float32, device="cuda")
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    sm.workspace(B, V)
    # eager steps
    state, packed, book = _fresh(prompts, gens, rows)
    eager = []
    for s in range(STEPS):
        lg.copy_(L[s])
        sm.run(packed, lg, out_tokens=tok)
        book.finish(rs, tok, state=state, rows=packed)
        eager.append(tok.cpu().tolist())
    torch.cuda.synchronize()
    # the oracle's autoregressive decode: step s at counter pos0 + s with the tokens emitted so far as history
    for b, r in enumerate(rows):
        hist = list(gens[b])
        for s in range(STEPS):
            pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=prompts[b],
                            gen=hist, stop=r.stop)
            want = S.sample_row(L[s, b], r.temperature, r.top_k, r.top_p, r.min_p, r.seed, pos0[b] + s, r.stream, r.row_key, pr).token
            assert eager[s][b] == want, f"row {b} step {s}: GPU {eager[s][b]} != oracle {want}"
            hist.append(want)
    assert book.read(0)["cycles"] == STEPS
    # one captured step, replayed
    state, packed, book = _fresh(prompts, gens, rows)
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            sm.run(packed, lg, out_tokens=tok)
            book.finish(rs, tok, state=state, rows=packed)
    torch.cuda.synchronize()
    for s in range(STEPS):
        lg.copy_(L[s])
        tok.fill_(-3)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert tok.cpu().tolist() == eager[s], f"replay {s}: {tok.cpu().tolist()} != {eager[s]}"
    assert book.read(1)["cycles"] == STEPS and book.read(1)["outn"] == STEPS


def test_sample_advance_takes_the_step_on_the_device():
    """qws_batch.advance: the sampling call itself notes each drawn token in the row's slot and increments the row's
    ngen and position, so consecutive calls (no finish launch) equal the oracle's autoregressive decode, a greedy row
    included; the same call captured once in a HIP graph replays to the same tokens."""
    g = torch.Generator().manual_seed(82)
    L = torch.randn(STEPS, B, V, generator=g) * 2.5
    L[:, :, 11] = 9.0
    prompts, gens, pos0, rows = _setup(g)
    rows[2].temperature = 0.0  # greedy: noted and advanced as well
    sm = q.Sampler("cuda")
    lg = torch.empty(B, V, dtype=torch.float32, device="cuda")
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    sm.workspace(B, V)
    state, packed, _ = _fresh(prompts, gens, rows)
    eager = []
    for s in range(STEPS):
        lg.copy_(L[s])
        sm.run(packed, lg, out_tokens=tok, advance=True)
        eager.append(tok.cpu().tolist())
    for b, r in enumerate(rows):
        hist = list(gens[b])
        for s in range(STEPS):
            pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=prompts[b],
                            gen=hist, stop=r.stop)
            want = S.sample_row(L[s, b], r.temperature, r.top_k, r.top_p, r.min_p, r.seed, pos0[b] + s, r.stream, r.row_key, pr).token
            assert eager[s][b] == want, f"row {b} step {s}: GPU {eager[s][b]} != oracle {want}"
            hist.append(want)
    from qwen_warp_amd._lib import Row
    got = (Row * B).from_buffer_copy(packed.rows_t.cpu().numpy().tobytes())
    assert [r.position for r in got] == [p + STEPS for p in pos0]
    assert [r.ngen for r in got] == [len(gens[b]) + STEPS for b in range(B)]
    # one captured call, replayed
    state, packed, _ = _fresh(prompts, gens, rows)
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            sm.run(packed, lg, out_tokens=tok, advance=True)
    torch.cuda.synchronize()
    for s in range(STEPS):
        lg.copy_(L[s])
        tok.fill_(-3)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert tok.cpu().tolist() == eager[s], f"replay {s}: {tok.cpu().tolist()} != {eager[s]}"
    with pytest.raises(q.ValidationError):
        rows2 = [q.RowSpec(temperature=1.0, presence=0.1, state_slot=0) for _ in range(2)]
        q.PackedBatch(rows2, V, "cuda", q.ProcState(1, V)).batch(lg[:2], tok[:2], advance=True)


def test_sample_advance_at_benchmark_shape():
    """The C4 rows as the benchmark's decode loop: slots built from their 4,096-token histories, three calls with advance
    on the rotated benchmark logits; all 64 rows at every step against the oracle's autoregressive decode, and each
    slot's counts read back afterwards equal to its history plus the three emitted tokens."""
    from qwen_warp_amd import workloads
    w = workloads.c4()
    Vf = w.logits.shape[1]
    state = q.ProcState(len(w.rows), Vf)
    rows = []
    for b, r in enumerate(w.rows):
        state.begin(b, r.prompt, r.gen)
        d = {k: getattr(r, k) for k in q.RowSpec.__dataclass_fields__}
        d.update(prompt=[], gen=[], state_slot=b, ngen=len(r.gen))
        rows.append(q.RowSpec(**d))
    packed = q.PackedBatch(rows, Vf, "cuda", state)
    sm = q.Sampler("cuda")
    lg = w.logits.cuda()
    toks = []
    for s in range(3):
        toks.append(sm.run(packed, torch.roll(lg, s, dims=0).contiguous(), advance=True).cpu().tolist())
    for b in range(len(w.rows)):
        r = w.rows[b]
        hist = list(r.gen)
        for s in range(3):
            x = torch.roll(w.logits, s, dims=0)[b]
            want = S.sample_row(x, r.temperature, r.top_k, r.top_p, r.min_p, r.seed, r.position + s, r.stream, r.row_key,
                                S.RowProcs(repetition=r.repetition, gen=hist)).token
            assert toks[s][b] == want, f"row {b} step {s}: GPU {toks[s][b]} != oracle {want}"
            hist.append(want)
        if b % 16 == 0:  # the slot read back (a few rows: each read is a V-sized copy)
            c = state.read(b)[0].cpu().numpy().astype(np.int64)
            assert np.array_equal(c, np.bincount(np.asarray(hist), minlength=Vf)), f"slot {b}: counts != history + emitted"
