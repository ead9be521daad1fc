"""Read-back and bookkeeping entry points on the GPU, through the C ABI:
  * a ProcState slot expanded to dense counts and prompt flags (qws_state_read, the reference's smk_engine_read what = 3)
    equals the request's history, and after decode steps with qws_batch.advance it equals the history plus the emitted
    tokens (the method of the reference's tests/test_proc_model.py:272,290);
  * qws_draft_pick writes every entry of its q buffer: two picks into one dirty buffer give the oracle's q both times,
    a greedy draft row the point mass at its token;
  * a row without a candidate emits token 0 and takes its step with it, under advance and under qws_finish_rows alike;
  * qws_finish_forced follows the reference's SS_FORCE schedule (engine/src/mtp_sample.h:68-70) on a host model;
  * qws_timing_read_verify times qws_verify's own kernels (the reference's smk_spec_launch which = 4)."""
import ctypes as C

import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from qwen_warp_amd import _lib
from qwen_warp_amd._lib import Row
from oracle import sampler as S

pytestmark = pytest.mark.gpu


def _dense(V, ids):
    return np.bincount(np.asarray(list(ids), dtype=np.int64), minlength=V).astype(np.int64) if len(ids) else np.zeros(V, np.int64)


def test_state_read_equals_history_and_emitted_tokens():
    V, B, steps = 65536, 3, 5
    g = torch.Generator().manual_seed(91)
    prompts = [torch.randint(0, V, (40,), generator=g).tolist() for _ in range(B)]
    gens = [torch.randint(0, 64, (30 + 7 * b,), generator=g).tolist() for b in range(B)]  # repeats: counts above 1
    st = q.ProcState(B, V)
    for b in range(B):
        st.begin(b, prompts[b], gens[b])
    for b in range(B):
        c, f = st.read(b)
        assert np.array_equal(c.cpu().numpy().astype(np.int64), _dense(V, gens[b])), b
        assert set(np.nonzero(f.cpu().numpy())[0].tolist()) == set(prompts[b]), b
    rows = [q.RowSpec(temperature=1.0, top_p=0.9, repetition=1.1, presence=0.2, seed=3 + b, position=b, row_key=b, state_slot=b, ngen=len(gens[b]))
            for b in range(B)]
    rows[1].temperature = 0.0  # greedy rows are noted as well
    packed = q.PackedBatch(rows, V, "cuda", st)
    sm = q.Sampler("cuda")
    emitted = [[] for _ in range(B)]
    for s in range(steps):
        lg = (torch.randn(B, V, generator=g) * 2.0).cuda()
        tok = sm.run(packed, lg, advance=True).cpu().tolist()
        for b in range(B):
            emitted[b].append(tok[b])
    for b in range(B):
        c, f = st.read(b)
        assert np.array_equal(c.cpu().numpy().astype(np.int64), _dense(V, gens[b] + emitted[b])), f"slot {b}: counts != history + emitted"
        assert set(np.nonzero(f.cpu().numpy())[0].tolist()) == set(prompts[b])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_draft_pick_into_a_dirty_buffer(dtype):
    """The q buffer is filled with NaN and 7.0 before each of two calls with different rows and logits: every entry is
    rewritten (0 outside the kept set), so q equals the oracle's both times; a greedy draft row's q is the point mass."""
    V, Vd, B = 248320, 64000, 4
    lib = _lib.load()
    g = torch.Generator().manual_seed(93)
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32).cuda()
    qbuf = torch.empty(B, Vd, dtype=torch.float32, device="cuda")
    red = torch.empty(B, dtype=torch.int32, device="cuda")
    ids = torch.empty(B, dtype=torch.int32, device="cuda")
    sm = q.Sampler("cuda")
    ws = sm.workspace(B, Vd)
    for call, fill in enumerate((float("nan"), 7.0)):
        dl = (torch.randn(B, Vd, generator=g) * 2.5).to(dtype)
        cfgs = [dict(temperature=0.7, top_k=20, top_p=0.8), dict(temperature=1.0, top_k=0, top_p=0.95, draft_top_k=50),
                dict(temperature=0.0, top_k=20, top_p=1.0), dict(temperature=0.9, top_k=64, top_p=1.0, draft_sample=0)]
        if call:
            cfgs = cfgs[::-1]
        rows = [q.draft_row(seed=11 + b + 10 * call, j=1 + b, position=call, row_key=b, **cfgs[b]) for b in range(B)]
        qbuf.fill_(fill)
        packed = q.PackedBatch(rows, Vd, "cuda")
        bt = packed.batch(dl.cuda(), red, out_probs=qbuf, row_stride=Vd)
        st = torch.cuda.current_stream().cuda_stream
        _lib.check(lib.qws_draft_pick(C.byref(bt), idmap.data_ptr(), ids.data_ptr(), ws.data_ptr(), ws.numel(), C.c_void_p(st)), "draft_pick")
        qp = qbuf.cpu()
        assert bool(torch.isfinite(qp).all()), f"call {call}: entries left unwritten"
        for b, r in enumerate(rows):
            want = S.sample_row(dl[b], r.temperature, r.top_k, r.top_p, 0.0, r.seed, r.position, r.stream, r.row_key)
            assert int(red[b]) == want.token, (call, b)
            got = torch.nonzero(qp[b]).flatten().numpy()
            if want.greedy:
                assert got.tolist() == [want.token] and float(qp[b, want.token]) == 1.0, (call, b)
                continue
            w = np.array([float(v) for v in want.weights])
            ref_ids = np.sort(np.asarray(want.kept)[w > 0])
            assert np.array_equal(got, ref_ids), (call, b)
            ref_p = np.zeros(Vd)
            ref_p[np.asarray(want.kept)] = w / float(want.S2)
            assert np.max(np.abs(qp[b, got].double().numpy() - ref_p[got]) / ref_p[got]) < 1e-5, (call, b)


def test_row_without_candidate_takes_its_step():
    """Every logit -inf (or masked): token 0 is emitted, noted in the slot and the row advanced, by qws_batch.advance and
    by qws_finish_rows over the same output alike; the other rows are unaffected."""
    V, B = 16384, 3
    g = torch.Generator().manual_seed(95)
    L = torch.randn(B, V, generator=g)
    L[1] = -float("inf")
    banned = np.full((V + 31) // 32, 0xFFFFFFFF, dtype=np.uint32)
    finals = []
    for form in ("advance", "finish"):
        st = q.ProcState(B, V)
        for b in range(B):
            st.begin(b, [5, 6], [7])
        rows = [q.RowSpec(temperature=1.0, top_p=0.9, repetition=1.1, seed=9, position=10 + b, row_key=b, state_slot=b, ngen=1) for b in range(B)]
        rows[2].banned = banned  # every token masked
        packed = q.PackedBatch(rows, V, "cuda", st)
        sm = q.Sampler("cuda")
        if form == "advance":
            tok = sm.run(packed, L.cuda(), advance=True)
        else:
            tok = sm.run(packed, L.cuda())
            book = q.StepBook(B)
            book.finish(list(range(B)), tok, state=st, rows=packed)
        t = tok.cpu().tolist()
        assert t[1] == 0 and t[2] == 0, t
        got = (Row * B).from_buffer_copy(packed.rows_t.cpu().numpy().tobytes())
        assert [r.position for r in got] == [11, 12, 13] and [r.ngen for r in got] == [2, 2, 2], form
        counts = [st.read(b)[0].cpu().numpy() for b in range(B)]
        assert counts[1][0] == 1 and counts[2][0] == 1 and counts[1][7] == 1, form
        finals.append((t, [c.tolist() for c in counts]))
    assert finals[0] == finals[1]


def test_finish_forced_schedule():
    """qws_finish_forced against a host model of spec_finish with the SS_FORCE rule: cycle c of a sequence keeps
    min(a, f) tokens, f = force[c % n] (f < 1: no limit); ring, position, last token, counters and the rows' ngen take
    the kept count, the histogram the natural one."""
    rng = np.random.default_rng(7)
    N, R, T, steps = 3, 32, 6, 9
    force = [2, 0, 1, 5]
    book = q.StepBook(N, R)
    for s in range(N):
        book.start(s, 10 * s, 100 + s)
    model = [dict(pos=10 * s, last=100 + s, outn=0, cycles=0, hist=[0] * 8, ring=[-1] * R) for s in range(N)]
    rows = q.PackedBatch([q.RowSpec(temperature=1.0, ngen=0) for _ in range(N)], 1024, "cuda")
    ngen = [0] * N
    fdev = torch.tensor(force, dtype=torch.int32, device="cuda")
    for step in range(steps):
        cnt = rng.integers(1, T + 1, size=N).astype(np.int32)
        toks = rng.integers(0, 1000, size=(N, T)).astype(np.int32)
        book.finish(list(range(N)), torch.from_numpy(toks).cuda(), torch.from_numpy(cnt).cuda(), rows=rows, force=fdev)
        for s in range(N):
            m = model[s]
            a_nat = int(cnt[s])
            f = force[m["cycles"] % len(force)]
            a = f if 1 <= f < a_nat else a_nat
            for i in range(a):
                m["ring"][(m["outn"] + i) % R] = int(toks[s, i])
            m.update(outn=m["outn"] + a, pos=m["pos"] + a, last=int(toks[s, a - 1]), cycles=m["cycles"] + 1)
            m["hist"][min(a_nat - 1, 7)] += 1
            ngen[s] += a
    rings = book.rings.cpu().numpy()
    for s in range(N):
        assert book.read(s) == {k: model[s][k] for k in ("pos", "last", "outn", "cycles", "hist")}, s
        assert rings[s].tolist() == model[s]["ring"], s
    got = (Row * N).from_buffer_copy(rows.rows_t.cpu().numpy().tobytes())
    assert [r.ngen for r in got] == ngen and [r.position for r in got] == [steps] * N


def test_verify_kernels_are_timed():
    from qwen_warp_amd import workloads
    lib = _lib.load()
    w = workloads.c3()
    x = w.extra
    sm = q.Sampler("cuda")
    tl, dp = w.logits.cuda(), x["draft_probs"].cuda()
    inv = sm.verify_map(x["idmap"].cuda(), tl.shape[-1])
    drafts = x["drafts"].cuda()
    sm.verify(tl, dp, inv, drafts, w.rows)  # warm-up, untimed
    _lib.check(lib.qws_timing(1), "timing")
    try:
        for _ in range(3):
            sm.verify(tl, dp, inv, drafts, w.rows)
        a, d, n = C.c_float(), C.c_float(), C.c_int()
        _lib.check(lib.qws_timing_read_verify(C.byref(a), C.byref(d), C.byref(n)), "timing_read_verify")
        s0, s1, n0 = C.c_float(), C.c_float(), C.c_int()
        _lib.check(lib.qws_timing_read(C.byref(s0), C.byref(s1), C.byref(n0)), "timing_read")
    finally:
        lib.qws_timing(0)
    assert n.value == 3 and a.value > 0 and d.value > 0
    assert n0.value == 3 and s0.value > 0 and s1.value > 0  # the target rows' sampling kernels
