"""The drafter's picks and delta proposals on the GPU, through the C ABI: qws_draft_pick (q and the drawn id of the
drafter's rows, make_sampp's draft parameters) bit-exact against the CPU oracle; qws_verify with prompt-lookup tail
tokens (n_chain: q = 1 at the draft) bit-exact against verify_seq; and the joint distribution of the emitted tokens of
whole speculative cycles (drafts picked on the GPU, tails fixed, penalties counting the drafts) against the exact
autoregressive joint, with the broken-residual and ignored-drafts controls required to fail (the method of the
reference's tests/test_spec_procs.py:76-144, its third scenario :163-164)."""
import itertools

import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from oracle import sampler as S
from _util import chi_square

pytestmark = pytest.mark.gpu


def _draft_case(seed, B, Vd, V):
    g = torch.Generator().manual_seed(seed)
    dl = torch.randn(B, Vd, generator=g) * 2.5
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32)
    return dl, idmap


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_draft_pick_parity(dtype):
    """Draft rows with and without draft_sample, the draft temperature / top-k / top-p and the target's as fallbacks:
    drawn reduced index and target id, and q over the reduced vocabulary, against the oracle's distribution."""
    V, Vd = 248320, 64000
    cfgs = [dict(temperature=0.7, top_k=20, top_p=0.8), dict(temperature=0.7, top_k=20, top_p=0.8, draft_sample=0),
            dict(temperature=1.0, top_k=0, top_p=0.95, draft_temperature=0.6, draft_top_k=50, draft_top_p=0.9),
            dict(temperature=1.2, top_k=0, top_p=1.0, draft_top_p=0.7), dict(temperature=0.9, top_k=64, top_p=1.0, draft_top_k=5)]
    B = 2 * len(cfgs)
    dl, idmap = _draft_case(61, B, Vd, V)
    dl = dl.to(dtype)
    rows = [q.draft_row(seed=77 + b, j=1 + b % 3, position=5 * b, row_key=b, **cfgs[b % len(cfgs)]) for b in range(B)]
    sm = q.Sampler("cuda")
    ids, qp, red = sm.draft_pick(dl.cuda(), rows, idmap.cuda())
    ids, qp, red = ids.cpu(), qp.cpu(), red.cpu()
    for b, r in enumerate(rows):
        c = cfgs[b % len(cfgs)]
        t, k, p = S.draft_params(c["temperature"], c["top_k"], c["top_p"], c.get("draft_sample", 1), c.get("draft_temperature", 0.0),
                                 c.get("draft_top_k", 0), c.get("draft_top_p", 0.0))
        assert (r.temperature, r.top_k, r.top_p, r.stream) == (t, k, p, S.ST_DRAFT + 1 + b % 3)
        want = S.sample_row(dl[b], t, k, p, 0.0, r.seed, r.position, r.stream, r.row_key)
        assert int(red[b]) == want.token and int(ids[b]) == int(idmap[want.token]), f"row {b}: {int(red[b])} vs {want.token}"
        got = torch.nonzero(qp[b]).flatten().numpy()
        w = np.array([float(v) for v in want.weights])
        ref_ids = np.sort(np.asarray(want.kept)[w > 0])
        assert np.array_equal(got, ref_ids), f"row {b}: q support differs"
        ref_p = np.zeros(Vd)
        ref_p[np.asarray(want.kept)] = w / float(want.S2)
        err = np.max(np.abs(qp[b, got].double().numpy() - ref_p[got]) / ref_p[got])
        assert err < 1e-5
        if not c.get("draft_sample", 1):
            assert len(got) == 1 and int(red[b]) == S.greedy(S.widen(dl[b]))  # q = the point mass at the argmax


def test_verify_chain_and_tail_parity():
    """Sequences whose last drafts are prompt-lookup tail tokens (n_chain per sequence, tails inside and outside the
    draft table, repeated tails), with processors counting every draft: emitted tokens bit-exact against verify_seq."""
    B, K, V, Vd = 12, 5, 248320, 30000
    g = torch.Generator().manual_seed(71)
    tl = torch.randn(B, K + 1, V, generator=g) * 8.0  # peaked rows: a tail at the row's argmax is likely accepted
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32)
    dlog = tl[:, :K, :][:, :, idmap.long()] + torch.randn(B, K, Vd, generator=g) * 0.5
    dp = torch.softmax(dlog, dim=2).float()
    j = torch.multinomial(dp.reshape(B * K, Vd).double(), 1, generator=g).reshape(B, K)
    drafts = idmap[j].to(torch.int32)
    nchain = torch.tensor([K, 0, 1, 0, 3, 0, 1, 2, 0, 3, 0, 4], dtype=torch.int32)
    for b in range(B):  # tails: mostly the target's argmax of the row (likely accepted), else a repeat or a token outside the table
        for t in range(int(nchain[b]), K):
            kind = 0 if (b + t) % 4 != 3 else 1 + (b % 2)
            drafts[b, t] = int(tl[b, t].argmax()) if kind == 0 else (int(drafts[b, t - 1]) if kind == 1 and t > 0 else 7 + b)
    seqs = []
    for b in range(B):
        hist = torch.randint(0, V, (100,), generator=g).tolist()
        seqs.append(q.RowSpec(temperature=[1.0, 0.8, 1.2][b % 3], top_k=[0, 40][b % 2], top_p=[0.95, 0.9, 1.0][b % 3], repetition=1.2,
                              presence=0.4, frequency=0.3, gen=hist, seed=300 + b, row_key=b, position=11 * b))
    sm = q.Sampler("cuda")
    inv = sm.verify_map(idmap.cuda(), V)
    out, n = sm.verify(tl.cuda(), dp.cuda(), inv, drafts.cuda(), seqs, n_chain=nchain.cuda())
    out, n = out.cpu(), n.cpu()
    acc = 0
    for b, r in enumerate(seqs):
        pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, gen=r.gen)
        want = S.verify_seq(tl[b], dp[b], idmap.numpy(), drafts[b].tolist(), temperature=r.temperature, top_k=r.top_k, top_p=r.top_p,
                            seed=r.seed, position=r.position, row_key=r.row_key, procs=pr, n_chain=int(nchain[b]))
        assert int(n[b]) == want.accepted and out[b, :int(n[b])].tolist() == want.tokens, f"seq {b}: {out[b].tolist()} vs {want.tokens}"
        acc += want.accepted - 1
    assert acc > 0


def _spec_scenario(N, nchain, tail, m, trials, cfg, procs_kw, gen, seed, flags=0, ignore_drafts=False, chunk=20000):
    """Whole speculative cycles per trial on the GPU: chain drafts picked by qws_draft_pick from the drafter's rows
    (position = trial), the fixed tail, then qws_verify with n_chain; emitted tokens completed to m tokens from the
    oracle's exact conditionals; chi-square against the exact autoregressive joint of m tokens."""
    g = torch.Generator().manual_seed(seed)
    k = nchain + len(tail)
    tl = torch.randn(k + 1, N, generator=g) * 1.5
    dl = tl[:nchain] + torch.randn(nchain, N, generator=g) * 0.8
    procs = S.RowProcs(gen=gen, **procs_kw)
    cache = {}

    def cond(h):
        if h not in cache:
            x = S.process(tl[len(h)], procs, list(h))
            ids, ws, S2 = S.distribution(x, cfg["temperature"], cfg["top_k"], cfg["top_p"], cfg.get("min_p", 0.0))
            p = np.zeros(N)
            p[np.asarray(ids)] = np.array(ws, dtype=np.float64) / S2
            cache[h] = p
        return cache[h]

    joint = np.zeros((N,) * m)
    for h in itertools.product(range(N), repeat=m):
        pr = 1.0
        for t in range(m):
            pr *= cond(h[:t])[h[t]]
            if pr == 0.0:
                break
        joint[h] = pr
    sm = q.Sampler("cuda")
    idmap = torch.arange(N, dtype=torch.int32).cuda()
    inv = sm.verify_map(idmap, N)
    rng = np.random.default_rng(seed)
    outs = []
    for c0 in range(0, trials, chunk):
        B = min(chunk, trials - c0)
        dr = torch.empty(B, k, dtype=torch.int32)
        qs = []
        for j in range(1, nchain + 1):
            rows = [q.draft_row(seed=seed, j=j, position=c0 + i, **cfg) for i in range(B)]
            ids, qj, _ = sm.draft_pick(dl[j - 1].cuda().reshape(1, N).expand(B, N), rows, idmap)
            dr[:, j - 1] = ids.cpu()
            qs.append(qj[0].cpu())
        for t, v in enumerate(tail):
            dr[:, nchain + t] = v
        dp = torch.stack(qs + [torch.zeros(N)] * len(tail)).unsqueeze(0).expand(B, k, N).contiguous()
        seqs = [q.RowSpec(temperature=cfg["temperature"], top_k=cfg["top_k"], top_p=cfg["top_p"], seed=seed, position=c0 + i, row_key=0,
                          gen=list(gen), test_flags=flags, **{kk: vv for kk, vv in procs_kw.items()}) for i in range(B)]
        vrows = sm.verify_rows(seqs, dr.tolist())
        if ignore_drafts:  # the broken control: every target row processed as if no draft had been generated
            for vr in vrows:
                vr.drafts = []
        packed = q.PackedBatch(vrows, N, "cuda")
        tlb = tl.unsqueeze(0).expand(B, k + 1, N).contiguous().cuda()
        out, n = sm.verify(tlb, dp.cuda(), inv, dr.cuda(), seqs, packed=packed, n_chain=torch.full((B,), nchain, dtype=torch.int32).cuda())
        outs.append((out.cpu().numpy(), n.cpu().numpy()))
    y = np.concatenate([o for o, _ in outs])
    a = np.concatenate([nn for _, nn in outs])
    full = np.where(np.arange(m)[None, :] < a[:, None], y[:, :m], -1).astype(np.int64)
    for col in range(m):
        groups = {}
        for i in np.nonzero(full[:, col] < 0)[0]:
            groups.setdefault(tuple(full[i, :col]), []).append(i)
        for h, ii in groups.items():
            p = cond(h)
            full[ii, col] = rng.choice(N, size=len(ii), p=p / p.sum())
    counts = np.bincount(np.ravel_multi_index(full.T, (N,) * m), minlength=N ** m)
    stat, dof, pv = chi_square(counts, joint.reshape(-1), trials)
    return pv, float(a.mean())


def test_spec_cycles_joint_with_tails():
    """2 chain drafts + 2 prompt-lookup tail tokens, penalties (presence 1.5, frequency 1.0, repetition 1.4) counting the
    drafts (the reference's third scenario): the joint of 4 emitted tokens matches the autoregressive reference; the
    broken residual and the ignored drafts both fail."""
    N, cfg = 8, dict(temperature=1.0, top_k=0, top_p=1.0)
    pk = dict(prompt=[1, 2], presence=1.5, frequency=1.0, repetition=1.4)
    pv, mean_a = _spec_scenario(N, 2, [3, 3], 4, 60000, cfg, pk, [3, 4], seed=13)
    print(f"engine: p {pv:.3g}, mean emitted {mean_a:.2f}")
    assert pv > 1e-3
    pb, _ = _spec_scenario(N, 2, [3, 3], 4, 60000, cfg, pk, [3, 4], seed=13, flags=1)
    assert pb < 1e-6, f"broken residual passed (p = {pb})"
    pi, _ = _spec_scenario(N, 2, [3, 3], 4, 60000, cfg, pk, [3, 4], seed=13, ignore_drafts=True)
    assert pi < 1e-6, f"ignored drafts passed (p = {pi})"


def test_spec_cycles_joint_three_chain_drafts():
    """3 chain drafts, no tail, top-k 5 and top-p 0.9 over 8 tokens, penalties counting the drafts (presence 1.0,
    repetition 1.3): the joint of 4 emitted tokens matches the autoregressive reference; the broken residual and the
    ignored drafts both fail."""
    N, cfg = 8, dict(temperature=0.9, top_k=5, top_p=0.9)
    pk = dict(prompt=[0], presence=1.0, repetition=1.3)
    pv, mean_a = _spec_scenario(N, 3, [], 4, 60000, cfg, pk, [1], seed=17)
    print(f"engine: p {pv:.3g}, mean emitted {mean_a:.2f}")
    assert pv > 1e-3
    pb, _ = _spec_scenario(N, 3, [], 4, 60000, cfg, pk, [1], seed=17, flags=1)
    assert pb < 1e-6, f"broken residual passed (p = {pb})"
    pi, _ = _spec_scenario(N, 3, [], 4, 60000, cfg, pk, [1], seed=17, ignore_drafts=True)
    assert pi < 1e-6, f"ignored drafts passed (p = {pi})"
