"""GPU speculative verify (qws_verify through the C ABI) against the CPU oracle's verify_seq: emitted tokens and
counts bit-exact per sequence; the emitted distribution equals the target's (chi-square), and the broken-residual
control (test flag bit 0, the reference's SampP.flags bit0) must fail that test."""
import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from qwen_warp_amd import workloads
from oracle import sampler as S
from _util import chi_square

pytestmark = pytest.mark.gpu


def procs_of(r: q.RowSpec):
    if not r.procs_on():
        return None
    return S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=r.prompt, gen=r.gen,
                      ngen=r.ngen, bias=r.bias, allowed=r.allowed, banned=r.banned, stop=r.stop)


def run_verify(sm, tl, dp, idmap, drafts, seqs):
    tl_d, dp_d = tl.cuda().contiguous(), dp.cuda().contiguous()
    inv = sm.verify_map(idmap.to(torch.int32).cuda(), tl.shape[2])
    out, n = sm.verify(tl_d, dp_d, inv, drafts.to(torch.int32).cuda().contiguous(), seqs)
    return out.cpu(), n.cpu(), inv.cpu()


def check_against_oracle(sm, tl, dp, idmap, drafts, seqs, label, bs=None):
    out, n, _ = run_verify(sm, tl, dp, idmap, drafts, seqs)
    K = drafts.shape[1]
    stats = {"accepted": 0, "sequences": 0}
    for b in (range(len(seqs)) if bs is None else bs):
        r = seqs[b]
        want = S.verify_seq(tl[b], dp[b], idmap.numpy(), drafts[b].tolist(), temperature=r.temperature, top_k=r.top_k, top_p=r.top_p,
                            min_p=r.min_p, seed=r.seed, position=r.position, row_key=r.row_key, procs=procs_of(r), test_flags=r.test_flags)
        got = out[b, : int(n[b])].tolist()
        assert int(n[b]) == want.accepted and got == want.tokens, f"{label} seq {b}: GPU {got} (n={int(n[b])}) != oracle {want.tokens}"
        assert out[b, int(n[b]):].tolist() == [-1] * (K + 1 - int(n[b]))
        stats["accepted"] += want.accepted - 1
        stats["sequences"] += 1
    return stats


def test_verify_map_inverse():
    sm = q.Sampler("cuda")
    V = 4096
    idmap = torch.tensor([5, 17, 4095, 0, 17, 9999, -3], dtype=torch.int32)  # 17 twice: the larger index wins
    inv = sm.verify_map(idmap.cuda(), V).cpu()
    want = torch.full((V,), -1, dtype=torch.int32)
    want[5], want[17], want[4095], want[0] = 0, 4, 2, 3
    assert torch.equal(inv, want)


@pytest.mark.parametrize("aligned", [False, True])
def test_verify_c3_parity(aligned):
    """B=4, K=8, fp32 [4][9][248,320], draft vocabulary 64,000 (and a drafter aligned with the
    target, which gets drafts accepted)."""
    w = workloads.c3(aligned=aligned)
    sm = q.Sampler("cuda")
    x = w.extra
    st = check_against_oracle(sm, w.logits, x["draft_probs"], x["idmap"], x["drafts"], w.rows, "c3")
    print(f"c3: {st['accepted']} drafts accepted over {st['sequences']} sequences")


def _case(seed, B, K, V, Vd, dtype=torch.float32, agree=1.0, noise=1.0, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    tl = torch.randn(B, K + 1, V, generator=g) * scale
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32)
    dl = tl[:, :K, :][:, :, idmap.long()] * agree + torch.randn(B, K, Vd, generator=g) * noise
    dp = torch.softmax(dl, dim=2).float()
    j = torch.multinomial(dp.reshape(B * K, Vd).double(), 1, generator=g).reshape(B, K)
    drafts = idmap[j].to(torch.int32)
    return tl.to(dtype), dp, idmap, drafts, g


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_processors_and_params(dtype):
    """Repetition / presence / frequency over a history that the drafts extend, top-k / min-p / top-p, per sequence."""
    B, K, V, Vd = 24, 4, 4096, 3000
    tl, dp, idmap, drafts, g = _case(11 if dtype == torch.float32 else 12, B, K, V, Vd, dtype)
    seqs = []
    for b in range(B):
        hist = torch.randint(0, V, (64,), generator=g).tolist() + drafts[b, :2].tolist()  # repeats of the drafts
        seqs.append(q.RowSpec(temperature=[1.0, 0.7, 1.3][b % 3], top_k=[0, 50, 7][b % 3], top_p=[0.95, 0.8, 1.0][b % 3],
                              min_p=[0.0, 0.05, 0.0][(b // 3) % 3], repetition=1.2, presence=0.4, frequency=0.3, gen=hist,
                              prompt=[int(drafts[b, 0])], seed=100 + b, row_key=b, position=3 * b))
    check_against_oracle(q.Sampler("cuda"), tl, dp, idmap, drafts, seqs, f"procs {dtype}")


def test_verify_all_accepted_and_greedy():
    """A drafter equal to the target (q = p on the table, the table covers the vocabulary) accepts every draft and
    draws the bonus from row K; greedy rows accept exactly the argmax."""
    B, K, V = 16, 6, 2048
    g = torch.Generator().manual_seed(5)
    tl = torch.randn(B, K + 1, V, generator=g) * 2.0
    idmap = torch.arange(V, dtype=torch.int32)
    seqs, dps, drs = [], [], []
    for b in range(B):
        greedy = b % 4 == 3
        r = q.RowSpec(temperature=0.0 if greedy else 1.0, top_p=0.9, seed=7 + b, row_key=b, position=b)
        seqs.append(r)
        dpb, db = [], []
        for t in range(K):
            x = S.process(tl[b, t], None, db)
            if greedy:
                p = torch.zeros(V)
                p[S.greedy(x)] = 1.0
                tok = S.greedy(x)
            else:
                ids, ws, S2 = S.distribution(x, 1.0, 0, 0.9, 0.0)
                p = torch.zeros(V, dtype=torch.float64)
                p[torch.from_numpy(ids)] = torch.tensor([w / S2 for w in ws], dtype=torch.float64)
                tok = int(torch.multinomial(p, 1, generator=g))
                p = p.float()
            dpb.append(p)
            db.append(tok)
        dps.append(torch.stack(dpb))
        drs.append(db)
    dp, drafts = torch.stack(dps), torch.tensor(drs, dtype=torch.int32)
    st = check_against_oracle(q.Sampler("cuda"), tl, dp, idmap, drafts, seqs, "agree")
    assert st["accepted"] >= B * K // 2


def test_verify_edge_drafts():
    """Drafts outside the table (q = 0), masked drafts (p = 0), drafts outside the kept set, a row without candidates,
    K = 15 and the broken-residual flag."""
    B, K, V, Vd = 12, 15, 1024, 700
    tl, dp, idmap, drafts, g = _case(9, B, K, V, Vd, scale=1.0)
    inside = set(idmap.tolist())
    outside = [i for i in range(V) if i not in inside]
    drafts[0, 0] = outside[0]
    drafts[1, :] = torch.tensor(outside[:K], dtype=torch.int32)
    seqs = []
    for b in range(B):
        r = q.RowSpec(temperature=1.0, top_k=[0, 5][b % 2], top_p=0.9, seed=50 + b, row_key=b, position=1, test_flags=1 if b >= 9 else 0)
        if b == 2:  # the drafts are banned: p(d) = 0
            m = np.zeros(V // 32, np.uint32)
            for d in drafts[b].tolist():
                m[d >> 5] |= np.uint32(1) << np.uint32(d & 31)
            r.banned = m
        if b == 3:  # a single allowed id: p is a point mass
            r.allowed = [int(drafts[b, 0])]
        if b == 4:  # every token banned: no candidate, the sequence ends with token 0
            r.banned = np.full(V // 32, 0xFFFFFFFF, np.uint32)
        seqs.append(r)
    check_against_oracle(q.Sampler("cuda"), tl, dp, idmap, drafts, seqs, "edges")


def _first_token_stats(flags, trials=40000, seed=31):
    V, Vd, K = 64, 48, 1
    g = torch.Generator().manual_seed(seed)
    tl1 = torch.randn(K + 1, V, generator=g) * 1.5
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32)
    q1 = torch.softmax(tl1[:K, idmap.long()] + torch.randn(K, Vd, generator=g) * 0.8, dim=1).float()
    rng = np.random.default_rng(seed)
    qd = q1[0].double().numpy()
    drafts = torch.from_numpy(idmap.numpy()[rng.choice(Vd, size=trials, p=qd / qd.sum())].reshape(trials, K).astype(np.int32))
    tl = tl1.unsqueeze(0).expand(trials, K + 1, V).contiguous()
    dp = q1.unsqueeze(0).expand(trials, K, Vd).contiguous()
    seqs = [q.RowSpec(temperature=1.0, top_p=0.95, seed=seed, row_key=b, position=0, test_flags=flags) for b in range(trials)]
    sm = q.Sampler("cuda")
    out, n, _ = run_verify(sm, tl, dp, idmap, drafts, seqs)
    ids, ws, S2 = S.distribution(tl1[0], 1.0, 0, 0.95, 0.0)
    p0 = np.zeros(V)
    p0[ids] = np.array(ws, dtype=np.float64) / S2
    counts = np.bincount(out[:, 0].numpy(), minlength=V)
    sub = list(range(0, trials, 997))
    check_against_oracle(sm, tl[sub], dp[sub], idmap, drafts[sub], [seqs[i] for i in sub], f"stats flags={flags}")
    return chi_square(counts, p0, trials)


def test_verify_preserves_target_distribution():
    _, _, p = _first_token_stats(0)
    assert p > 1e-3, f"verified first tokens do not follow the target distribution (p = {p})"
    _, _, pb = _first_token_stats(1)
    assert pb < 1e-6, f"the broken-residual control passed the chi-square test (p = {pb})"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_narrow_workgroups(dtype):
    """Launch shapes past one workgroup per CU: 10 sequences x 31 blocks at V = 248,320 run k_vres in 512-thread
    workgroups, and 300 sequences run k_vfin in 512-thread workgroups as well; processors count the drafts."""
    sm = q.Sampler("cuda")
    for B, K, V, Vd, seed in ((10, 3, 248320, 20000, 41), (300, 2, 1024, 600, 42)):
        tl, dp, idmap, drafts, g = _case(seed if dtype == torch.float32 else seed + 100, B, K, V, Vd, dtype, noise=0.5)
        seqs = []
        for b in range(B):
            hist = torch.randint(0, V, (200,), generator=g).tolist() + drafts[b, :1].tolist()
            seqs.append(q.RowSpec(temperature=[1.0, 0.8][b % 2], top_k=[0, 40][(b // 2) % 2], top_p=[0.95, 0.9][b % 2], repetition=1.15,
                                  presence=0.3, frequency=0.2, gen=hist, seed=900 + b, row_key=b, position=b))
        bs = None if B <= 10 else list(range(0, B, 7))
        check_against_oracle(sm, tl, dp, idmap, drafts, seqs, f"narrow B={B} {dtype}", bs=bs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_chunk_and_block_rescans_agree(dtype):
    """The residual draw's two forms give the same tokens: 4 sequences at V = 248,320 (4 x 31 blocks fit one workgroup
    per CU: k_vres records chunk prefixes and k_vfin rescans one chunk of the drawn block) and the same 4 sequences as
    the first of 12 (372 workgroups: 512-thread k_vres and the whole-block rescan).  Processors count the drafts."""
    sm = q.Sampler("cuda")
    B, K, V, Vd = 12, 3, 248320, 30000
    tl, dp, idmap, drafts, g = _case(61 if dtype == torch.float32 else 62, B, K, V, Vd, dtype, noise=0.7)
    seqs = []
    for b in range(B):
        hist = torch.randint(0, V, (100,), generator=g).tolist()
        seqs.append(q.RowSpec(temperature=[1.0, 0.8, 1.2][b % 3], top_k=[0, 0, 500][b % 3], top_p=[0.95, 0.9, 1.0][b % 3],
                              repetition=[1.0, 1.1][b % 2], presence=[0.0, 0.2][b % 2], gen=hist, seed=700 + b, row_key=b, position=b))
    out_all, n_all, _ = run_verify(sm, tl, dp, idmap, drafts, seqs)
    out4, n4, _ = run_verify(sm, tl[:4], dp[:4], idmap, drafts[:4], seqs[:4])
    assert n4.tolist() == n_all[:4].tolist() and out4.tolist() == out_all[:4].tolist(), (out4.tolist(), out_all[:4].tolist())
    assert int((n_all[:4] <= K).sum()) > 0, "no sequence ended in a residual draw"  # the draws compared include residuals


def test_verify_zero_residual_and_bonus():
    """q = 1 on every table id (q_fix = S2 at each: the residual max(0, w - S2) is 0 everywhere), so a rejected draft
    falls back to the row's own draw from p; drafts that the target surely accepts (q = 0 at them) reach the bonus row;
    and the broken-residual control draws from p too.  Those draws from p are taken by the verify kernels for rows that
    the resolver left at S2 (more than 64 candidates) and by the resolver itself for rows of at most 64 (top-k 20)."""
    B, K, V, Vd = 12, 3, 24584, 24584
    g = torch.Generator().manual_seed(77)
    tl = torch.randn(B, K + 1, V, generator=g) * 2.0
    idmap = torch.arange(V, dtype=torch.int32)
    dp = torch.ones(B, K, Vd)
    drafts = torch.randint(0, V, (B, K), generator=g, dtype=torch.int32)
    seqs = []
    for b in range(B):
        if b % 3 == 1:  # every draft accepted: q = 0 at the draft, which the target keeps (its argmax)
            for t in range(K):
                d = int(torch.argmax(tl[b, t]))
                drafts[b, t] = d
                dp[b, t, d] = 0.0
        seqs.append(q.RowSpec(temperature=[1.0, 0.7][b % 2], top_k=[0, 20, 0, 0][b % 4], top_p=[0.95, 1.0, 0.8][b % 3], seed=300 + b,
                              row_key=b, position=b, test_flags=1 if b % 6 == 5 else 0))
    check_against_oracle(q.Sampler("cuda"), tl, dp, idmap, drafts, seqs, "zero residual / bonus")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_lower_clamp(dtype):
    """Targets at the lower clamp of x * K (temperatures 1e-20 / 1e-12 over negative logits): every finite token ties
    at t = -2^30 with -inf (masked tokens, the padding past V = 1,000), so the target is uniform over its finite tokens
    and the residual draws after a rejection must weigh those alone."""
    B, K, V, Vd = 12, 3, 1000, 1000
    tl, dp, idmap, drafts, g = _case(61 if dtype == torch.float32 else 62, B, K, V, Vd, dtype)
    tl = -(tl.float().abs() + 0.5)
    seqs = []
    for b in range(B):
        allowed = torch.randperm(V, generator=g)[: [3, 40, 300][b % 3]].tolist() if b % 4 != 3 else None
        if allowed:  # drafts inside the allowed set half the time, so that some are accepted and some rejected
            for t in range(0, K, 2):
                drafts[b, t] = allowed[t % len(allowed)]
        seqs.append(q.RowSpec(temperature=[1e-20, 1e-12][b % 2], top_k=[0, 2, 0][b % 3], top_p=[1.0, 1.0, 0.6][b % 3], allowed=allowed,
                              seed=70 + b, row_key=b, position=b))
    check_against_oracle(q.Sampler("cuda"), tl.to(dtype), dp, idmap, drafts, seqs, f"lower clamp {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_row_distributions(dtype):
    """The verify rows' distributions and processed logits (target out_probs / out_logits, the reference's read-back
    smk_spec_read what = 2): row t of a sequence, with d_1..d_t counted as generated, equals the oracle's processed row
    and its distribution (survivor set exact, probabilities within 1e-5 relative); a greedy sequence's rows are the
    point mass at the argmax; buffers that start dirty are written whole; the emitted tokens are verify_seq's."""
    B, K, V, Vd = 6, 3, 4096, 3000
    tl, dp, idmap, drafts, g = _case(21 if dtype == torch.float32 else 22, B, K, V, Vd, dtype)
    seqs = []
    for b in range(B):
        hist = torch.randint(0, V, (40,), generator=g).tolist() + drafts[b, :1].tolist()
        seqs.append(q.RowSpec(temperature=[1.0, 0.7, 0.0][b % 3], top_k=[0, 50, 0][b % 3], top_p=[0.9, 1.0, 1.0][b % 3],
                              min_p=[0.0, 0.05][b % 2], repetition=1.2, presence=0.3, gen=hist, seed=50 + b, row_key=b, position=b))
    sm = q.Sampler("cuda")
    inv = sm.verify_map(idmap.to(torch.int32).cuda(), V)
    probs = torch.full((B, K + 1, V), 7.0, device="cuda")
    lg = torch.full((B, K + 1, V), 7.0, device="cuda")
    out, n = sm.verify(tl.cuda().contiguous(), dp.cuda().contiguous(), inv, drafts.to(torch.int32).cuda().contiguous(), seqs,
                       out_probs=probs, out_logits=lg)
    probs, lg, out, n = probs.cpu(), lg.cpu(), out.cpu(), n.cpu()
    for b, r in enumerate(seqs):
        for t in range(K + 1):
            x = S.process(tl[b, t], procs_of(r), drafts[b, :t].tolist())
            assert torch.equal(lg[b, t], x + 0.0), f"{dtype} seq {b} row {t}: processed logits differ"
            p = probs[b, t]
            if r.temperature == 0.0:
                want = torch.zeros(V)
                want[S.greedy(x)] = 1.0
                assert torch.equal(p, want), f"{dtype} seq {b} row {t}: greedy point mass"
                continue
            ids, ws, S2 = S.distribution(x, r.temperature, r.top_k, r.top_p, r.min_p)
            w = np.array([float(v) for v in ws], dtype=np.float64)
            keep = w > 0
            ref_ids = np.asarray(ids)[keep]
            o = np.argsort(ref_ids)
            ref_ids, ref_p = ref_ids[o], (w[keep] / float(S2))[o]
            got_ids = torch.nonzero(p).flatten().numpy()
            assert np.array_equal(got_ids, ref_ids), f"{dtype} seq {b} row {t}: survivor sets differ ({len(got_ids)} vs {len(ref_ids)})"
            err = float(np.max(np.abs(p[got_ids].double().numpy() - ref_p) / ref_p))
            assert err < 1e-5, f"{dtype} seq {b} row {t}: probability rel err {err}"
        want = S.verify_seq(tl[b], dp[b], idmap.numpy(), drafts[b].tolist(), temperature=r.temperature, top_k=r.top_k, top_p=r.top_p,
                            min_p=r.min_p, seed=r.seed, position=r.position, row_key=r.row_key, procs=procs_of(r))
        assert out[b, : int(n[b])].tolist() == want.tokens, f"{dtype} seq {b}: tokens"
