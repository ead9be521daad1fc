"""Seeded random cases through qws_sample against the oracle: vocabularies from one partial block to 49 blocks, batches
that run either k_scan width (fp32 and bf16), flat / peaked / spiky / huge-magnitude / tied logits with NaN and +-inf,
every truncation parameter (extreme temperatures and top-p included) and every processor mixed per row (histories
with repeats, all three penalties, +-100 biases, stop ids while min_tokens holds, banned and allowed masks), and the
test flags that force the resolver's rescans, staged draws and split selections.  Tokens and dense probabilities
(survivor sets exact, probabilities within 1e-5 relative) for every row."""
import math

import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from oracle import sampler as S

pytestmark = pytest.mark.gpu

PROB_RTOL = 1e-5


def _oracle(x, r):
    pr = None
    if r.procs_on():
        pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=r.prompt,
                        gen=r.gen, ngen=r.ngen, bias=r.bias, allowed=r.allowed, banned=r.banned, stop=r.stop)
    return S.sample_row(x, r.temperature, r.top_k, r.top_p, r.min_p, r.seed, r.position, r.stream, r.row_key, pr)


def _case(seed, v=2):
    """Case `seed` of generator version v (1: without the huge / tied logits, extreme parameters and test flags)."""
    rng = np.random.default_rng(seed)
    V = int(rng.choice([8, 64, 1000, 8192, 24576, 65536, 131072, 400000]))
    V = max(8, V // 8 * 8)
    B = int(rng.choice([1, 3, 9, 40])) if V < 65536 else int(rng.choice([1, 6, 40])) if V <= 131072 else int(rng.choice([1, 2, 6]))
    if seed % 4 == 0:  # every fourth case: more workgroups than CUs (the 512-thread scan)
        V = int(rng.choice([65536, 131072, 400000]))
        B = 40 if V <= 131072 else 6
    elif v >= 2 and seed % 7 == 0:  # wide batches, not multiples of the 8 XCDs (rows spread over the resolver's grid)
        V = int(rng.choice([1000, 8192]))
        B = int(rng.choice([65, 97, 130]))
    dtype = torch.bfloat16 if rng.random() < 0.4 else torch.float32
    g = torch.Generator().manual_seed(seed)
    kind = rng.integers(5 if v >= 2 else 3)
    sigma = [0.4, 3.0, 8.0, 3.0, 1.0][kind]
    x = torch.randn(B, V, generator=g) * sigma
    if kind == 2:  # spikes
        n = max(1, V // 500)
        for b in range(B):
            x[b, torch.randint(0, V, (n,), generator=g)] += 15.0
    elif kind == 3:  # huge magnitudes, and a row of equal values
        x *= 1e4
        x[0] = 1.5
    elif kind == 4:  # few distinct values: long runs of ties
        x = torch.round(x * 4) / 4
    if rng.random() < 0.3:
        x[0, torch.randint(0, V, (max(1, V // 100),), generator=g)] = float("nan")
    if rng.random() < 0.2:
        x[B - 1, int(rng.integers(V))] = math.inf
    if rng.random() < 0.2:
        x[0, int(rng.integers(V)):] = -math.inf
    x = x.to(dtype)
    rows = []
    for b in range(B):
        if v >= 2:
            kw = dict(temperature=float(rng.choice([0.0, 1e-20, 0.05, 0.3, 0.7, 1.0, 3.0, 1e4])), top_k=int(rng.choice([0, 0, 1, 5, 50, 1000, V + 5])),
                      top_p=float(rng.choice([1.0, 1.0, 0.9, 0.5, 0.01, 1e-7])), min_p=float(rng.choice([0.0, 0.0, 0.01, 0.3, 1.0])),
                      seed=int(rng.integers(1 << 40)), position=int(rng.integers(1 << 20)), row_key=b,
                      test_flags=int(rng.choice([0, 0, 0, q.TF_RESCAN, q.TF_STAGED_DRAW, q.TF_SPLIT_SELECT, q.TF_RESCAN | q.TF_STAGED_DRAW])))
        else:
            kw = dict(temperature=float(rng.choice([0.0, 0.05, 0.3, 0.7, 1.0, 3.0])), top_k=int(rng.choice([0, 0, 1, 5, 50, 1000, V + 5])),
                      top_p=float(rng.choice([1.0, 1.0, 0.9, 0.5, 0.01])), min_p=float(rng.choice([0.0, 0.0, 0.01, 0.3])),
                      seed=int(rng.integers(1 << 40)), position=int(rng.integers(1 << 20)), row_key=b)
        if rng.random() < 0.7:
            n_hist = int(rng.choice([0, 10, 300, 3000]))
            hist = rng.integers(0, V, n_hist)
            if n_hist:
                hist[: n_hist // 3] = hist[0]  # repeats
            kw.update(gen=hist.tolist(), prompt=rng.integers(0, V, int(rng.choice([0, 5, 50]))).tolist(),
                      repetition=float(rng.choice([1.0, 1.3, 0.8])), presence=float(rng.choice([0.0, 0.5, -1.0])),
                      frequency=float(rng.choice([0.0, 0.3])))
        if rng.random() < 0.5:
            ids = rng.choice(V, size=min(V, int(rng.choice([1, 20, 300]))), replace=False)
            kw["bias"] = {int(i): float(v) for i, v in zip(ids, rng.uniform(-100, 100, ids.size))}
        if rng.random() < 0.3:
            kw.update(stop=rng.choice(V, size=min(V, 3), replace=False).tolist(), min_tokens=int(rng.choice([1, 5])), ngen=int(rng.integers(3)))
        m = rng.random()
        if m < 0.15:
            kw["allowed"] = rng.choice(V, size=max(1, V // 7), replace=False).tolist()
        elif m < 0.3:
            bits = rng.random(V) < 0.05
            w = np.zeros((V + 31) // 32, dtype=np.uint32)
            nz = np.nonzero(bits)[0]
            np.bitwise_or.at(w, nz >> 5, (np.uint32(1) << (nz & 31).astype(np.uint32)))
            kw["banned"] = w
        rows.append(q.RowSpec(**kw))
    return x, rows


# 32 seeds, plus cases that once failed: of the first generator, min-p beside top-k 5 with one block holding more than 5
# candidates above the row's min-p cut (the block's bins stop at its own 5th candidate); of the second, temperature
# 1e-20 over penalised or biased logits at the lower clamp of x * K, where -inf and the padding past V = 8 share the
# best's t = -2^30
@pytest.mark.parametrize("seed,v", [(s, 2) for s in range(32)] + [(s, 1) for s in (166, 182, 221, 321)] + [(s, 2) for s in (51, 187, 223)])
def test_fuzz_rows(seed, v):
    x, rows = _case(1000 + seed, v)
    sm = q.Sampler("cuda")
    tok, probs, info = sm.probs(x.cuda(), rows)
    tok, probs = tok.cpu().tolist(), probs.cpu()
    xf = x.float()
    for b, r in enumerate(rows):
        want = _oracle(xf[b], r)
        label = f"seed {1000 + seed} V={x.shape[1]} B={x.shape[0]} {x.dtype} row {b} ({r.temperature}, {r.top_k}, {r.top_p}, {r.min_p})"
        assert tok[b] == want.token, f"{label}: token {tok[b]} != oracle {want.token}"
        if want.greedy:
            continue
        got = torch.nonzero(probs[b]).flatten().numpy()
        w = np.array([float(v) for v in want.weights], dtype=np.float64)
        keep = w > 0
        ref = np.asarray(want.kept)[keep]
        o = np.argsort(ref)
        ref, ref_p = ref[o], (w[keep] / float(want.S2))[o]
        assert np.array_equal(got, ref), f"{label}: survivor sets differ ({len(got)} vs {len(ref)})"
        if len(ref):
            err = float(np.max(np.abs(probs[b, got].double().numpy() - ref_p) / ref_p))
            assert err < PROB_RTOL, f"{label}: probability rel err {err}"


def _procs(r):
    if not r.procs_on():
        return None
    return S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=r.prompt,
                      gen=r.gen, ngen=r.ngen, bias=r.bias, allowed=r.allowed, banned=r.banned, stop=r.stop)


def _verify_case(seed):
    """A random speculative verify: B sequences of K drafts over V, the drafter's table of Vd ids (duplicates and ids
    outside the vocabulary among them), draft probabilities with zeros, NaN, negatives and values above 1, drafts drawn
    from them or replaced by ids outside the table, masked ids and the target's argmax, prompt-lookup tails (n_chain),
    and the target rows of _case's kinds and parameters (greedy and 1e-20 temperatures, processors, test flags)."""
    rng = np.random.default_rng(seed)
    V = int(rng.choice([8, 64, 1000, 8192, 24584, 65536]))
    K = int(rng.choice([1, 2, 4, 8, 15]))
    B = int(rng.choice([1, 3, 10])) if V <= 8192 else int(rng.choice([1, 3]))
    dtype = torch.bfloat16 if rng.random() < 0.4 else torch.float32
    g = torch.Generator().manual_seed(seed)
    kind = rng.integers(5)
    tl = torch.randn(B, K + 1, V, generator=g) * [0.4, 3.0, 8.0, 3.0, 1.0][kind]
    if kind == 2:
        tl[..., : max(1, V // 500)] += 15.0
    elif kind == 3:
        tl *= 1e4
    elif kind == 4:
        tl = torch.round(tl * 4) / 4
    if rng.random() < 0.3:
        tl[0, :, torch.randint(0, V, (max(1, V // 100),), generator=g)] = float("nan")
    Vd = int(rng.integers(1, V + 1))
    idmap = torch.randperm(V, generator=g)[:Vd].to(torch.int32)
    if rng.random() < 0.3 and Vd >= 3:
        idmap[0], idmap[1], idmap[2] = idmap[Vd - 1], -3, V + 7  # a duplicate (the larger index wins) and two ids outside V
    agree = float(rng.choice([0.0, 1.0]))
    dl = tl.float()[:, :K, :][:, :, idmap.clamp(0, V - 1).long()] * agree + torch.randn(B, K, Vd, generator=g) * float(rng.choice([0.3, 2.0]))
    dp = torch.softmax(torch.nan_to_num(dl, nan=0.0), dim=2)
    drafts = idmap.clamp(0, V - 1)[torch.multinomial(dp.reshape(B * K, Vd), 1, generator=g).reshape(B, K)].to(torch.int32)
    if rng.random() < 0.3:
        dp[0, 0, : max(1, Vd // 3)] = 0.0
    if rng.random() < 0.2:
        dp[B - 1, K - 1, int(rng.integers(Vd))] = float(rng.choice([float("nan"), -0.5, 1.5, 1.0]))
    for b in range(B):
        for t in range(K):
            u = rng.random()
            if u < 0.1:
                drafts[b, t] = int(rng.integers(V))  # any id, inside the table or not
            elif u < 0.15:
                drafts[b, t] = int(torch.argmax(torch.nan_to_num(tl[b, t].float(), nan=-math.inf)))
    x0, rows = _case(seed + 7, 2)  # parameters and processors only (its logits are not used)
    seqs = []
    for b in range(B):
        r = rows[b % len(rows)]
        kw = {k: getattr(r, k) for k in q.RowSpec.__dataclass_fields__ if k not in ("drafts", "draw_word", "stream", "state_slot")}
        kw["row_key"] = b
        kw["test_flags"] = int(rng.choice([0, 0, 0, q.TF_BROKEN, q.TF_RESCAN, q.TF_STAGED_DRAW]))
        V0 = x0.shape[1]
        for name in ("gen", "prompt", "stop", "allowed"):  # ids of _case's vocabulary folded into this one
            if kw.get(name):
                kw[name] = [int(i) % V for i in kw[name]]
        if kw.get("bias"):
            kw["bias"] = {int(i) % V: v for i, v in kw["bias"].items()}
        if kw.get("banned") is not None:
            bits = np.zeros(V, dtype=bool)
            w = np.asarray(kw["banned"], dtype=np.uint32)
            ids = np.nonzero((w[np.arange(V0) >> 5] >> (np.arange(V0) & 31).astype(np.uint32)) & 1)[0] % V
            bits[ids] = True
            mw = np.zeros((V + 31) // 32, dtype=np.uint32)
            nz = np.nonzero(bits)[0]
            np.bitwise_or.at(mw, nz >> 5, (np.uint32(1) << (nz & 31).astype(np.uint32)))
            kw["banned"] = mw
        if kw.get("stop"):
            kw["stop"] = list(dict.fromkeys(kw["stop"]))
        if kw.get("allowed"):
            kw["allowed"] = list(dict.fromkeys(kw["allowed"]))
        kw["top_k"] = min(kw["top_k"], V + 5)
        seqs.append(q.RowSpec(**kw))
    # drafts that the target likely accepts: the processed row's argmax, often with q lowered at it (q <= p accepts)
    tq = tl.to(dtype).float()
    inv = {int(i): j for j, i in enumerate(idmap.tolist())}
    for b in range(B):
        if rng.random() < 0.6:
            for t in range(K):
                if rng.random() < 0.8:
                    d = S.greedy(S.process(tq[b, t], _procs(seqs[b]), drafts[b, :t].tolist()))
                    drafts[b, t] = d
                    if d in inv and rng.random() < 0.6:
                        dp[b, t, inv[d]] = float(rng.choice([0.0, 1e-6]))
    n_chain = None
    if rng.random() < 0.3:
        n_chain = torch.tensor(rng.integers(0, K + 1, B), dtype=torch.int32)
    return tl.to(dtype), dp, idmap, drafts, seqs, n_chain


@pytest.mark.parametrize("seed", range(16))
def test_fuzz_verify(seed):
    tl, dp, idmap, drafts, seqs, n_chain = _verify_case(2000 + seed)
    B, K1, V = tl.shape
    K = K1 - 1
    sm = q.Sampler("cuda")
    inv = sm.verify_map(idmap.cuda(), V)
    out, n = sm.verify(tl.cuda().contiguous(), dp.cuda().contiguous(), inv, drafts.cuda().contiguous(), seqs,
                       n_chain=None if n_chain is None else n_chain.cuda())
    out, n = out.cpu(), n.cpu()
    tf = tl.float()
    for b, r in enumerate(seqs):
        want = S.verify_seq(tf[b], dp[b], idmap.numpy(), drafts[b].tolist(), temperature=r.temperature, top_k=r.top_k, top_p=r.top_p,
                            min_p=r.min_p, seed=r.seed, position=r.position, row_key=r.row_key, procs=_procs(r), test_flags=r.test_flags,
                            n_chain=None if n_chain is None else int(n_chain[b]))
        got = out[b, : int(n[b])].tolist()
        label = f"seed {2000 + seed} V={V} K={K} B={B} {tl.dtype} seq {b} ({r.temperature}, {r.top_k}, {r.top_p}, {r.min_p}, flags {r.test_flags})"
        assert int(n[b]) == want.accepted and got == want.tokens, f"{label}: GPU {got} (n={int(n[b])}) != oracle {want.tokens}"
        assert out[b, int(n[b]):].tolist() == [-1] * (K + 1 - int(n[b])), label


def _decode_case(seed):
    """Random decode loops: rows whose histories sit in ProcState slots, several steps each (the step taken by the
    sampling call itself, qws_batch.advance, or by a finish launch), min_tokens lifting the stop mask during the loop,
    stop ids made likely once allowed, greedy and extreme temperatures, every processor and truncation parameter."""
    rng = np.random.default_rng(seed)
    V = int(rng.choice([8, 64, 1000, 8192, 24584, 65536, 131072]))
    B = int(rng.choice([1, 3, 8, 12])) if V <= 65536 else int(rng.choice([1, 3]))
    steps = int(rng.integers(3, 8))
    dtype = torch.bfloat16 if rng.random() < 0.4 else torch.float32
    g = torch.Generator().manual_seed(seed)
    kind = rng.integers(5)
    L = torch.randn(steps, B, V, generator=g) * [0.4, 3.0, 8.0, 3.0, 1.0][kind]
    if kind == 2:
        L[..., : max(1, V // 500)] += 15.0
    elif kind == 3:
        L *= 1e4
    elif kind == 4:
        L = torch.round(L * 4) / 4
    if rng.random() < 0.3:
        L[:, 0, torch.randint(0, V, (max(1, V // 100),), generator=g)] = float("nan")
    prompts, gens, rows = [], [], []
    for b in range(B):
        prompt = rng.integers(0, V, int(rng.choice([0, 5, 50]))).tolist()
        gen = rng.integers(0, V, int(rng.choice([0, 10, 300])))
        if gen.size:
            gen[: gen.size // 3] = gen[0]
        gen = gen.tolist()
        kw = dict(temperature=float(rng.choice([0.0, 1e-20, 0.3, 0.7, 1.0, 3.0])), top_k=int(rng.choice([0, 0, 1, 5, 50, V + 5])),
                  top_p=float(rng.choice([1.0, 0.9, 0.5, 0.01])), min_p=float(rng.choice([0.0, 0.0, 0.05, 0.3])),
                  seed=int(rng.integers(1 << 40)), position=int(rng.integers(1 << 20)), row_key=b, state_slot=b, ngen=len(gen),
                  repetition=float(rng.choice([1.0, 1.3, 0.8])), presence=float(rng.choice([0.0, 0.5, -1.0])), frequency=float(rng.choice([0.0, 0.3])))
        if rng.random() < 0.5:
            stop = rng.choice(V, size=min(V, 3), replace=False).tolist()
            kw.update(stop=stop, min_tokens=len(gen) + int(rng.choice([0, 1, 2, 4])))
            if rng.random() < 0.6:
                L[:, b, stop[0]] = float(L[:, b].nan_to_num(nan=0.0).max()) + 1.0  # likely as soon as the mask lifts
        if rng.random() < 0.4:
            ids = rng.choice(V, size=min(V, int(rng.choice([1, 20, 300]))), replace=False)
            kw["bias"] = {int(i): float(v) for i, v in zip(ids, rng.uniform(-100, 100, ids.size))}
        m = rng.random()
        if m < 0.15:
            kw["allowed"] = rng.choice(V, size=max(1, V // 7), replace=False).tolist()
        elif m < 0.3:
            bits = rng.random(V) < (0.05 if rng.random() < 0.9 else 1.0)  # now and then every token banned
            w = np.zeros((V + 31) // 32, dtype=np.uint32)
            nz = np.nonzero(bits)[0]
            np.bitwise_or.at(w, nz >> 5, (np.uint32(1) << (nz & 31).astype(np.uint32)))
            kw["banned"] = w
        prompts.append(prompt)
        gens.append(gen)
        rows.append(q.RowSpec(**kw))
    return L.to(dtype), prompts, gens, rows, bool(rng.random() < 0.5)


@pytest.mark.parametrize("seed", range(8))
def test_fuzz_decode(seed):
    L, prompts, gens, rows, by_finish = _decode_case(3000 + seed)
    steps, B, V = L.shape
    state = q.ProcState(B, V)
    for b in range(B):
        state.begin(b, prompts[b], gens[b])
    packed = q.PackedBatch(rows, V, "cuda", state)
    sm = q.Sampler("cuda")
    book = None
    if by_finish:
        book = q.StepBook(B)
        for b in range(B):
            book.start(b, 0, -1)
    rs = torch.arange(B, dtype=torch.int32, device="cuda")
    lg = torch.empty(B, V, dtype=L.dtype, device="cuda")
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    got = []
    for s in range(steps):
        lg.copy_(L[s])
        if by_finish:
            sm.run(packed, lg, out_tokens=tok)
            book.finish(rs, tok, state=state, rows=packed)
        else:
            sm.run(packed, lg, out_tokens=tok, advance=True)
        got.append(tok.cpu().tolist())
    Lf = L.float()
    for b, r in enumerate(rows):
        hist = list(gens[b])
        for s in range(steps):
            pr = S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=prompts[b],
                            gen=hist, bias=r.bias, allowed=r.allowed, banned=r.banned, stop=r.stop)
            want = S.sample_row(Lf[s, b], r.temperature, r.top_k, r.top_p, r.min_p, r.seed, r.position + s, r.stream, r.row_key, pr).token
            label = (f"seed {3000 + seed} V={V} B={B} {L.dtype} {'finish' if by_finish else 'advance'} row {b} step {s} "
                     f"({r.temperature}, {r.top_k}, {r.top_p}, {r.min_p}, stop {list(r.stop)} min_tokens {r.min_tokens} ngen {len(hist)})")
            assert got[s][b] == want, f"{label}: GPU {got[s][b]} != oracle {want}"
            hist.append(want)


@pytest.mark.parametrize("seed", range(12))
def test_fuzz_head(seed):
    """Random candidate selects + exact rescores against oracle/head.py: N from 4 to 262,144 (ragged last tiles), T 1-16,
    R 1-64, hidden sizes 8-1,024, a sub-vocabulary now and then, and rows of NaN, +-inf, signed zeros, long runs of
    ties, all-equal rows and rows with fewer non-NaN logits than R."""
    from test_gpu_head import _head, check
    from qwen_warp_amd import _lib
    rng = np.random.default_rng(4000 + seed)
    g = torch.Generator().manual_seed(4000 + seed)
    N = int(rng.choice([4, 40, 4096, 4100, 20492, 65536, 100000, 262144]))
    T = int(rng.choice([1, 2, 5, 16]))
    R = int(rng.choice([1, 2, 7, 20, 63, 64]))
    K = int(rng.choice([8, 64, 512, 1024]))
    lg = torch.randn(T, N, generator=g) * float(rng.choice([0.01, 1.0, 30.0]))
    for t in range(T):
        k = rng.integers(7)
        if k == 1:
            lg[t] = torch.round(lg[t] * 2) / 2  # ties
        elif k == 2:
            lg[t] = 0.25  # all equal
        elif k == 3:
            lg[t, torch.randint(0, N, (max(1, N // 10),), generator=g)] = float("nan")
        elif k == 4:
            lg[t, : max(0, N - int(rng.integers(0, R + 1)))] = float("nan")  # at most R non-NaN logits
        elif k == 5:
            lg[t, int(rng.integers(N))] = math.inf
            lg[t, int(rng.integers(N))] = -math.inf
            lg[t, :: max(1, N // 50)] = 0.0
            lg[t, 1 :: max(1, N // 50)] = -0.0
    ids = None
    V = N
    if rng.random() < 0.3:
        V = N + int(rng.integers(1, 5000))
        ids = torch.sort(torch.randperm(V, generator=g)[:N]).values.to(torch.int32)
    w = _head(V, K, g)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    check(_lib.load(), lg.contiguous(), w, x, R, ids=ids, label=f"seed {4000 + seed} N={N} T={T} R={R} K={K} ids={ids is not None}")


@pytest.mark.parametrize("seed", range(8))
def test_fuzz_pld(seed):
    """Random prompt-lookup proposers against oracle/pld.py: configurations across their ranges (n-gram widths, minimum
    lengths, tails, caps, look-back windows, first or longest match), small and large alphabets, histories from empty
    to past max_len (the overflow rule), proposals with and without drafts, appends of 1..T tokens with -1 padding."""
    import random
    from oracle.pld import Pld, PldCfg
    from qwen_warp_amd import _lib
    from qwen_warp_amd.pld import DevicePld
    rng = random.Random(5000 + seed)
    cfg = PldCfg(n=rng.randint(1, 5), min_len=rng.randint(0, 5), max_tail=rng.randint(0, 8), cap=rng.choice([1, 2, 5, 64, 1000]),
                 back=rng.choice([1, 4, 64, 500]), longest=rng.randint(0, 1))
    S, max_len = rng.choice([1, 5, 16]), rng.choice([64, 512, 4096])
    dev = DevicePld(S, max_len, _lib.PldCfg(cfg.n, cfg.min_len, cfg.max_tail, cfg.cap, cfg.back, cfg.longest))
    refs = [Pld(cfg) for _ in range(S)]
    alpha = rng.choice([2, 4, 12, 1000])
    size = [0] * S  # history lengths: past max_len a sequence proposes nothing until its next reset
    for s in range(S):
        ctx = [rng.randrange(alpha) for _ in range(min(max_len - 3, rng.choice([0, 1, 5, 100, max_len - 3])))]
        dev.reset(s, ctx)
        refs[s].reset(ctx)
        size[s] = len(ctx)
    for step in range(20):
        seqs = rng.sample(range(S), rng.randint(1, S))
        nd = rng.randint(0, 7)
        drafts = [[rng.randrange(alpha) for _ in range(nd)] for _ in seqs] if nd else None
        mt, ml = rng.randint(0, 8), rng.randint(0, 6)
        d = torch.tensor(drafts, dtype=torch.int32, device="cuda") if drafts else None
        out, n, l = dev.propose(seqs, d, mt, ml)
        out, n, l = out.cpu().numpy(), n.cpu().numpy(), l.cpu().numpy()
        for b, s in enumerate(seqs):
            want, wl = refs[s].propose(drafts[b] if drafts else [], mt, ml) if size[s] <= max_len else ([], 0)
            got = out[b, : n[b]].tolist()
            assert (got, int(l[b])) == (want, wl), f"seed {5000 + seed} {cfg} step {step} row {b} (seq {s}): {got}, l={int(l[b])} != {want}, l={wl}"
        T = rng.randint(1, 10)
        arr = np.full((len(seqs), T), -1, dtype=np.int32)
        for b, s in enumerate(seqs):
            k = rng.randint(1, T)
            toks = [rng.randrange(alpha) for _ in range(k)]
            arr[b, :k] = toks
            refs[s].append(toks)
            size[s] += k
        dev.append(seqs, torch.from_numpy(arr).cuda())
