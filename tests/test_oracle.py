"""Pins the CPU oracle (oracle/sampler.py) before it is trusted as the parity reference: known-answer vectors,
the literal cases of the reference's tests, closed forms, a textbook double-precision restatement and exact
enumeration.  CPU only."""
import math

import numpy as np
import pytest
import torch

from oracle import sampler as S
from _util import GOLDEN, chi_square, chi2_sf, textbook_dist

Vs = 2000  # small vocabulary for the semantic cases


def test_chi2_sf_known_values():
    for c in GOLDEN["chi2_sf"]:
        assert abs(chi2_sf(c["x"], c["dof"]) - c["sf"]) < c["tol"]


# ---------------------------------------------------------------------------------------------- Philox
def test_philox_known_answers():
    for v in GOLDEN["philox_kat"]:
        out = S.philox(*v["ctr"], *v["key"])
        assert [int(o) for o in out] == v["out"]


def test_philox_vectorised_matches_scalar():
    seed = 0x123456789ABCDEF
    pos = np.arange(1000)
    vec = S.philox(pos, S.ST_DRAW, 7, 0, seed & 0xFFFFFFFF, seed >> 32)
    for i in (0, 1, 517, 999):
        one = S.philox(i, S.ST_DRAW, 7, 0, seed & 0xFFFFFFFF, seed >> 32)
        assert all(int(vec[w][i]) == int(one[w]) for w in range(4))


def test_u24_range_and_uniformity():
    u = S.draw_u24(42, np.arange(200000), S.ST_DRAW).astype(np.int64)
    assert u.min() >= 0 and u.max() < (1 << 24)
    counts = np.bincount(u >> 18, minlength=64)
    _, _, p = chi_square(counts, np.full(64, 1 / 64), len(u))
    assert p > 1e-4


# ---------------------------------------------------------------------------------------------- exp2 mantissa
def test_exp2_table_accuracy_and_range():
    """mu / 2^23 approximates 2^(a - floor(a)) to 1.7e-7 (a = t / 1024); closed forms at exact points."""
    t = torch.linspace(-3 * 1024, 3 * 1024, 600001, dtype=torch.float32)
    q, mu = S.exp2_table(t)
    n = q >> 10
    ref = torch.pow(2.0, t.double() / 1024 - n.double())
    rel = ((mu.double() / 2.0 ** 23 - ref) / ref).abs().max().item()
    assert rel < 1.8e-7, rel
    assert int(mu.min()) >= 1 << 23 and int(mu.max()) <= 1 << 24
    # table points: r = 0 gives TAB_T exactly; the table itself is 2^(j/1024) rounded once
    n, mu = S.mantissa(torch.tensor([0.0, 512.0, 1023.9999, -3.25 * 1024, 7.0 * 1024]))
    assert n.tolist() == [0, 0, 0, -4, 7]
    assert int(mu[0]) == 1 << 23 and int(mu[4]) == 1 << 23
    assert int(mu[1]) == int(S.TAB_T[512]) == round(2 ** 0.5 * 2 ** 23)
    for j in (0, 1, 511, 1023):
        assert int(S.TAB_T[j]) == round(2 ** (j / 1024) * 2 ** 23)
        assert abs(float(S.TAB_T[j]) + float(S.TAB_S[j]) - 2 ** ((j + 1) / 1024) * 2 ** 23) <= 1.0
    # fine bin = floor(a * 64) = q >> 4; n = floor(a) = q >> 10
    q, _ = S.exp2_table(torch.tensor([0.0, 16.0, -16.0, 5.0 * 1024 - 0.5]))
    assert (q >> 4).tolist() == [0, 1, -1, 319]
    # the fraction stays below 1 where t - floor(t) rounds up to 1 (tiny negative t)
    q, mu = S.exp2_table(torch.tensor([-2.0 ** -30]))
    assert int(q[0]) == -1 and int(mu[0]) <= 1 << 24


def test_device_table_matches_oracle():
    """The HIP library's interpolation table (qws_device.h) holds the oracle's constants."""
    import re
    from pathlib import Path
    src = (Path(__file__).resolve().parent.parent / "qwen-warp_amd" / "csrc" / "qws_device.h").read_text()
    body = src[src.index("EXP2_TS[2048]"):]
    body = body[: body.index("};")]
    words = [int(w, 16) for w in re.findall(r"0x[0-9a-fA-F]{8}", body)]
    assert len(words) == 2048
    assert words[0::2] == S.TAB_T.view(np.uint32).tolist()
    assert words[1::2] == S.TAB_S.view(np.uint32).tolist()


def test_temperature_scaling_is_exact():
    """t = fl(x * kappa * 1024) equals fl(x * kappa) * 1024 (power-of-two scaling commutes with rounding)."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(100000, generator=g) * 5
    for T in (0.3, 0.7, 1.0, 1.37):
        k = S.kappa32(T)
        a = (x * torch.tensor(k)) * torch.tensor(np.float32(1024.0))
        assert torch.equal(a, S.t_units(x, T))
    assert S.sampled_row(1e-30) and not S.sampled_row(1e-37) and not S.sampled_row(0.0)


def test_weights_close_to_exp():
    """w_i / w_max approximates exp((x_i - x_max) / T) to ~2^-23."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(500, generator=g) * 2
    ids, ws, S2 = S.distribution(x, 0.7)
    xm = float(x.max())
    for i, w in zip(ids[:50], ws[:50]):
        ref = math.exp((float(x[i]) - xm) / float(np.float32(0.7)))
        assert abs(w / ws[0] - ref) <= 2e-6 * max(ref, 1e-30) + 1e-15


# ---------------------------------------------------------------------------------------------- processors
def rows(x, **kw):
    return S.process(x, S.RowProcs(**kw))


def test_sglang_literal_cases():
    for c in GOLDEN["sglang"]:
        x = torch.full((Vs,), c["logits"])
        o = rows(x, gen=c["gen"], frequency=c.get("frequency", 0.0), presence=c.get("presence", 0.0))
        for k, v in c["check"].items():
            assert float(o[int(k)]) == v


def test_min_tokens_sglang_cases():
    # rows with 0 and 1 generated tokens (the second row's drafts count as generated): stop ids blocked
    for d in ([], [9]):
        o = S.process(torch.zeros(Vs), S.RowProcs(min_tokens=3, stop=[2, 5, 10], gen=[]), drafts_before=d)
        assert all(float(o[i]) == -math.inf for i in (2, 5, 10)) and float(o[0]) == 0.0
    o = rows(torch.zeros(Vs), min_tokens=2, stop=[2], gen=[10, 11])
    assert float(o[2]) == 0.0
    # boundary: min_tokens = ngen + 1 masks, ngen masks nothing (tests/test_logit_procs.py:129-131)
    assert float(rows(torch.zeros(Vs), min_tokens=3, stop=[4], gen=[1, 1])[4]) == -math.inf
    assert float(rows(torch.zeros(Vs), min_tokens=2, stop=[4], gen=[1, 1])[4]) == 0.0


def test_vllm_argmin_cases():
    c = torch.full((Vs,), 1e-2)
    out_tok = [3, 4, 5, 5, 4, 3]
    o = rows(c, gen=out_tok, presence=2.0)
    assert int(o.argmin()) in out_tok and int(o.argmax()) not in out_tok
    o = rows(c, gen=out_tok, presence=-2.0)
    assert int(o.argmax()) in out_tok and int(o.argmin()) not in out_tok
    o = rows(c, gen=[3, 4, 4, 5, 5, 5], frequency=2.0)
    assert int(o.argmin()) == 5 and int(o.argmax()) not in (3, 4, 5)
    o = rows(c, gen=[3, 4, 4, 5, 5, 5], frequency=-2.0)
    assert int(o.argmax()) == 5 and int(o.argmin()) not in (3, 4, 5)
    for rp in (0.1, 1.9):
        o = rows(c, prompt=[20, 21], gen=[30], repetition=rp)
        seen = {20, 21, 30}
        pen, non = int(o.argmin()), int(o.argmax())
        assert (pen in seen and non not in seen) if rp > 1 else (non in seen and pen not in seen)
    o = rows(c, allowed=[3, 4])
    assert bool(torch.all(torch.isinf(o[5:]))) and bool(torch.all(o[:3] == -math.inf)) and bool(torch.all(o[3:5] == c[3:5]))


def test_llama_cpp_penalty_probabilities():
    lp = torch.full((Vs,), -math.inf)
    lp[:5] = math.log(0.2)
    for c in GOLDEN["llama_penalties"]:
        o = rows(lp, gen=c["gen"], repetition=c.get("repetition", 1.0), frequency=c.get("frequency", 0.0), presence=c.get("presence", 0.0))
        p = torch.softmax(o.double(), 0)[:5].tolist()
        assert all(abs(a - b) <= c["tol"] for a, b in zip(p, c["probs"])), (c, p)


def test_repetition_sign_rule_and_order():
    x = torch.zeros(Vs)
    x[1], x[2] = 2.0, -2.0
    o = rows(x, prompt=[1, 2], repetition=2.0)
    assert float(o[1]) == 1.0 and float(o[2]) == -4.0 and float(o[0]) == 0.0
    # bias is added before the penalties: (x + b) / r, not x / r + b (tests/test_logit_procs.py:157-158)
    x = torch.zeros(Vs)
    x[7] = 3.0
    o = rows(x, gen=[7], bias={7: 1.0}, repetition=2.0)
    assert float(o[7]) == 2.0          # (3 + 1) / 2
    assert float(o[7]) != 3.0 / 2 + 1.0  # the wrong order gives 2.5


def test_drafts_count_as_generated():
    x = torch.zeros(Vs)
    for t, want in ((0, 0.0), (1, -0.5), (2, -1.0)):
        o = S.process(x, S.RowProcs(frequency=0.5), drafts_before=[5, 5][:t])
        assert float(o[5]) == want
    # presence is flat in the count, repetition sees the drafts
    o = S.process(torch.full((Vs,), 4.0), S.RowProcs(presence=1.0, repetition=2.0), drafts_before=[9, 9])
    assert float(o[9]) == 1.0 and float(o[8]) == 4.0


def test_banned_mask_and_nan():
    x = torch.randn(Vs)
    x[11] = float("nan")
    m = S.pack_bits([3, 64, 1999], Vs)
    o = rows(x, banned=m)
    assert float(o[3]) == float(o[64]) == float(o[1999]) == -math.inf and float(o[11]) == -math.inf
    assert float(o[4]) == float(x[4])
    assert float(S.process(x, None)[11]) == -math.inf


def test_bias_minus_zero_canonical_and_greedy_ties():
    x = torch.zeros(Vs)
    x[5] = -0.0
    assert S.greedy(x) == 0  # -0 ties +0: lowest index
    x = torch.full((Vs,), -math.inf)
    assert S.greedy(x) == 0
    x = torch.full((Vs,), 1.0)
    x[17] = 2.0
    x[9] = 2.0
    assert S.greedy(x) == 9


# ---------------------------------------------------------------------------------------------- selection
def test_llama_cpp_min_p_cases():
    probs = torch.tensor([0.1, 0.2, 0.3, 0.4])
    x = torch.full((16,), -math.inf)
    x[:4] = torch.log(probs)
    for c in GOLDEN["llama_min_p"]:
        ids, ws, S2 = S.distribution(x, 1.0, top_k=4, top_p=1.0, min_p=c["min_p"])
        got = sorted(w / S2 for w in ws)
        assert len(got) == len(c["probs"]) and all(abs(a - b) < 1e-6 for a, b in zip(got, sorted(c["probs"]))), (c, got)


@pytest.mark.parametrize("T", [0.7, 1.0, 1.5])
@pytest.mark.parametrize("k,tp", [(64, 1.0), (20, 0.95), (5, 0.8), (0, 0.9), (0, 1.0), (1000, 0.5)])
@pytest.mark.parametrize("mp", [0.0, 0.02, 0.5])
def test_distribution_matches_textbook(T, k, tp, mp):
    g = torch.Generator().manual_seed(int(T * 10) + k + int(tp * 100) + int(mp * 1000))
    x = torch.randn(3000, generator=g) * 2.5
    ids, ws, S2 = S.distribution(x, T, top_k=k, top_p=tp, min_p=mp)
    got = {int(i): w / S2 for i, w in zip(ids, ws) if w > 0}
    ref = textbook_dist(x, T, k, tp, mp)
    # the fixed-point weights drop tokens below 2^-35 of the top power of two (probability < 2^-34)
    assert set(got) <= set(ref)
    assert all(ref[i] < 2.0 ** -34 for i in set(ref) - set(got))
    assert max(abs(got.get(i, 0.0) - ref[i]) for i in ref) < 1e-6


def test_ties_keep_exactly_k_lowest_index():
    x = torch.tensor([1.0, 3.0, 3.0, 2.0, 3.0, 3.0, 0.0, 3.0])
    ids, ws, S2 = S.distribution(x, 1.0, top_k=3)
    assert sorted(ids.tolist()) == [1, 2, 4]
    ids, ws, S2 = S.distribution(x, 1.0, top_k=0, top_p=0.5)  # 5 tokens tie at 3: the nucleus cuts by index
    ref = textbook_dist(x, 1.0, 0, 0.5)
    assert sorted(ids.tolist()) == sorted(ref)


def test_draws_chi_square_against_textbook():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(60, generator=g) * 1.5
    ref = textbook_dist(x, 0.9, 0, 0.9)
    ids, ws, S2 = S.distribution(x, 0.9, top_p=0.9)
    n = 20000
    u = S.draw_u24(11, np.arange(n), S.ST_DRAW)
    toks = [S.draw_index_order(ids, ws, S2, int(v)) for v in u]
    counts = np.bincount(toks, minlength=60)
    assert set(np.nonzero(counts)[0].tolist()) <= set(ref)
    probs = np.array([ref.get(i, 0.0) for i in range(60)])
    _, _, p = chi_square(counts, probs, n)
    assert p > 1e-3
    # negative control: a wrong temperature is rejected
    bad = textbook_dist(x, 0.6, 0, 0.9)
    _, _, pb = chi_square(counts, np.array([bad.get(i, 0.0) for i in range(60)]), n)
    assert pb < 1e-6


def test_draw_inverse_cdf_edges():
    ids = np.array([9, 2, 5])
    ws = [6, 3, 1]
    assert S.draw_index_order(ids, ws, 10, 0) == 2                      # t = 0: first in index order
    assert S.draw_index_order(ids, ws, 10, (1 << 24) - 1) == 9          # t = 9: last
    assert S.draw_index_order(ids, ws, 10, (3 << 24) // 10) == 2        # t = 2 -> inside id 2's mass [0, 3)
    assert S.draw_index_order(ids, ws, 10, -(-(3 << 24) // 10)) == 5    # t = 3 -> id 5's mass [3, 4)


# ---------------------------------------------------------------------------------------------- speculative verify
def _joint_check(K, N, procs_kw, gen, cfg, trials, flags, seed, tail=(), m=2, tail_as_table=False):
    """Emitted tokens of verify_seq (K chain drafts drawn from the drafter's q, then the fixed prompt-lookup `tail`
    tokens as delta proposals), completed to m tokens from the exact conditionals, against the exact autoregressive
    joint of m tokens (the method of tests/test_spec_procs.py:76-144).  tail_as_table: the broken control that
    treats the tail tokens as dense-table drafts with q = 0 (accepted whenever p > 0)."""
    import itertools
    g = torch.Generator().manual_seed(seed)
    k = K + len(tail)
    tl = torch.randn(k + 1, N, generator=g) * 1.5
    dl = tl[:K] + torch.randn(K, N, generator=g) * 0.8
    q = torch.cat([torch.softmax(dl / cfg["temperature"], 1).float(), torch.zeros(len(tail), N)])
    idmap = np.arange(N)
    procs = S.RowProcs(gen=gen, **procs_kw)
    cache = {}

    def cond(h):
        if h not in cache:
            x = S.process(tl[len(h)], procs, list(h))
            ids, ws, S2 = S.distribution(x, cfg["temperature"], cfg.get("top_k", 0), cfg.get("top_p", 1.0), cfg.get("min_p", 0.0))
            p = np.zeros(N)
            for i, w in zip(ids, ws):
                p[i] = w / S2
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
    rng = np.random.default_rng(seed)
    out = np.zeros((trials, m), dtype=np.int64)
    for tr in range(trials):
        drafts = [int(rng.choice(N, p=q[j].double().numpy() / q[j].double().sum().item())) for j in range(K)] + list(tail)
        r = S.verify_seq(tl, q, idmap, drafts, seed=seed, position=tr, procs=procs, test_flags=flags,
                         n_chain=None if (tail_as_table or not tail) else K, **cfg)
        y = list(r.tokens)[:m]
        while len(y) < m:
            p = cond(tuple(y))
            y.append(int(rng.choice(N, p=p / p.sum())))
        out[tr] = y
    counts = np.bincount(np.ravel_multi_index(out.T, (N,) * m), minlength=N ** m)
    return chi_square(counts, joint.reshape(-1), trials)


def test_verify_preserves_target_distribution():
    cfg = dict(temperature=1.0, top_k=0, top_p=0.95)
    pk = dict(prompt=[1, 2], presence=1.2, frequency=0.9, repetition=1.3)
    _, _, p = _joint_check(2, 6, pk, [3, 3], cfg, 6000, 0, 21)
    assert p > 1e-3
    _, _, pb = _joint_check(2, 6, pk, [3, 3], cfg, 6000, 1, 21)  # broken: resample from p, not the residual
    assert pb < 1e-6


def test_verify_chain_and_tail_preserves_target_distribution():
    """One chain draft and two prompt-lookup tail tokens (delta proposals, k_delta_q engine/src/mtp_sample.cu:286-296),
    penalties counting the drafts: the joint of 3 emitted tokens equals the autoregressive one (the reference's third
    scenario, tests/test_spec_procs.py:163-164); tails taken as dense-table drafts with q = 0 fail the same test."""
    cfg = dict(temperature=1.0, top_k=0, top_p=1.0)
    pk = dict(prompt=[1, 2], presence=1.5, frequency=1.0, repetition=1.4)
    _, _, p = _joint_check(1, 6, pk, [3, 4], cfg, 8000, 0, 23, tail=(3, 3), m=3)
    assert p > 1e-3
    _, _, pb = _joint_check(1, 6, pk, [3, 4], cfg, 8000, 0, 23, tail=(3, 3), m=3, tail_as_table=True)
    assert pb < 1e-6


def test_draft_params_make_sampp():
    """engine/src/mtp_sample.cu:379-383: the draft values where set, else the target's; top_k 1 without draft_sample."""
    assert S.draft_params(0.7, 20, 0.9) == (0.7, 20, 0.9)
    assert S.draft_params(0.7, 20, 0.9, draft_sample=0) == (0.7, 1, 0.9)
    assert S.draft_params(0.7, 20, 0.9, 1, 1.3, 8, 0.5) == (1.3, 8, 0.5)
    assert S.draft_params(0.7, 0, 1.0, 1, 0.0, 0, 0.0) == (0.7, 0, 1.0)


def test_q_fix_exact():
    from fractions import Fraction
    S2 = (1 << 79) + 12345
    for q in (0.0, 1.0, 0.5, 1e-30, 0.3, 0.999999, 1e-45, 1.2e-38):  # the last two are fp32 subnormals
        assert S.q_fix(q, S2) == math.floor(Fraction(float(np.float32(q))) * S2)
    assert S.q_fix(float("nan"), S2) == 0 and S.q_fix(-0.5, S2) == 0 and S.q_fix(1.5, S2) == S2
