"""GPU parity of libqws against the CPU oracle, through the C ABI: processed logits bit-identical, greedy tokens,
survivor sets and Philox-driven token choices bit-exact, probabilities within 1e-5 relative (fp32)."""
import copy
import ctypes as C
import math

import numpy as np
import pytest
import torch

import qwen_warp_amd as q
from qwen_warp_amd import _lib, workloads
from oracle import sampler as S
from _util import GOLDEN, V, chi_square

pytestmark = pytest.mark.gpu
PROB_RTOL = 1e-5


def procs_of(r: q.RowSpec):
    if not r.procs_on():
        return None
    return S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=r.prompt, gen=r.gen,
                      ngen=r.ngen, bias=r.bias, allowed=r.allowed, banned=r.banned, stop=r.stop)


def oracle_row(x: torch.Tensor, r: q.RowSpec) -> S.RowResult:
    return S.sample_row(x, r.temperature, r.top_k, r.top_p, r.min_p, r.seed, r.position, r.stream, r.row_key, procs_of(r), list(r.drafts))


def check_rows(sampler, logits_cpu, rows, dense=True, label="", lg=None):
    """Tokens (and with `dense` the survivor sets and probabilities) of the rows against the oracle; `lg`: the logits on
    the GPU when they are not logits_cpu copied (a strided view, say)."""
    lg = logits_cpu.cuda() if lg is None else lg
    if dense:
        tok, probs, info = sampler.probs(lg, rows)
        probs = probs.cpu()
    else:
        tok = sampler.sample(lg, rows)
        info = None
    tok = tok.cpu().tolist()
    for b, r in enumerate(rows):
        want = oracle_row(logits_cpu[b], r)
        assert tok[b] == want.token, f"{label} row {b}: token {tok[b]} != oracle {want.token} (info {None if info is None else int(info[b])})"
        if dense and not want.greedy:
            got_ids = torch.nonzero(probs[b]).flatten().numpy()
            w = np.array([float(v) for v in want.weights], dtype=np.float64)
            keep = w > 0
            ref_ids = np.asarray(want.kept)[keep]
            o = np.argsort(ref_ids)
            ref_ids, ref_p = ref_ids[o], (w[keep] / float(want.S2))[o]
            assert np.array_equal(got_ids, ref_ids), f"{label} row {b}: survivor sets differ ({len(got_ids)} vs {len(ref_ids)})"
            err = float(np.max(np.abs(probs[b, got_ids].double().numpy() - ref_p) / ref_p))
            assert err < PROB_RTOL, f"{label} row {b}: probability rel err {err}"
    return info


def test_philox_hook_known_answers():
    lib = _lib.load()
    for v in GOLDEN["philox_kat"]:
        c = (C.c_uint * 4)(*v["ctr"])
        k = (C.c_uint * 2)(*v["key"])
        out = (C.c_uint * 4)()
        _lib.check(lib.qws_test_philox(c, k, out), "philox")
        assert list(out) == v["out"]


def _random_case(seed, T=4):
    """tests/test_logit_procs.py:99-107: logits with exact zeros, a 300-token prompt, repeated generated tokens."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, V, generator=g) * 3.0
    logits[:, :50] = 0.0
    prompt = torch.randint(0, V, (300,), generator=g).tolist()
    pool = torch.randint(0, V, (12,), generator=g).tolist()
    gen = [pool[int(i)] for i in torch.randint(0, 12, (40,), generator=g)]
    drafts = [pool[0], prompt[5], 7][: T - 1]
    return g, logits, prompt, gen, drafts, pool


def _hook_rows(lib, logits, prompt=(), gen=(), drafts=(), pres=0.0, freq=0.0, rep=1.0, min_tokens=0, stop=(), bias=None, allowed=None):
    T = logits.shape[0]
    p, keep = q.make_procs(prompt=prompt, presence=pres, frequency=freq, repetition=rep, min_tokens=min_tokens, bias=bias, allowed=allowed, stop=stop)
    g = (C.c_int * max(1, len(gen)))(*gen)
    d = (C.c_int * 8)(*(list(drafts) + [0] * (8 - len(drafts))))
    lg = logits.contiguous().float()
    out = torch.empty_like(lg)
    _lib.check(lib.qws_test_proc_logits(C.byref(p), T, lg.shape[1], g, len(gen), d, C.c_void_p(lg.data_ptr()), C.c_void_p(out.data_ptr())), "proc")
    assert keep is not None
    return out


def _oracle_rows(logits, prompt=(), gen=(), drafts=(), pres=0.0, freq=0.0, rep=1.0, min_tokens=0, stop=(), bias=None, allowed=None):
    pr = S.RowProcs(presence=pres, frequency=freq, repetition=rep, min_tokens=min_tokens, prompt=prompt, gen=gen, bias=bias, allowed=allowed, stop=stop)
    return torch.stack([S.process(logits[t], pr, list(drafts[:t])) for t in range(logits.shape[0])])


def test_processed_logits_bit_identical():
    """The 17 parameter cases of tests/test_logit_procs.py:117-135, T = 4 verify rows with drafts."""
    lib = _lib.load()
    g, logits, prompt, gen, drafts, pool = _random_case(1)
    stop = [248046, 248044]
    bias = {pool[1]: 5.5, 11: -100.0, pool[2]: 100.0, 123456: -3.25}
    allowed_small = [pool[0], 4242]
    allowed_big = torch.randperm(V, generator=g)[:10000].tolist() + pool
    base = dict(prompt=prompt, gen=gen, drafts=drafts)
    cases = {
        "presence 1.5": dict(pres=1.5), "presence -2": dict(pres=-2.0), "frequency 0.7": dict(freq=0.7), "frequency -1.3": dict(freq=-1.3),
        "repetition 1.0": dict(rep=1.0), "repetition 1.3": dict(rep=1.3), "repetition 0.6": dict(rep=0.6), "repetition 2": dict(rep=2.0),
        "logit_bias": dict(bias=bias), "allowed 2": dict(allowed=allowed_small), "allowed 10k": dict(allowed=allowed_big),
        "min_tokens rows 0,1": dict(min_tokens=len(gen) + 2, stop=stop), "min_tokens reached": dict(min_tokens=len(gen), stop=stop),
        "min_tokens all rows": dict(min_tokens=len(gen) + 4, stop=stop), "all penalties": dict(pres=0.5, freq=0.4, rep=1.2),
        "everything": dict(pres=0.5, freq=0.4, rep=1.2, bias=bias, allowed=allowed_big, min_tokens=len(gen) + 2, stop=stop + [pool[3]]),
        "everything, allowed 2": dict(pres=1.0, freq=1.0, rep=1.5, bias=bias, allowed=allowed_small, min_tokens=len(gen) + 1, stop=[allowed_small[1]]),
    }
    for name, kw in cases.items():
        kw = {**base, **kw}
        got = _hook_rows(lib, logits, **kw)
        ref = _oracle_rows(logits, **kw)
        assert torch.equal(got, ref), f"{name}: {int((got != ref).sum())} of {ref.numel()} differ"
    # T = 8 rows with 7 drafts
    l8 = torch.randn(8, V, generator=g) * 3.0
    d8 = [pool[0], pool[0], pool[1], 9, pool[0], prompt[1], pool[1]]
    kw = dict(prompt=prompt, gen=gen, drafts=d8, pres=0.8, freq=0.6, rep=1.1, min_tokens=len(gen) + 5, stop=stop)
    assert torch.equal(_hook_rows(lib, l8, **kw), _oracle_rows(l8, **kw))


def test_greedy_edge_cases(sampler):
    x = torch.randn(6, V) * 2
    x[0, 1000] = x[0, 2000] = 50.0                   # tie: lowest index
    x[1, :] = float("nan")
    x[1, 77] = -5.0                                   # NaN never wins
    x[2, :] = -math.inf                               # all masked: index 0
    x[3, :] = 0.0
    x[3, 0] = -0.0                                    # -0 ties +0
    x[4, 12345] = float("inf")
    x[5, 248319] = 99.0                               # last token
    rows = [q.RowSpec(temperature=0.0) for _ in range(6)]
    tok = sampler.sample(x.cuda(), rows).cpu().tolist()
    assert tok == [S.greedy(S.widen(x[b])) for b in range(6)] == [1000, 77, 0, 0, 12345, 248319]


def test_argmax_drop_in():
    lib = _lib.load()
    x = (torch.randn(16, V) * 3).cuda()
    x[3, 5] = x[3, 9] = 100.0
    ws = torch.empty(lib.qws_argmax_ws_bytes(), dtype=torch.uint8, device="cuda")
    tok = torch.empty(16, dtype=torch.int32, device="cuda")
    val = torch.empty(16, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.qws_argmax(x.data_ptr(), 16, V, tok.data_ptr(), val.data_ptr(), ws.data_ptr(), C.c_void_p(st)), "argmax")
    xc = x.cpu()
    assert tok.cpu().tolist() == [S.greedy(xc[b]) for b in range(16)]
    assert torch.equal(val.cpu(), xc.max(1).values)


@pytest.mark.parametrize("name", ["c1", "c1_greedy", "c2", "c5"])
def test_config_parity(sampler, name):
    """Every row of the configuration at its benchmark batch size, so the launch shape checked is the one timed
    (C5's 32 rows x 31 blocks run the 512-thread scan)."""
    w = workloads.ALL[name]()
    info = check_rows(sampler, w.logits, w.rows, label=name)
    print(f"{name}: {len(w.rows)} rows, fallback rows {int((info == 1).sum())}")


def test_config_c4_parity(sampler):
    """All 64 rows of the headline configuration in one call: the launch shape bench.py times."""
    w = workloads.c4()
    info = check_rows(sampler, w.logits, w.rows, label="c4")
    assert int((info == 1).sum()) == 0, "c4 rows resolved by rescans"


def test_min_p_llama_cases_dist_hook():
    lib = _lib.load()
    probs = torch.tensor([0.1, 0.2, 0.3, 0.4])
    N = 64
    x = torch.full((1, N), -math.inf)
    x[0, :4] = torch.log(probs)
    for c in GOLDEN["llama_min_p"]:
        cfg = q.make_sampling(temperature=1.0, top_k=4, top_p=1.0, min_p=c["min_p"])
        out_p = torch.zeros(1, N)
        out_t = torch.zeros(1, dtype=torch.int32)
        _lib.check(lib.qws_test_dist(C.c_void_p(x.data_ptr()), 1, N, C.byref(cfg), 0, C.c_void_p(out_p.data_ptr()), C.c_void_p(out_t.data_ptr())), "dist")
        got = sorted(v for v in out_p[0].tolist() if v > 0)
        assert len(got) == len(c["probs"]) and all(abs(a - b) < 1e-6 for a, b in zip(got, sorted(c["probs"]))), (c, got)


@pytest.mark.parametrize("T,k,tp,mp", [(0.7, 20, 0.8, 0.0), (1.0, 0, 0.95, 0.0), (1.3, 0, 1.0, 0.0), (0.8, 1000, 0.9, 0.05),
                                      (1.0, 0, 0.9, 0.02), (0.5, 5, 1.0, 0.0), (1.0, 0, 1.0, 0.1)])
def test_random_rows_parity(sampler, T, k, tp, mp):
    g = torch.Generator().manual_seed(int(T * 100) + k + int(tp * 1000) + int(mp * 1e4))
    x = torch.randn(4, V, generator=g) * 2.0
    rows = [q.RowSpec(temperature=T, top_k=k, top_p=tp, min_p=mp, seed=7 + b, position=b, row_key=b) for b in range(4)]
    check_rows(sampler, x, rows, label=f"T{T} k{k} p{tp} m{mp}")


def test_many_draws_chi_square_and_bit_exact():
    """10^6 draws (counter = i, stream DRAW) from one processed row through the production kernels."""
    N = 4096
    g = torch.Generator().manual_seed(9)
    x = torch.randn(N, generator=g) * 1.5
    ss = q.SeqSampler(row_key=3)
    ss.set_sampling(temperature=0.9, top_k=0, top_p=0.9, seed=123)
    ss.set_procs(presence=0.5, repetition=1.2, prompt=[1, 2, 3])
    ss.note([5, 5, 9])
    n = 1_000_000
    toks = ss.test_draw(x.cuda(), n).cpu().numpy()
    r = ss.row(stream=S.ST_DRAW)
    pr = procs_of(r)
    xp = S.process(x, pr)
    ids, ws, S2 = S.distribution(xp, r.temperature, r.top_k, r.top_p, r.min_p)
    u = S.draw_u24(r.seed, np.arange(1000), S.ST_DRAW, r.row_key)
    assert [S.draw_index_order(ids, ws, S2, int(v)) for v in u] == toks[:1000].tolist()
    probs = np.zeros(N)
    for i, w in zip(ids, ws):
        probs[i] = w / S2
    counts = np.bincount(toks, minlength=N)
    assert set(np.nonzero(counts)[0].tolist()) <= set(int(i) for i in ids)
    _, _, p = chi_square(counts, probs, n)
    assert p > 0.01


@pytest.mark.parametrize("name", ["c1", "c4"])
def test_many_draws_full_vocabulary(name):
    """10^6 draws (counter = i, stream DRAW) from the first row of C1 / C4 (V = 248,320, the configuration's
    temperature, top-k, top-p and repetition over its history) through the production kernels, in chunks of 8,192
    rows that share the logits: the first 1,000 draws bit-exact against the oracle, then a chi-square of all of them
    against the oracle's kept distribution."""
    w = workloads.ALL[name]()
    r0 = w.rows[0]
    x = w.logits[0]
    ss = q.SeqSampler(row_key=r0.row_key)
    ss.set_sampling(temperature=r0.temperature, top_k=r0.top_k, top_p=r0.top_p, min_p=r0.min_p, seed=r0.seed)
    ss.set_procs(repetition=r0.repetition, presence=r0.presence, frequency=r0.frequency)
    ss.note(list(r0.gen))
    n, chunk = 1_000_000, 8192
    xd = x.cuda()
    toks = np.concatenate([ss.test_draw(xd, min(chunk, n - c0), ctr0=c0).cpu().numpy() for c0 in range(0, n, chunk)])
    r = ss.row(stream=S.ST_DRAW)
    xp = S.process(x, procs_of(r))
    ids, ws, S2 = S.distribution(xp, r.temperature, r.top_k, r.top_p, r.min_p)
    ids = np.asarray(ids, dtype=np.int64)
    o = np.argsort(ids, kind="stable")
    cum = np.cumsum(np.asarray([int(v) for v in ws], dtype=object)[o])  # exact prefix sums in index order
    u = S.draw_u24(r.seed, np.arange(1000), S.ST_DRAW, r.row_key)
    want = [int(ids[o[int(np.searchsorted(cum, (int(v) * int(S2)) >> 24, side="right"))]]) for v in u]
    assert want == toks[:1000].tolist()
    probs = np.zeros(x.numel())
    probs[ids] = np.array([float(v) for v in ws]) / float(S2)
    counts = np.bincount(toks, minlength=x.numel())
    assert set(np.nonzero(counts)[0].tolist()) <= set(ids.tolist())
    stat, dof, p = chi_square(counts, probs, n)
    print(f"{name}: {len(ids)} kept, chi-square {stat:.0f} on {dof} dof, p {p:.3g}")
    assert p > 0.01


def _with_flags(rows, flags):
    out = []
    for r in rows:
        c = copy.copy(r)
        c.test_flags = r.test_flags | flags
        out.append(c)
    return out


@pytest.mark.parametrize("name", ["c1", "c2", "c5"])
def test_rescan_path_parity(sampler, name):
    """The resolver's rescan fallback (QWS_TF_RESCAN: every cut bin's elements from rescans of the blocks instead of
    the first pass's lists) against the oracle."""
    w = workloads.ALL[name]()
    n = min(len(w.rows), 4)
    info = check_rows(sampler, w.logits[:n], _with_flags(w.rows[:n], q.TF_RESCAN), label=name + " rescan")
    assert all(int(i) in (0, 1, 2) for i in info)
    # c5's rows weigh fewer than top_k = 50 candidates (the +100 biases): no cut, nothing gathered; c1's cut bins each
    # hold the one boosted token at the cut, taken whole from the bin words: nothing gathered either
    if name == "c2":
        assert any(int(i) == 1 for i in info)


def test_rescan_path_parity_without_processors(sampler):
    """Rescans of blocks without processed tokens read the raw logits straight into registers: C4's and C3's first
    rows without penalties, every cut bin from rescans (QWS_TF_RESCAN), against the oracle."""
    for name in ("c4", "c3"):
        w = workloads.ALL[name]()
        lg = w.logits.reshape(-1, w.logits.shape[-1])[:4]
        rows = [q.RowSpec(temperature=1.0, top_k=0, top_p=[0.95, 0.5, 0.99, 0.8][b], min_p=[0.0, 0.0, 0.0, 0.05][b], seed=50 + b,
                          row_key=b, position=3 + b, test_flags=q.TF_RESCAN) for b in range(4)]
        info = check_rows(sampler, lg, rows, label=name + " rescan, no processors")
        assert any(int(i) == 1 for i in info)


def test_fast_and_rescan_paths_agree(sampler):
    """Every row of the headline workload draws the same token from the records and from exact rescans."""
    w = workloads.c4()
    lg = w.logits.cuda()
    a = sampler.sample(lg, w.rows).cpu().tolist()
    b = sampler.sample(lg, _with_flags(w.rows, q.TF_RESCAN)).cpu().tolist()
    assert a == b


def _row(**kw):
    base = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=11, position=3, row_key=0)
    base.update(kw)
    return q.RowSpec(**base)


@pytest.mark.parametrize("V_", [8, 16, 64, 8192, 8200, 24584, 400000, 524288])
def test_sampled_small_and_ragged_vocab(sampler, V_):
    """Vocabularies of one partial block, exactly one block, a ragged last block, and more blocks than a wave has lanes
    (49, and 64: the most a row may have)."""
    g = torch.Generator().manual_seed(V_)
    x = torch.randn(5, V_, generator=g) * 2.0
    rows = [_row(top_k=5, row_key=0), _row(top_p=0.9, row_key=1), _row(min_p=0.05, row_key=2), _row(temperature=0.5, top_k=0, top_p=0.7, row_key=3),
            _row(temperature=2.0, row_key=4)]
    check_rows(sampler, x, rows, label=f"V={V_}")


@pytest.mark.parametrize("B_,V_,pad,dtype", [(5, 24584, 8, torch.float32), (40, 65536, 64, torch.float32), (40, 65536, 8, torch.bfloat16)])
def test_padded_row_stride(sampler, B_, V_, pad, dtype):
    """Logits as a view of wider rows (row_stride = V + pad, as a padded head output): the 1,024-thread scan (B * G <=
    the CU count) and the 512-thread one, fp32 and bf16, against the oracle.  The padding holds 1e4, which would win
    every row if it were read."""
    g = torch.Generator().manual_seed(V_ + pad)
    wide = (torch.randn(B_, V_ + pad, generator=g) * 2.0).to(dtype)
    wide[:, V_:] = 1e4
    x = wide[:, :V_].float()
    lg = wide.cuda()[:, :V_]
    assert lg.stride(0) == V_ + pad and not lg.is_contiguous()
    rows = [_row(top_k=[0, 5, 50][b % 3], top_p=[0.9, 1.0, 0.7][b % 3], min_p=0.02 * (b % 2), temperature=0.5 + 0.1 * (b % 7), row_key=b)
            for b in range(B_)]
    check_rows(sampler, x, rows, label=f"stride {V_ + pad} {dtype}", lg=lg)


def test_bias_bound_block_skips(sampler):
    """Rows whose biased tokens tower over the rest: blocks whose best lies more than 35 powers of two below the biased
    tokens' bound record only their header, and the elements past every row's window are neither weighed nor counted.
    The bound must leave out a biased token that is banned, one that is a stop token while min_tokens holds, and every
    row whose penalties count tokens; each row against the oracle.  40 rows x 8 blocks: more workgroups than CUs, the
    512-thread scan that applies the bound."""
    V_ = 65536
    g = torch.Generator().manual_seed(91)
    x = torch.randn(40, V_, generator=g) * 3.0
    banned = np.zeros((V_ + 31) // 32, dtype=np.uint32)
    banned[1000 >> 5] |= np.uint32(1 << (1000 & 31))
    rows = [
        _row(temperature=0.6, top_k=50, bias={40000: 100.0, 7: 60.0}, row_key=0),                 # most blocks below
        _row(temperature=0.6, bias={1000: 100.0, 30000: 20.0}, banned=banned, row_key=1),         # the +100 token banned
        _row(temperature=0.6, bias={12: 100.0, 50000: 25.0}, stop=[12], min_tokens=3, row_key=2),  # the +100 token a stop id
        _row(temperature=0.6, bias={12: 100.0}, stop=[12], min_tokens=1, ngen=1, row_key=3),      # min_tokens met: kept
        _row(temperature=0.6, bias={300: 100.0}, repetition=1.3, gen=[300, 300], row_key=4),      # penalties: no bound
        _row(temperature=1.0, top_p=0.9, bias={60000: 40.0, 5: -100.0}, row_key=5),
        _row(temperature=0.2, bias={9: 8.0}, row_key=6),
        _row(temperature=0.6, top_p=0.95, bias={i * 997 % V_: 100.0 - i for i in range(40)}, row_key=7),
    ]
    rows = [q.RowSpec(**{**{k: getattr(r, k) for k in q.RowSpec.__dataclass_fields__}, "row_key": 8 * c + i, "seed": 11 + c})
            for c in range(5) for i, r in enumerate(rows)]
    assert len(rows) * ((V_ + 8191) // 8192) > 256
    check_rows(sampler, x, rows, label="bias bound")
    check_rows(sampler, x.to(torch.bfloat16).float(), rows, label="bias bound bf16 values")


@pytest.mark.parametrize("V_", [8, 1000, 8192, 65536])
def test_min_p_beside_top_k(sampler, V_):
    """min-p keeps more than K candidates, most or all of them in one block, and top-k then cuts to K: a block writes
    its bins only down to its own K-th candidate, so the count above the row's min-p cut saturates at K and the top-k
    cut must still run (K == the count seen); also K equal to and above the min-p set, and top-p after both."""
    g = torch.Generator().manual_seed(V_ + 5)
    x = torch.randn(12, V_, generator=g) * 0.4
    x[:, : min(V_, 16)] += 3.0  # a cluster of candidates at the top, in the first block
    rows = []
    for i, (k, mp, tp) in enumerate([(5, 0.3, 1.0), (5, 0.01, 1.0), (1, 0.3, 1.0), (8, 0.3, 1.0), (16, 0.3, 1.0), (64, 0.3, 1.0),
                                    (5, 0.3, 0.5), (3, 0.9, 1.0), (2, 0.5, 0.9), (7, 0.05, 1.0), (40, 0.2, 0.95), (5, 0.6, 1.0)]):
        rows.append(_row(temperature=[1.0, 0.7, 3.0][i % 3], top_k=min(k, V_), min_p=mp, top_p=tp, row_key=i))
    check_rows(sampler, x, rows, label=f"min-p + top-k V={V_}")


@pytest.mark.parametrize("V_,B_,dt", [(8, 24, torch.float32), (1000, 24, torch.bfloat16), (65536, 40, torch.float32), (65536, 24, torch.bfloat16)])
def test_lower_clamp(sampler, V_, B_, dt):
    """Rows whose best logit lies at or below the lower clamp of x * K (x / T below about -7.4e8: tiny temperatures
    with negative logits): every finite candidate ties at t = -2^30 with -inf (masked tokens, the padding past V), and
    only the finite ones may be weighed, counted or drawn.  Every cut and test flag; 40 rows x 8 blocks run the
    512-thread scan, 24 rows the 1,024-thread one."""
    g = torch.Generator().manual_seed(V_ + B_)
    x = -(torch.rand(B_, V_, generator=g) * 5.0 + 0.5)
    cuts = [(0, 1.0, 0.0), (50, 1.0, 0.0), (0, 0.5, 0.0), (2, 1.0, 0.0), (0, 1.0, 0.3), (5, 0.9, 0.1), (1, 1.0, 0.0), (0, 1e-7, 0.0)]
    flags = [0, q.TF_RESCAN, q.TF_STAGED_DRAW, q.TF_SPLIT_SELECT, q.TF_RESCAN | q.TF_STAGED_DRAW]
    rows = []
    for b in range(B_):
        k, tp, mp = cuts[b % len(cuts)]
        kw = dict(temperature=[1e-20, 1e-12][b % 2], top_k=min(k, V_), top_p=tp, min_p=mp, row_key=b, position=b, test_flags=flags[b % len(flags)])
        if b % 3 == 0:  # a few finite tokens, the rest -inf
            x[b, torch.randperm(V_, generator=g)[: V_ - 3]] = -math.inf
        elif b % 3 == 1:  # an allowed set
            kw["allowed"] = torch.randperm(V_, generator=g)[: max(2, V_ // 9)].tolist()
        if b % 4 == 3:  # a finite best above the clamp in the row: the clamped blocks carry no weight
            x[b, int(torch.randint(V_, (1,), generator=g))] = 1.0
        rows.append(_row(**kw))
    check_rows(sampler, x.to(dt), rows, label=f"lower clamp V={V_} {dt}")


def test_sampled_special_values(sampler):
    """NaN, +inf and -inf logits, a single survivor, all-equal rows and rows with nothing left."""
    N = 4096
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, N, generator=g) * 2.0
    x[0, ::7] = float("nan")                       # NaN is -inf
    x[1, 100] = float("inf")                       # one +inf: it takes all the mass
    x[1, 200] = float("inf")                       # two: split between them by index order
    x[2, :] = -math.inf
    x[2, 33] = 1.0                                 # a single candidate
    x[3, :] = 0.5                                  # all tied: top-k takes the lowest indices
    x[4, :] = 0.5
    x[5, :] = -math.inf                            # nothing: greedy index 0
    x[6, 1::2] = float("nan")
    rows = [_row(top_p=0.9), _row(row_key=1), _row(top_k=3, row_key=2), _row(top_k=5, row_key=3), _row(top_p=0.5, row_key=4), _row(row_key=5),
            _row(min_p=0.2, top_k=50, row_key=6)]
    check_rows(sampler, x, rows, label="special")


def test_sampled_extreme_parameters(sampler):
    """top_k at and beyond the candidate count, top_k 1, tiny top_p, min_p 1, tiny min_p, tiny and huge temperatures."""
    N = 20000
    g = torch.Generator().manual_seed(4)
    x = torch.randn(9, N, generator=g) * 3.0
    x[0, N // 2:] = -math.inf
    rows = [_row(top_k=N // 2), _row(top_k=N, row_key=1), _row(top_k=1, row_key=2), _row(top_p=1e-6, row_key=3), _row(min_p=1.0, row_key=4),
            _row(min_p=1e-6, top_p=0.99, row_key=5), _row(temperature=1e-30, row_key=6), _row(temperature=1e6, top_k=100, row_key=7),
            _row(temperature=1e-4, top_p=0.99, row_key=8)]
    check_rows(sampler, x, rows, label="extreme")


def test_bf16_ties_split_by_top_k(sampler):
    """bf16 logits from a handful of values: top-k and top-p boundaries fall inside runs of equal values and must keep
    the lowest indices."""
    N = 50000
    g = torch.Generator().manual_seed(5)
    vals = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0])
    x = vals[torch.randint(0, 5, (4, N), generator=g)].to(torch.bfloat16)
    rows = [_row(top_k=1000), _row(top_k=7, row_key=1), _row(top_p=0.3, row_key=2), _row(min_p=0.5, top_k=20000, row_key=3)]
    check_rows(sampler, x, rows, label="bf16 ties")


def test_many_touched_tokens(sampler):
    """Histories that touch more tokens per block than the patch capacity (1,024: the resolver rebuilds the block from
    the lists), than the scan's token list (1,152: processed in place; short histories list from a bitmap, long ones
    from the table words) and than the resolver's compacted list (2,048: processed in place)."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, V, generator=g) * 2.0
    h1 = torch.randint(0, V, (60000,), generator=g).tolist()          # ~1,900 distinct tokens per 8,192-token block
    rows = [_row(repetition=1.3, presence=0.2, gen=h1, top_p=0.9), _row(frequency=0.5, gen=h1, top_k=40, row_key=1)]
    check_rows(sampler, x, rows, label="touched > TCAP")
    N = 16384
    xs = torch.randn(2, N, generator=g) * 2.0
    h2 = torch.randint(0, N, (65000,), generator=g).tolist()          # every token of both blocks touched
    rows = [_row(repetition=1.2, frequency=0.1, gen=h2, top_p=0.8), _row(presence=0.7, gen=h2, min_p=0.05, row_key=1)]
    check_rows(sampler, xs, rows, label="touched > LCAP")
    h3 = torch.randint(0, 8192, (6000,), generator=g).tolist()         # a short history: ~4,300 distinct tokens in block 0
    rows = [_row(repetition=1.1, presence=0.3, gen=h3, top_p=0.9), _row(frequency=0.4, prompt=h3[:100], gen=h3[100:], top_k=50, row_key=1)]
    check_rows(sampler, x, rows, label="short history, touched > list")


def _whole_bin_case():
    """Peaked rows (background ~N(-6, 1), eight levels of 1-6 equal values at random positions) and their parameters."""
    N = 6 * 8192
    g = torch.Generator().manual_seed(21)
    xs, rows = [], []
    for b in range(48):
        x = torch.randn(N, generator=g) - 6.0
        kind = b % 4
        counts = [1] * 8 if kind == 2 else torch.randint(1, 7, (8,), generator=g).tolist()
        pos = torch.randperm(N, generator=g)
        p = 0
        for j, c in enumerate(counts):
            x[pos[p:p + c]] = 9.0 - 0.37 * j  # levels about half a power of two apart at T = 1
            p += c
        cum = np.cumsum(counts).tolist()
        j = int(torch.randint(0, 7, (1,), generator=g))
        T = float(0.5 + torch.rand(1, generator=g))
        base = dict(temperature=T, seed=100 + b, position=7 * b + 1, row_key=b % 5)
        if kind == 0:    # top-k at the end of a level: its bin kept whole
            rows.append(_row(top_k=cum[j], **base))
        elif kind == 1:  # top-k inside a level when it has several elements (selected, lowest indices first)
            k = cum[j] - 1 if counts[j] > 1 else cum[j]
            rows.append(_row(top_k=k, top_p=0.9, **base))
        elif kind == 2:  # top-p over single-element levels
            rows.append(_row(top_p=float(0.2 + 0.7 * torch.rand(1, generator=g)), **base))
        else:            # min-p (cut far below; or just below level j, in its fine bin, where min-p alone keeps levels 0..j),
                         # top-k at level j's end, top-p
            mp = 0.02 if b % 8 == 3 else 0.999 * 2.0 ** (-0.37 * j / T * math.log2(math.e))
            rows.append(_row(min_p=mp, top_k=cum[j], top_p=0.85, **base))
        xs.append(x)
    return torch.stack(xs), rows


def test_whole_cut_bins(sampler):
    """Peaked rows whose top-k / top-p boundary ends a fine bin, so that every kept element of the cut's bin stays kept
    (the resolver takes such a bin whole from the row bins instead of gathering and selecting it), with the bin's
    equal elements spread over several blocks; and, beside them, boundaries inside a run of equal values.  Survivor
    sets, probabilities and the token of every row (each its own draw position) against the oracle."""
    x, rows = _whole_bin_case()
    check_rows(sampler, x, rows, label="whole bins")


def test_no_cut_wide_rows(sampler):
    """Rows without any cut (top-k 0, top-p 1, min-p 0) whose candidates span more than 36 powers of two (N(0,5) at
    T 1.2): the fine bin just past the weight window (36 powers below the row's top) holds candidates in most blocks,
    and with no cut it must weigh nothing in the draw's block rescan (regression: it once took a shifted weight)."""
    g = torch.Generator().manual_seed(15)
    x = torch.randn(8, V, generator=g) * 5.0
    rows = [_row(temperature=1.2, seed=40 + b, position=3 * b, row_key=b) for b in range(8)]
    check_rows(sampler, x, rows, label="no cut, wide")


def test_listed_and_staged_draws_agree(sampler):
    """The draw inside the drawn block from its listed elements (taken when the block's whole kept set lies in its list:
    small top-k sets, min-p cuts high up, rows whose weight window holds fewer candidates than top-k) against the draw
    from a rescan of the block (QWS_TF_STAGED_DRAW), over 40 draw positions per row; the first two positions of every
    row against the oracle as well."""
    g = torch.Generator().manual_seed(33)
    x = torch.randn(16, V, generator=g) * 3.0
    rows = []
    for b, k in enumerate((1, 2, 5, 20, 40, 50, 64, 100)):  # peaked rows, small top-k (with and without top-p)
        rows.append(_row(temperature=0.6, top_k=k, top_p=0.9 if b % 2 else 1.0, seed=60 + b, row_key=b))
    for b in range(4):  # a few strongly biased tokens: fewer weighted candidates than top_k (no cut)
        ids = torch.randint(0, V, (12,), generator=g).tolist()
        bias = {i: float(60.0 + 3.0 * j) for j, i in enumerate(ids)}
        rows.append(_row(temperature=0.6, top_k=50, bias=bias, seed=70 + b, row_key=8 + b))
    for b in range(4):  # min-p high up, alone or with top-k / top-p
        rows.append(_row(temperature=0.8, min_p=[0.3, 0.05, 0.5, 0.1][b], top_k=[0, 30, 0, 10][b], top_p=[1.0, 1.0, 0.7, 0.95][b],
                         seed=80 + b, row_key=12 + b))
    lg = x.cuda()
    for pos in range(40):
        rs = [copy.copy(r) for r in rows]
        for r in rs:
            r.position = pos
        listed = sampler.sample(lg, rs).cpu().tolist()
        staged = sampler.sample(lg, _with_flags(rs, q.TF_STAGED_DRAW)).cpu().tolist()
        assert listed == staged, f"position {pos}: listed {listed} staged {staged}"
        if pos < 2:
            check_rows(sampler, x, rs, dense=False, label=f"listed draw, position {pos}")


def test_fused_and_split_cut_selections_agree(sampler):
    """The cut bin gathered and selected in one pass when every block lists its part of it (flat rows ~N(0, 0.5): the
    bin holds hundreds to a thousand elements) against the oracle and against the separate gather and selection
    (QWS_TF_SPLIT_SELECT), for top-p and top-k cuts in fp32 and bf16.  In the bf16 rows each value is shared by
    hundreds of tokens, so the bucket where the prefix crosses holds more than a wave of elements and the selection
    goes on with more rounds.  No row rescans a block (out_info 0), so the one-pass selection ran."""
    g = torch.Generator().manual_seed(44)
    params = [dict(top_p=0.95), dict(top_p=0.5), dict(top_k=5000), dict(top_k=1000, top_p=0.9), dict(top_k=1000),
              dict(top_p=0.7, temperature=0.8)]
    for dt in (torch.float32, torch.bfloat16):
        x = (torch.randn(len(params), V, generator=g) * 0.5).to(dt)
        rows = [_row(seed=90 + b, row_key=b, position=5 + b, **p) for b, p in enumerate(params)]
        info = check_rows(sampler, x, rows, label=f"one-pass cut {dt}")
        assert all(int(i) == 0 for i in info), f"{dt}: out_info {info.tolist()}"
        lg = x.cuda()
        for pos in range(8):
            rs = [copy.copy(r) for r in rows]
            for r in rs:
                r.position = pos
            fused = sampler.sample(lg, rs).cpu().tolist()
            split = sampler.sample(lg, _with_flags(rs, q.TF_SPLIT_SELECT)).cpu().tolist()
            assert fused == split, f"{dt} position {pos}: one pass {fused} separate {split}"
