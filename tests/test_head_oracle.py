"""The quantised head's select + rescore oracle (oracle/head.py) pinned without a GPU: known answers for the key
order (ties to the lower index, -0 below +0, NaN never), the candidate list against a brute-force rank count, and the
float64 rescore against a plain float64 matmul, with every fp32 accumulation order inside its stated bound."""
import numpy as np
import torch

from oracle import head as H


def test_known_answers():
    v = np.array([1.0, 3.0, 3.0, np.nan, 2.0], dtype=np.float32)
    assert H.candidates(v, 3).tolist() == [1, 2, 4]
    assert H.candidates(v, 6).tolist() == [1, 2, 4, 0, -1, -1]
    z = np.array([-0.0, 0.0, -1.0], dtype=np.float32)
    assert H.candidates(z, 3).tolist() == [1, 0, 2]  # +0 ranks above -0
    assert H.candidates(np.array([np.nan] * 4, dtype=np.float32), 2).tolist() == [-1, -1]
    inf = np.array([-np.inf, 5.0, np.inf], dtype=np.float32)
    assert H.candidates(inf, 3).tolist() == [2, 1, 0]


def test_candidates_match_brute_force_rank():
    rng = np.random.default_rng(7)
    for trial in range(30):
        n = int(rng.integers(1, 300))
        v = (np.round(rng.normal(size=n) * 3) / 3).astype(np.float32)  # many ties
        v[rng.random(n) < 0.1] = np.nan
        R = int(rng.integers(1, 70))
        c = H.candidates(v, R)
        # brute force: a valid element's rank = the valid elements ahead of it: a larger value, +0 against -0, or the
        # same value and sign at a lower index
        sb = np.signbit(v)

        def ahead(j, i):
            if v[j] != v[i]:
                return v[j] > v[i]
            if sb[j] != sb[i]:
                return sb[i]
            return j < i

        ranks = {}
        for i in range(n):
            if np.isnan(v[i]):
                continue
            ranks[i] = sum(1 for j in range(n) if not np.isnan(v[j]) and j != i and ahead(j, i))
        want = [i for i, r in sorted(ranks.items(), key=lambda kv: kv[1]) if r < R]
        assert c[: len(want)].tolist() == want and (c[len(want):] == -1).all()


def test_rescore_and_bound():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(8, 5120, generator=g).to(torch.bfloat16)
    x = torch.randn(5120, generator=g).to(torch.bfloat16)
    ex, tol = H.exact_logits(w, x)
    ref = (w.double() @ x.double()).numpy()
    assert np.array_equal(ex, ref)
    prod = (w.float() * x.float()).numpy()  # bf16 x bf16 products are exact in fp32
    for r in range(8):
        for order in (np.arange(5120), np.random.default_rng(r).permutation(5120)):
            acc = np.float32(0.0)
            for k in order:
                acc = np.float32(acc + prod[r, k])
            assert abs(float(acc) - ex[r]) <= tol[r]
