"""The PLD proposer oracle (oracle/pld.py) pinned two ways, without a GPU: hand-derived cases of the algorithm's
definition (agreement, longest vs most recent, back / cap limits, the min_len gate, tails running into the drafts),
and bit-equality with the reference's own proposer built from its source (oracle/build_ref.sh ->
oracle/_ref/libpld_ref.so, engine/src/pld.cu) on randomized histories, configurations and draft tails."""
import ctypes as C
import random
from pathlib import Path

import pytest

from oracle.pld import Pld, PldCfg

REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libpld_ref.so"


class _Cfg(C.Structure):  # engine/include/pld.h:13-20
    _fields_ = [(k, C.c_int) for k in ("n", "min_len", "max_tail", "cap", "back", "longest")]


class RefPld:
    """ctypes handle on the reference proposer (engine/include/pld.h:22-39)."""

    def __init__(self, lib, cfg: PldCfg):
        self.lib = lib
        c = _Cfg(cfg.n, cfg.min_len, cfg.max_tail, cfg.cap, cfg.back, cfg.longest)
        self.p = lib.smk_pld_create(C.byref(c))

    def __del__(self):
        self.lib.smk_pld_destroy(self.p)

    def reset(self, ctx):
        a = (C.c_int * max(1, len(ctx)))(*ctx)
        self.lib.smk_pld_reset(self.p, a, len(ctx))

    def append(self, toks):
        a = (C.c_int * max(1, len(toks)))(*toks)
        self.lib.smk_pld_append(self.p, a, len(toks))

    def propose(self, drafts, max_tail, min_len):
        d = (C.c_int * max(1, len(drafts)))(*drafts)
        out = (C.c_int * 8)()
        l = C.c_int(-5)
        k = self.lib.smk_pld_propose_ex(self.p, d, len(drafts), max_tail, min_len, out, C.byref(l))
        return list(out[:k]), l.value


@pytest.fixture(scope="module")
def ref():
    if not REF.exists():  # build the checker on demand where the reference sources are present (this container)
        import subprocess
        subprocess.run(["bash", str(REF.parents[1] / "build_ref.sh")], check=False, capture_output=True)
    if not REF.exists():
        pytest.skip("oracle/_ref/libpld_ref.so not built (oracle/build_ref.sh needs the reference sources)")
    lib = C.CDLL(str(REF))
    lib.smk_pld_create.restype = C.c_void_p
    lib.smk_pld_create.argtypes = [C.c_void_p]
    lib.smk_pld_destroy.argtypes = [C.c_void_p]
    lib.smk_pld_reset.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.smk_pld_append.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.smk_pld_propose_ex.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.smk_pld_propose_ex.restype = C.c_int
    return lib


def _pld(ctx, **kw):
    p = Pld(PldCfg(**kw))
    p.reset(ctx)
    return p


def test_hand_derived_cases():
    # the anchor's own n-gram never matches itself; the only earlier (1, 2) ends at 1 and cannot extend left
    assert _pld([1, 2, 3, 9, 1, 2]).propose([]) == ([], 2)
    assert _pld([1, 2, 3, 9, 1, 2]).propose([], min_len=2) == ([3, 9, 1, 2], 2)
    # a draft extends the query: (2, 3) ends at 2, agreement 3 (K[0] == K[4]); the tail runs to the draft
    assert _pld([1, 2, 3, 9, 1, 2]).propose([3]) == ([9, 1, 2, 3], 3)
    assert _pld([1, 2, 3, 9, 1, 2]).propose([3], max_tail=2) == ([9, 1], 3)
    S = [5, 1, 2, 8, 7, 1, 2, 8, 5, 1, 2]
    # (1, 2) ends at 6 (agreement 2: 7 != 5) and at 2 (agreement 3: 5 == 5): the longest wins
    assert _pld(S).propose([]) == ([8, 7, 1, 2], 3)
    # only the most recent candidate: longest = 0, or cap = 1
    assert _pld(S, longest=0).propose([]) == ([], 2)
    assert _pld(S, cap=1).propose([]) == ([], 2)
    # back = 2 caps both agreements at 2: the tie goes to the most recent (j = 6), gated by min_len
    assert _pld(S, back=2).propose([]) == ([], 2)
    assert _pld(S, back=2).propose([], min_len=2) == ([8, 5, 1, 2], 2)
    # n = 1: the 4 at 2 agrees back to position 0 (l = 3); its tail ends at the anchor
    assert _pld([4, 6, 4, 6, 4], n=1).propose([], min_len=1) == ([6, 4], 3)
    # n = 3 keys; no candidate at all; empty history
    assert _pld([1, 2, 3, 4, 1, 2, 3], n=3).propose([]) == ([4, 1, 2, 3], 3)
    assert _pld([1, 2, 3]).propose([7]) == ([], 0)
    assert Pld().propose([1, 2]) == ([], 0)
    # appended tokens are indexed: (9, 9) appears once the history grows
    p = _pld([9, 9, 5])
    p.append([9, 9])
    assert p.propose([], min_len=2) == ([5, 9, 9], 2)


CFGS = [PldCfg(), PldCfg(n=1, min_len=1, max_tail=7), PldCfg(n=3, min_len=3, max_tail=2, cap=5, back=9), PldCfg(n=4, min_len=4, cap=2, back=4),
        PldCfg(longest=0, min_len=2), PldCfg(n=2, min_len=0, max_tail=7, cap=1000, back=200), PldCfg(n=0, max_tail=12, cap=0, back=0)]


@pytest.mark.parametrize("ci", range(len(CFGS)))
def test_oracle_matches_reference_build(ref, ci):
    cfg = CFGS[ci]
    rng = random.Random(1234 + ci)
    for trial in range(12):
        alpha = rng.choice([3, 5, 12, 60])
        ctx = [rng.randrange(alpha) for _ in range(rng.randrange(0, 400))]
        mine, theirs = Pld(cfg), RefPld(ref, cfg)
        mine.reset(ctx)
        theirs.reset(ctx)
        for step in range(40):
            nd = rng.randrange(0, 8)
            drafts = [rng.randrange(alpha) for _ in range(nd)]
            mt, ml = rng.randrange(0, 9), rng.randrange(0, 7)
            assert mine.propose(drafts, mt, ml) == theirs.propose(drafts, mt, ml), (ci, trial, step)
            toks = [rng.randrange(alpha) for _ in range(rng.randrange(1, 5))]
            mine.append(toks)
            theirs.append(toks)
