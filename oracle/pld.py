"""CPU restatement of the reference's prompt-lookup (PLD) tail proposer -- TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).  Restates engine/include/pld.h:13-39 and engine/src/pld.cu:32-121.

State: the committed history S (its last token is the anchor) and, for every position e >= n - 1 of S, the
n-gram S[e - n + 1 .. e] (engine/src/pld.cu:36-41, index_end; drafts are never indexed).

propose(drafts, max_tail, min_len) (engine/src/pld.cu:88-119):
  K = S ++ drafts, end = len(S) - 1 + len(drafts); nothing when len(S) == 0 or end + 1 < n.
  Query = K[end - n + 1 .. end].  Candidates = end positions j of that n-gram in S with j < end, most recent
  first; at most `cap` of them are examined (only the first when longest = 0).
  Agreement l = n, extended while l < back and j - l >= 0 and K[j - l] == K[end - l].
  Best = largest l, ties to the most recent candidate.  l_out = best l (0 without a candidate).
  The tail is K[j + 1 .. min(j + 1 + max_tail, end + 1) - 1] when best l >= min_len, else empty.

Configuration clamps (engine/src/pld.cu:54-62): n in [1, 4], max_tail in [0, 7], cap >= 1, back >= 1,
longest in {0, 1}; defaults n 2, min_len 3, max_tail 4, cap 64, back 64, longest 1 (pld.cu:45-52).
"""
from collections import defaultdict
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple


@dataclass
class PldCfg:
    n: int = 2
    min_len: int = 3
    max_tail: int = 4
    cap: int = 64
    back: int = 64
    longest: int = 1

    def clamped(self) -> "PldCfg":
        return PldCfg(n=min(4, max(1, self.n)), min_len=self.min_len, max_tail=min(7, max(0, self.max_tail)), cap=max(1, self.cap),
                      back=max(1, self.back), longest=1 if self.longest else 0)


class Pld:
    def __init__(self, cfg: Optional[PldCfg] = None):
        self.c = (cfg or PldCfg()).clamped()
        self.S: List[int] = []
        self.idx = defaultdict(list)  # n-gram tuple -> ascending end positions

    def reset(self, ctx: Sequence[int]):
        self.S, self.idx = [], defaultdict(list)
        self.append(ctx)

    def append(self, toks: Sequence[int]):
        n = self.c.n
        for t in toks:
            self.S.append(int(t))
            e = len(self.S) - 1
            if e >= n - 1:
                self.idx[tuple(self.S[e - n + 1:e + 1])].append(e)

    def propose(self, drafts: Sequence[int] = (), max_tail: Optional[int] = None, min_len: Optional[int] = None) -> Tuple[List[int], int]:
        """(tail tokens, agreement length l_out)."""
        c = self.c
        max_tail = c.max_tail if max_tail is None else max_tail
        min_len = c.min_len if min_len is None else min_len
        pa = len(self.S) - 1
        if pa < 0:
            return [], 0
        K = self.S + [int(d) for d in drafts]
        end = len(K) - 1
        n = c.n
        if end + 1 < n:
            return [], 0
        occ = self.idx.get(tuple(K[end - n + 1:end + 1]), [])
        lim = c.cap if c.longest else 1
        best_j, best_l, seen = -1, -1, 0
        for j in reversed(occ):
            if j >= end:
                continue
            if seen >= lim:
                break
            seen += 1
            l = n
            while l < c.back and j - l >= 0 and K[j - l] == K[end - l]:
                l += 1
            if l > best_l:
                best_j, best_l = j, l
        l_out = max(best_l, 0)
        if best_l < min_len:
            return [], l_out
        return K[best_j + 1:min(best_j + 1 + max_tail, end + 1)], l_out
