"""CPU restatement of the sampling stage (TEST INFRASTRUCTURE ONLY: see oracle/__init__.py).

The definition this module fixes, and which the HIP library reproduces bit for bit
----------------------------------------------------------------------------------
V tokens, one row of logits `x_raw` (fp32, or bf16 widened exactly to fp32).

1. Processors (engine/src/proc.h:39-49 proc_logit; order engine/src/proc.h:4-5, docs/USAGE.md:92-93).
   NaN logits become -inf first (a deliberate rule: the reference's key order lets a NaN win,
   engine/src/mtp_sample.cu:31-35, while its argmax never picks one, engine/src/misc.cu:54).
   A row's processors are "on" iff presence != 0, frequency != 0, repetition != 1, min_tokens > 0,
   or a bias / allowed list / banned mask is given (engine/src/proc.cu:149).  When on, per token, in
   this order, every operation an IEEE fp32 operation rounded to nearest, no fused multiply-add:
     banned bit set (banned mask) or not allowed (allowed list)  -> -inf
     min_tokens > ngen and token is a stop id                    -> -inf
     x = x + bias                                   (bias = 0 where unset)
     repetition != 1 and (token in prompt or count > 0): x = x > 0 ? x / rep : x * rep
     count > 0: x = x - frequency * count; x = x - presence
   `count` = occurrences among the generated tokens (plus, for verify row t, the drafts d_1..d_t;
   engine/src/proc.cu:24, tests/test_logit_procs.py:40), `ngen` = generated tokens so far (+ t).
2. Rank order: key = ord32(x + 0.0f) (order-preserving bits, -0 folded into +0), larger key first,
   then lower index first (engine/src/mtp_sample.cu:31-35, engine/src/misc.cu:54).
   Greedy (temperature <= 0): the first token in rank order.
3. Sampling.  Candidates = tokens with x != -inf (none: the greedy token).
     inv_t = 1.0f / temperature (fp32, engine/src/mtp_sample.cu:377)
     kappa = (float)((double)inv_t * LOG2E)        (one rounding)
     a_i   = clamp(x_i * kappa, -2^22, 2^22)       (fp32; x_i / T in log2 units)
     q_i   = (int)floor(a_i * 256),  r_i = a_i * 256 - floor(a_i * 256) in [0, 1)
     n_i   = q_i >> 8 (= floor(a_i)),  fine bin = q_i >> 2 (= floor(a_i * 64))
     m_i   = TAB[q_i & 255] * (1 + r_i * (C1 + r_i * C2))   fp32, one rounding per operation;
             TAB[j] = fp32(2^(j/256)), C1 = fp32(ln2 / 256), C2 = fp32((ln2 / 256)^2 / 2)
     mu_i  = (uint32)(m_i * 2^23)                  (24-bit mantissa of 2^(a_i - n_i))
     a_max = a of the first candidate, N = floor(a_max)
   min_p > 0: keep candidates with a_i >= a_cut, a_cut = (float)((double)a_max + log2(min_p))
              (log2 from libm, once per row) -- p_i >= min_p * p_max (vLLM min_p, before top-k).
   top-k (K > 0): keep the first K remaining candidates in rank order.
   weight w_i = mu_i * 2^(n_i - N + 38) if n_i >= N - 38 else 0    (exact integer < 2^63;
              the dropped tail is below 2^-37 of the top token's weight)
   S = sum of w over the kept candidates (exact integer).
   top-p (top_p < 1): TP = floor(top_p * 2^32), thr = ceil(TP * S / 2^32); keep the candidates in
              rank order up to and including the first position whose inclusive prefix sum is
              >= thr  (= "keep token i iff the mass before it is < top_p", at least one:
              engine/src/mtp_sample.cu:163-169, tests/test_logit_procs.py:250-251).
   S2 = sum of the kept weights.  Probabilities p_i = w_i / S2.
   Draw: (r0, r1, r2, r3) = Philox4x32-10(counter = (position, stream, row_key, 0),
              key = (seed_lo, seed_hi)); u24 = r0 >> 8 (engine/src/mtp_sample.cu:24-27);
              t = floor(u24 * S2 / 2^24); token = the smallest kept INDEX whose prefix sum of kept
              weights, in index order, exceeds t.
4. Speculative verify (engine/src/mtp_sample.cu:227-258), per sequence with drafts d_1..d_K and
   draft probabilities q_t over a reduced vocabulary mapped to token ids by an injective table:
     for t in 0..K-1, row t's distribution (kept set, w, S2_t); Q_i = floor(q_t(i) * S2_t) exactly;
       (r0, r1) = Philox(counter = (position, ACCEPT + t, row_key, 0));
       accept d_{t+1} iff (r0 >> 8) * Q_d < w_d * 2^24   (u * q(d) < p(d); w_d = 0 if not kept);
       else residual r_i = max(0, w_i - Q_i) over the kept set (R = 0, or test flag bit0: r = w),
            draw from r in index order with u24 = r1 >> 8, emit t + 1 tokens, stop;
     all accepted: bonus token from row K with u24 = Philox(position, ACCEPT + K).r1 >> 8.

Everything above is integer or correctly rounded IEEE arithmetic, so the CPU and the GPU agree
exactly.  The weights approximate exp((x_i - x_max) / T) to ~1.4e-7 relative error.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

# Philox4x32-10 (Random123's published constants; engine/src/mtp_sample.cu:13-20)
PHILOX_M0, PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
PHILOX_W0, PHILOX_W1 = 0x9E3779B9, 0xBB67AE85
# rng streams = counter word 1 (engine/src/mtp_sample.h:45)
ST_ACCEPT, ST_DRAFT, ST_FIRST, ST_DRAW = 0x1000, 0x2000, 0x3000, 0x4000

LOG2E = 1.4426950408889634  # fp64 log2(e) = 0x1.71547652b82fep+0
A_CLAMP = float(2 ** 22)
D_EXP = 38  # weights below 2^-38 of the top exponent are dropped
# TAB[j] = fp32(2^(j/256)), j = 0..255, and the quadratic 2^(r/256) ~ 1 + r * (C1 + r * C2) on r in [0, 1)
TAB = np.array([
    0x3f800000, 0x3f8058d8, 0x3f80b1ed, 0x3f810b41, 0x3f8164d2, 0x3f81bea1, 0x3f8218af, 0x3f8272fc,
    0x3f82cd87, 0x3f832850, 0x3f838359, 0x3f83dea1, 0x3f843a29, 0x3f8495f0, 0x3f84f1f6, 0x3f854e3d,
    0x3f85aac3, 0x3f86078a, 0x3f866491, 0x3f86c1d9, 0x3f871f62, 0x3f877d2b, 0x3f87db35, 0x3f883981,
    0x3f88980f, 0x3f88f6dd, 0x3f8955ee, 0x3f89b541, 0x3f8a14d5, 0x3f8a74ad, 0x3f8ad4c6, 0x3f8b3523,
    0x3f8b95c2, 0x3f8bf6a4, 0x3f8c57ca, 0x3f8cb933, 0x3f8d1adf, 0x3f8d7cd0, 0x3f8ddf04, 0x3f8e417d,
    0x3f8ea43a, 0x3f8f073b, 0x3f8f6a81, 0x3f8fce0c, 0x3f9031dc, 0x3f9095f2, 0x3f90fa4d, 0x3f915eed,
    0x3f91c3d3, 0x3f922900, 0x3f928e72, 0x3f92f42c, 0x3f935a2b, 0x3f93c072, 0x3f9426ff, 0x3f948dd4,
    0x3f94f4f0, 0x3f955c53, 0x3f95c3ff, 0x3f962bf2, 0x3f96942d, 0x3f96fcb1, 0x3f97657d, 0x3f97ce92,
    0x3f9837f0, 0x3f98a197, 0x3f990b88, 0x3f9975c2, 0x3f99e046, 0x3f9a4b13, 0x3f9ab62b, 0x3f9b218d,
    0x3f9b8d3a, 0x3f9bf931, 0x3f9c6573, 0x3f9cd201, 0x3f9d3eda, 0x3f9dabfe, 0x3f9e196e, 0x3f9e872a,
    0x3f9ef532, 0x3f9f6387, 0x3f9fd228, 0x3fa04116, 0x3fa0b051, 0x3fa11fd9, 0x3fa18faf, 0x3fa1ffd2,
    0x3fa27043, 0x3fa2e102, 0x3fa3520f, 0x3fa3c36b, 0x3fa43516, 0x3fa4a70f, 0x3fa51958, 0x3fa58bef,
    0x3fa5fed7, 0x3fa6720e, 0x3fa6e595, 0x3fa7596c, 0x3fa7cd94, 0x3fa8420c, 0x3fa8b6d5, 0x3fa92bef,
    0x3fa9a15b, 0x3faa1718, 0x3faa8d26, 0x3fab0387, 0x3fab7a3a, 0x3fabf13f, 0x3fac6897, 0x3face041,
    0x3fad583f, 0x3fadd090, 0x3fae4934, 0x3faec22d, 0x3faf3b79, 0x3fafb519, 0x3fb02f0e, 0x3fb0a957,
    0x3fb123f6, 0x3fb19ee9, 0x3fb21a32, 0x3fb295d0, 0x3fb311c4, 0x3fb38e0e, 0x3fb40aaf, 0x3fb487a6,
    0x3fb504f3, 0x3fb58298, 0x3fb60094, 0x3fb67ee7, 0x3fb6fd92, 0x3fb77c95, 0x3fb7fbf0, 0x3fb87ba3,
    0x3fb8fbaf, 0x3fb97c14, 0x3fb9fcd2, 0x3fba7dea, 0x3fbaff5b, 0x3fbb8126, 0x3fbc034a, 0x3fbc85ca,
    0x3fbd08a4, 0x3fbd8bd8, 0x3fbe0f68, 0x3fbe9353, 0x3fbf179a, 0x3fbf9c3c, 0x3fc0213b, 0x3fc0a695,
    0x3fc12c4d, 0x3fc1b261, 0x3fc238d2, 0x3fc2bfa1, 0x3fc346cd, 0x3fc3ce57, 0x3fc4563f, 0x3fc4de85,
    0x3fc5672a, 0x3fc5f02e, 0x3fc67991, 0x3fc70353, 0x3fc78d75, 0x3fc817f7, 0x3fc8a2d8, 0x3fc92e1b,
    0x3fc9b9be, 0x3fca45c1, 0x3fcad226, 0x3fcb5eed, 0x3fcbec15, 0x3fcc799f, 0x3fcd078c, 0x3fcd95da,
    0x3fce248c, 0x3fceb3a1, 0x3fcf4319, 0x3fcfd2f4, 0x3fd06334, 0x3fd0f3d7, 0x3fd184df, 0x3fd2164c,
    0x3fd2a81e, 0x3fd33a54, 0x3fd3ccf1, 0x3fd45ff3, 0x3fd4f35b, 0x3fd58729, 0x3fd61b5e, 0x3fd6affa,
    0x3fd744fd, 0x3fd7da67, 0x3fd87039, 0x3fd90673, 0x3fd99d16, 0x3fda3421, 0x3fdacb94, 0x3fdb6371,
    0x3fdbfbb8, 0x3fdc9468, 0x3fdd2d82, 0x3fddc706, 0x3fde60f5, 0x3fdefb4e, 0x3fdf9613, 0x3fe03143,
    0x3fe0ccdf, 0x3fe168e7, 0x3fe2055b, 0x3fe2a23c, 0x3fe33f89, 0x3fe3dd44, 0x3fe47b6d, 0x3fe51a03,
    0x3fe5b907, 0x3fe65879, 0x3fe6f85b, 0x3fe798ab, 0x3fe8396a, 0x3fe8da99, 0x3fe97c38, 0x3fea1e47,
    0x3feac0c7, 0x3feb63b7, 0x3fec0719, 0x3fecaaec, 0x3fed4f30, 0x3fedf3e7, 0x3fee9910, 0x3fef3eab,
    0x3fefe4ba, 0x3ff08b3b, 0x3ff13231, 0x3ff1d99a, 0x3ff28177, 0x3ff329c9, 0x3ff3d290, 0x3ff47bcc,
    0x3ff5257d, 0x3ff5cfa4, 0x3ff67a41, 0x3ff72555, 0x3ff7d0df, 0x3ff87ce1, 0x3ff9295a, 0x3ff9d64a,
    0x3ffa83b3, 0x3ffb3194, 0x3ffbdfed, 0x3ffc8ec0, 0x3ffd3e0c, 0x3ffdedd2, 0x3ffe9e11, 0x3fff4ecb,
], dtype=np.uint32).view(np.float32)
C1 = np.array([0x3B317218], dtype=np.uint32).view(np.float32)[0]
C2 = np.array([0x3675FDF0], dtype=np.uint32).view(np.float32)[0]
_MASK32 = np.uint64(0xFFFFFFFF)


# ---------------------------------------------------------------------------------------------- Philox4x32-10
def philox(c0, c1, c2, c3, k0, k1):
    """Philox4x32-10 (engine/src/mtp_sample.cu:10-23), vectorised over numpy arrays (any broadcastable
    shapes of uint32 values).  Returns four uint64 arrays holding the 32-bit output words."""
    c = [np.asarray(v, dtype=np.uint64) & _MASK32 for v in (c0, c1, c2, c3)]
    k0 = np.asarray(k0, dtype=np.uint64) & _MASK32
    k1 = np.asarray(k1, dtype=np.uint64) & _MASK32
    m0, m1 = np.uint64(PHILOX_M0), np.uint64(PHILOX_M1)
    for _ in range(10):
        p0 = m0 * c[0]  # < 2^64: exact in uint64
        p1 = m1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & _MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & _MASK32
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(PHILOX_W0)) & _MASK32
        k1 = (k1 + np.uint64(PHILOX_W1)) & _MASK32
    return tuple(c)


def draw_u24(seed: int, position, stream, row_key=0, word: int = 0):
    """24-bit uniform integer of the draw at counter (position, stream, row_key, 0), key = seed
    (engine/src/mtp_sample.cu:24-27: u01(x) = (x >> 8) * 2^-24).  word 0 = .x, 1 = .y."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    r = philox(position, stream, row_key, 0, seed & 0xFFFFFFFF, seed >> 32)
    return r[word] >> np.uint64(8)


# ---------------------------------------------------------------------------------------------- processors
@dataclass
class RowProcs:
    """One row's request-level logit processors: include/engine.h smk_procs (engine/include/engine.h:142-154)
    plus the row's history, which the reference keeps on the device (engine/src/proc.h:16-25).
    `gen` = generated tokens (frequency / presence counts, repetition set), `prompt` = prompt tokens
    (repetition set only), `ngen` = tokens generated so far (default len(gen)), `banned` = bit-packed
    uint32 mask, bit (id & 31) of word (id >> 5) set = banned."""
    presence: float = 0.0
    frequency: float = 0.0
    repetition: float = 1.0
    min_tokens: int = 0
    prompt: Sequence[int] = ()
    gen: Sequence[int] = ()
    ngen: Optional[int] = None
    bias: Optional[dict] = None
    allowed: Optional[Sequence[int]] = None
    banned: Optional[np.ndarray] = None
    stop: Sequence[int] = ()

    def active(self) -> bool:
        """engine/src/proc.cu:149: any elementwise processor active."""
        return bool(self.presence != 0.0 or self.frequency != 0.0 or self.repetition != 1.0 or self.min_tokens > 0
                    or self.bias or self.allowed or self.banned is not None)


def f32(v) -> np.float32:
    return np.float32(v)


def widen(logits: torch.Tensor) -> torch.Tensor:
    """fp32 or bf16 logits -> fp32 (exact), NaN -> -inf."""
    x = logits.detach().to("cpu").float().clone()
    x[torch.isnan(x)] = -math.inf
    return x


def process(logits: torch.Tensor, procs: Optional[RowProcs], drafts_before: Sequence[int] = ()) -> torch.Tensor:
    """Processed logits of one row (engine/src/proc.h:39-49).  `drafts_before` = the draft tokens of the
    verify rows before this one, counted as generated (engine/src/proc.cu:24)."""
    x = widen(logits)
    if procs is None or not procs.active():
        return x
    V = x.numel()
    neg = torch.tensor(-math.inf, dtype=torch.float32)
    if procs.allowed:
        keep = torch.zeros(V, dtype=torch.bool)
        keep[torch.as_tensor(list(procs.allowed), dtype=torch.long)] = True
        x = torch.where(keep, x, neg)
    if procs.banned is not None:
        x = torch.where(banned_bits(procs.banned, V), neg, x)
    hist = list(procs.gen) + list(drafts_before)
    ngen = (len(procs.gen) if procs.ngen is None else int(procs.ngen)) + len(drafts_before)
    if procs.min_tokens > ngen and len(procs.stop):
        x[torch.as_tensor(list(procs.stop), dtype=torch.long)] = neg
    bias = torch.zeros(V, dtype=torch.float32)
    if procs.bias:
        ids = torch.as_tensor(list(procs.bias.keys()), dtype=torch.long)
        bias[ids] = torch.as_tensor(np.array(list(procs.bias.values()), dtype=np.float32))
    x = x + bias  # every token: -0 + 0 = +0, as __fadd_rn(x, 0) in the reference
    counts = torch.bincount(torch.as_tensor(hist, dtype=torch.long), minlength=V) if hist else torch.zeros(V, dtype=torch.long)
    rep = torch.tensor(f32(procs.repetition))
    if f32(procs.repetition) != f32(1.0):
        seen = counts > 0
        if len(procs.prompt):
            seen[torch.as_tensor(list(procs.prompt), dtype=torch.long)] = True
        x = torch.where(seen, torch.where(x > 0, x / rep, x * rep), x)
    gen_seen = counts > 0
    cnt = counts.to(torch.float32)
    freq = torch.tensor(f32(procs.frequency))
    pres = torch.tensor(f32(procs.presence))
    x = torch.where(gen_seen, (x - freq * cnt) - pres, x)
    return x


def banned_bits(mask: np.ndarray, V: int) -> torch.Tensor:
    """bool [V] from a bit-packed uint32 mask (bit id & 31 of word id >> 5)."""
    m = np.asarray(mask, dtype=np.uint32)
    ids = np.arange(V)
    return torch.from_numpy(((m[ids >> 5] >> (ids & 31).astype(np.uint32)) & 1).astype(bool))


def pack_bits(ids: Sequence[int], V: int) -> np.ndarray:
    """Bit-packed uint32 mask of ceil(V / 32) words with the given ids set."""
    m = np.zeros((V + 31) // 32, dtype=np.uint32)
    for i in ids:
        m[int(i) >> 5] |= np.uint32(1 << (int(i) & 31))
    return m


# ---------------------------------------------------------------------------------------------- order, greedy
def rank_keys(x: torch.Tensor) -> torch.Tensor:
    """Order-preserving 32-bit keys (int64 tensor) of fp32 values, -0 folded into +0
    (engine/src/mtp_sample.cu:31-35 mkkey's high word)."""
    u = (x + 0.0).view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    neg = (u & 0x80000000) != 0
    return torch.where(neg, (~u) & 0xFFFFFFFF, u | 0x80000000)


def rank_order(x: torch.Tensor, ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Indices (into x) sorted by key descending, index ascending."""
    keys = rank_keys(x)
    idx = torch.arange(x.numel()) if ids is None else ids
    o = np.lexsort((idx.numpy(), -keys.numpy()))
    return torch.from_numpy(o)


def greedy(x: torch.Tensor) -> int:
    """First token in rank order: the largest value, lowest index on ties (engine/src/misc.cu:54)."""
    keys = rank_keys(x)
    top = int(keys.max())
    return int(torch.nonzero(keys == top)[0])


# ---------------------------------------------------------------------------------------------- weights
def kappa32(temperature: float) -> np.float32:
    """kappa = (float)((double)(1.0f / T) * LOG2E)."""
    return np.float32(float(f32(1.0) / f32(temperature)) * LOG2E)


def log2_units(x: torch.Tensor, temperature: float) -> torch.Tensor:
    """a = clamp(x * kappa, -2^22, 2^22), fp32."""
    a = x.to(torch.float32) * torch.tensor(kappa32(temperature), dtype=torch.float32)
    return a.clamp(-A_CLAMP, A_CLAMP)


def exp2_table(a: torch.Tensor):
    """(q, mu) of fp32 log2 units a: q = floor(a * 256) (n = q >> 8, fine bin = q >> 2), mu = 24-bit mantissa of 2^(a - n)."""
    t = a.to(torch.float32) * torch.tensor(256.0, dtype=torch.float32)
    fl = torch.floor(t)
    q = fl.to(torch.int64)
    r = t - fl
    p = r * torch.tensor(C2)
    p = p + torch.tensor(C1)
    p = p * r
    p = p + torch.tensor(1.0, dtype=torch.float32)
    m = torch.from_numpy(TAB)[(q & 255)] * p
    mu = (m * torch.tensor(8388608.0, dtype=torch.float32)).to(torch.int64)
    return q, mu


def mantissa(a: torch.Tensor):
    """(n, mu): n = floor(a), mu = 24-bit mantissa of 2^(a - n)."""
    q, mu = exp2_table(a)
    return q >> 8, mu


def min_p_cut(a_max: float, min_p: float) -> np.float32:
    """a_cut = (float)((double)a_max + log2(min_p))."""
    return np.float32(float(a_max) + math.log2(float(f32(min_p))))


@dataclass
class RowResult:
    token: int
    kept: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int64))     # kept token ids, rank order
    weights: list = field(default_factory=list)                                 # their weights (python ints)
    S2: int = 0
    greedy: bool = False

    def probs(self) -> dict:
        return {int(i): (w / self.S2) for i, w in zip(self.kept, self.weights) if w > 0}


def _prefix_first(ws: Sequence[int], target: int, strict: bool) -> int:
    """First position j with inclusive prefix sum of ws (non-negative ints) >= target (strict=False)
    or > target (strict=True).  Exact (python ints); vectorised prefix sums in two 31-bit halves."""
    w = np.array(ws, dtype=object)
    lo = np.array([int(v) & 0x7FFFFFFF for v in ws], dtype=np.int64)
    hi = np.array([int(v) >> 31 for v in ws], dtype=np.int64)
    clo, chi = np.cumsum(lo), np.cumsum(hi)
    n = len(w)
    a, b = 0, n - 1  # binary search over the monotone prefix
    def cum(j):
        return (int(chi[j]) << 31) + int(clo[j])
    while a < b:
        mid = (a + b) // 2
        c = cum(mid)
        if (c > target) if strict else (c >= target):
            b = mid
        else:
            a = mid + 1
    return a


def distribution(x: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0, min_p: float = 0.0):
    """Kept candidates of a processed row in rank order with their weights: (ids int64 [n], weights list[int], S2)."""
    cand = torch.nonzero(x != -math.inf).flatten()
    if cand.numel() == 0:
        return None
    xc = x[cand]
    order = rank_order(xc, cand)
    ids = cand[order]
    a = log2_units(x[ids], temperature)
    if f32(min_p) > 0:
        keep = a >= torch.tensor(min_p_cut(float(a[0]), min_p))
        ids, a = ids[keep], a[keep]
    if top_k > 0 and top_k < ids.numel():
        ids, a = ids[:top_k], a[:top_k]
    n, mu = mantissa(a)
    N = int(n[0])
    sh = n - N + D_EXP
    w_t = torch.where(sh >= 0, mu << sh.clamp_min(0), torch.zeros_like(mu))
    ws = [int(v) for v in w_t.tolist()]
    S = sum(ws)
    tp = f32(top_p)
    if tp < f32(1.0):
        TP = math.floor(float(tp) * 2 ** 32)
        thr = -((-TP * S) >> 32)
        j = _prefix_first(ws, thr, strict=False)
        ids, ws = ids[: j + 1], ws[: j + 1]
    return ids.numpy(), ws, sum(ws)


def draw_index_order(ids: np.ndarray, ws: Sequence[int], S2: int, u24: int) -> int:
    """Inverse CDF in index order: the smallest kept id whose prefix sum exceeds floor(u24 * S2 / 2^24)."""
    t = (int(u24) * int(S2)) >> 24
    o = np.argsort(ids, kind="stable")
    j = _prefix_first([ws[i] for i in o], t, strict=True)
    return int(ids[o[j]])


def sample_row(logits: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0, min_p: float = 0.0,
               seed: int = 0, position: int = 0, stream: int = ST_FIRST, row_key: int = 0,
               procs: Optional[RowProcs] = None, drafts_before: Sequence[int] = ()) -> RowResult:
    """One row: processors, then greedy (temperature <= 0) or the sampled token."""
    x = process(logits, procs, drafts_before)
    if not (f32(temperature) > 0):
        return RowResult(token=greedy(x), greedy=True)
    d = distribution(x, temperature, top_k, top_p, min_p)
    if d is None:
        return RowResult(token=greedy(x), greedy=True)
    ids, ws, S2 = d
    u = int(draw_u24(seed, position, stream, row_key))
    tok = draw_index_order(ids, ws, S2, u)
    return RowResult(token=tok, kept=ids, weights=ws, S2=S2)


# ---------------------------------------------------------------------------------------------- speculative verify
def q_fix(q: float, S2: int) -> int:
    """floor(q * S2) exactly for an fp32 probability q >= 0."""
    qd = float(f32(q))
    if qd <= 0.0:
        return 0
    m, e = math.frexp(qd)  # qd = m * 2^e, m in [0.5, 1)
    M = int(m * (1 << 53))
    s = 53 - e
    return (M * S2) >> s if s >= 0 else (M * S2) << (-s)


@dataclass
class VerifyResult:
    tokens: list
    accepted: int   # emitted tokens = accepted drafts + 1


def verify_seq(target_logits: torch.Tensor, draft_probs: torch.Tensor, idmap: np.ndarray, drafts: Sequence[int],
               temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0, min_p: float = 0.0, seed: int = 0,
               position: int = 0, row_key: int = 0, procs: Optional[RowProcs] = None, test_flags: int = 0) -> VerifyResult:
    """One sequence: target rows [K+1][V], draft probabilities [K][Vd] over the reduced vocabulary with
    token ids idmap[Vd], draft tokens d_1..d_K (engine/src/mtp_sample.cu:227-258)."""
    K = len(drafts)
    inv = {int(t): j for j, t in enumerate(np.asarray(idmap).tolist())}
    out = []
    for t in range(K + 1):
        x = process(target_logits[t], procs, list(drafts[:t]))
        d = distribution(x, temperature, top_k, top_p, min_p)
        if d is None:  # no candidate: greedy row
            out.append(greedy(x))
            return VerifyResult(out, len(out))
        ids, ws, S2 = d
        r = philox(position, ST_ACCEPT + t, row_key, 0, seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)
        u_acc, u_res = int(r[0] >> np.uint64(8)), int(r[1] >> np.uint64(8))
        if t == K:  # every draft accepted: bonus token from the last row
            out.append(draw_index_order(ids, ws, S2, u_res))
            return VerifyResult(out, len(out))
        dt = int(drafts[t])
        qrow = draft_probs[t].numpy()
        qd = float(qrow[inv[dt]]) if dt in inv else 0.0
        wd = 0
        pos = np.nonzero(ids == dt)[0]
        if len(pos):
            wd = ws[int(pos[0])]
        if u_acc * q_fix(qd, S2) < wd * (1 << 24):
            out.append(dt)
            continue
        res = ws
        if not (test_flags & 1):
            res = [max(0, w - q_fix(float(qrow[inv[int(i)]]), S2)) if int(i) in inv else w for i, w in zip(ids, ws)]
            if sum(res) == 0:
                res = ws
        out.append(draw_index_order(ids, res, sum(res), u_res))
        return VerifyResult(out, len(out))
    raise AssertionError("unreachable")
