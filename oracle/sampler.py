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
3. Sampling.  Candidates = tokens with x != -inf (none: the greedy token).  A row samples when T > 0 and
   K below is finite (otherwise it is greedy).
     inv_t = 1.0f / temperature (fp32, engine/src/mtp_sample.cu:377)
     kappa = (float)((double)inv_t * LOG2E)        (one rounding);  K = kappa * 1024 (exact)
     t_i   = clamp(fl(x_i * K), -2^30, 2^30)        (x_i / T in log2 units times 1024: a_i = t_i / 1024)
     q_i   = floor(t_i),  r_i = min(fl(t_i - q_i), 1 - 2^-24)
     n_i   = q_i >> 10 (= floor(a_i)),  fine bin = q_i >> 4 (= floor(a_i * 64)),  j_i = q_i & 1023
     mu_i  = (uint32)(fl(fl(r_i * TAB_S[j]) + TAB_T[j]))   the 24-bit mantissa of 2^(a_i - n_i), by linear
             interpolation of the 1024-point table TAB_T[j] = fp32(2^(j/1024) * 2^23),
             TAB_S[j] = fp32((2^((j+1)/1024) - 2^(j/1024)) * 2^23)  (relative error <= 1.7e-7)
     t_max = t of the first candidate, N = floor(t_max / 1024)
   min_p > 0: keep candidates with t_i >= t_cut, t_cut = (float)((double)(t_max / 1024) + log2(min_p)) * 1024
              (log2 from libm, once per row) -- p_i >= min_p * p_max (vLLM min_p, before top-k).
   top-k (K > 0): keep the first K remaining candidates in rank order.
   weight w_i = mu_i * 2^(n_i - N + 35) if n_i >= N - 35 else 0    (exact integer <= 2^59;
              the dropped tail is below 2^-34 of the top token's weight)
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
     for t in 0..K-1, row t's distribution (kept set, w, S2_t; a greedy row is its argmax with w = S2 = 1; a row
       without candidates emits its greedy token and stops); Q_i = floor(q_t(i) * S2_t) exactly (q NaN or <= 0
       counts as 0, q >= 1 as 1; ids outside the table have q = 0);
       (r0, r1) = Philox(counter = (position, ACCEPT + t, row_key, 0));
       accept d_{t+1} iff (r0 >> 8) * Q_d < w_d * 2^24   (u * q(d) < p(d); w_d = 0 if not kept);
       else residual r_i = max(0, w_i - Q_i) over the kept set (R = 0, or test flag bit0: r = w),
            draw from r in index order with u24 = r1 >> 8, emit t + 1 tokens, stop;
     all accepted: bonus token from row K with u24 = Philox(position, ACCEPT + K).r1 >> 8.

Everything above is integer or correctly rounded IEEE arithmetic, so the CPU and the GPU agree
exactly.  The weights approximate exp((x_i - x_max) / T) to ~1.7e-7 relative error.
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
T_CLAMP = float(2 ** 30)    # t = x / T in units of 2^-10 powers of two, clamped to +-2^30 (|a| <= 2^20)
D_EXP = 35                  # weights below 2^-35 of the row's top power of two are dropped
# 2^(r / 1024) on r in [0, 1) by linear interpolation between table points:
# TAB_T[j] = fp32(2^(j / 1024) * 2^23), TAB_S[j] = fp32((2^((j + 1) / 1024) - 2^(j / 1024)) * 2^23)
TAB_T = np.array([
    0x4b000000, 0x4b001630, 0x4b002c64, 0x4b00429c, 0x4b0058d8, 0x4b006f17, 0x4b00855b, 0x4b009ba2,
    0x4b00b1ed, 0x4b00c83c, 0x4b00de8f, 0x4b00f4e6, 0x4b010b41, 0x4b01219f, 0x4b013802, 0x4b014e68,
    0x4b0164d2, 0x4b017b40, 0x4b0191b2, 0x4b01a828, 0x4b01bea1, 0x4b01d51f, 0x4b01eba1, 0x4b020226,
    0x4b0218af, 0x4b022f3c, 0x4b0245ce, 0x4b025c63, 0x4b0272fc, 0x4b028998, 0x4b02a039, 0x4b02b6de,
    0x4b02cd87, 0x4b02e433, 0x4b02fae4, 0x4b031198, 0x4b032850, 0x4b033f0d, 0x4b0355cd, 0x4b036c91,
    0x4b038359, 0x4b039a25, 0x4b03b0f5, 0x4b03c7c9, 0x4b03dea1, 0x4b03f57d, 0x4b040c5d, 0x4b042341,
    0x4b043a29, 0x4b045115, 0x4b046804, 0x4b047ef8, 0x4b0495f0, 0x4b04aceb, 0x4b04c3eb, 0x4b04daef,
    0x4b04f1f6, 0x4b050902, 0x4b052012, 0x4b053725, 0x4b054e3d, 0x4b056558, 0x4b057c78, 0x4b05939c,
    0x4b05aac3, 0x4b05c1ef, 0x4b05d91f, 0x4b05f052, 0x4b06078a, 0x4b061ec6, 0x4b063606, 0x4b064d4a,
    0x4b066491, 0x4b067bdd, 0x4b06932d, 0x4b06aa81, 0x4b06c1d9, 0x4b06d935, 0x4b06f095, 0x4b0707f9,
    0x4b071f62, 0x4b0736ce, 0x4b074e3e, 0x4b0765b3, 0x4b077d2b, 0x4b0794a8, 0x4b07ac28, 0x4b07c3ad,
    0x4b07db35, 0x4b07f2c2, 0x4b080a53, 0x4b0821e8, 0x4b083981, 0x4b08511e, 0x4b0868c0, 0x4b088065,
    0x4b08980f, 0x4b08afbc, 0x4b08c76e, 0x4b08df23, 0x4b08f6dd, 0x4b090e9b, 0x4b09265d, 0x4b093e24,
    0x4b0955ee, 0x4b096dbc, 0x4b09858f, 0x4b099d66, 0x4b09b541, 0x4b09cd20, 0x4b09e503, 0x4b09fcea,
    0x4b0a14d5, 0x4b0a2cc5, 0x4b0a44b9, 0x4b0a5cb1, 0x4b0a74ad, 0x4b0a8cad, 0x4b0aa4b1, 0x4b0abcba,
    0x4b0ad4c6, 0x4b0aecd7, 0x4b0b04ec, 0x4b0b1d05, 0x4b0b3523, 0x4b0b4d44, 0x4b0b656a, 0x4b0b7d94,
    0x4b0b95c2, 0x4b0badf4, 0x4b0bc62b, 0x4b0bde65, 0x4b0bf6a4, 0x4b0c0ee7, 0x4b0c272f, 0x4b0c3f7a,
    0x4b0c57ca, 0x4b0c701e, 0x4b0c8876, 0x4b0ca0d2, 0x4b0cb933, 0x4b0cd198, 0x4b0cea01, 0x4b0d026e,
    0x4b0d1adf, 0x4b0d3355, 0x4b0d4bcf, 0x4b0d644d, 0x4b0d7cd0, 0x4b0d9556, 0x4b0dade1, 0x4b0dc671,
    0x4b0ddf04, 0x4b0df79c, 0x4b0e1038, 0x4b0e28d8, 0x4b0e417d, 0x4b0e5a25, 0x4b0e72d3, 0x4b0e8b84,
    0x4b0ea43a, 0x4b0ebcf3, 0x4b0ed5b2, 0x4b0eee74, 0x4b0f073b, 0x4b0f2006, 0x4b0f38d5, 0x4b0f51a9,
    0x4b0f6a81, 0x4b0f835d, 0x4b0f9c3e, 0x4b0fb523, 0x4b0fce0c, 0x4b0fe6fa, 0x4b0fffec, 0x4b1018e2,
    0x4b1031dc, 0x4b104adb, 0x4b1063de, 0x4b107ce6, 0x4b1095f2, 0x4b10af02, 0x4b10c816, 0x4b10e12f,
    0x4b10fa4d, 0x4b11136e, 0x4b112c94, 0x4b1145be, 0x4b115eed, 0x4b117820, 0x4b119158, 0x4b11aa93,
    0x4b11c3d3, 0x4b11dd18, 0x4b11f661, 0x4b120fae, 0x4b122900, 0x4b124256, 0x4b125bb0, 0x4b12750f,
    0x4b128e72, 0x4b12a7da, 0x4b12c146, 0x4b12dab7, 0x4b12f42c, 0x4b130da5, 0x4b132723, 0x4b1340a5,
    0x4b135a2b, 0x4b1373b6, 0x4b138d46, 0x4b13a6d9, 0x4b13c072, 0x4b13da0e, 0x4b13f3af, 0x4b140d55,
    0x4b1426ff, 0x4b1440ae, 0x4b145a60, 0x4b147418, 0x4b148dd4, 0x4b14a794, 0x4b14c159, 0x4b14db22,
    0x4b14f4f0, 0x4b150ec2, 0x4b152898, 0x4b154274, 0x4b155c53, 0x4b157637, 0x4b159020, 0x4b15aa0d,
    0x4b15c3ff, 0x4b15ddf5, 0x4b15f7ef, 0x4b1611ee, 0x4b162bf2, 0x4b1645fa, 0x4b166006, 0x4b167a18,
    0x4b16942d, 0x4b16ae47, 0x4b16c866, 0x4b16e289, 0x4b16fcb1, 0x4b1716dd, 0x4b17310e, 0x4b174b43,
    0x4b17657d, 0x4b177fbc, 0x4b1799ff, 0x4b17b446, 0x4b17ce92, 0x4b17e8e3, 0x4b180338, 0x4b181d92,
    0x4b1837f0, 0x4b185253, 0x4b186cbb, 0x4b188727, 0x4b18a197, 0x4b18bc0d, 0x4b18d686, 0x4b18f105,
    0x4b190b88, 0x4b19260f, 0x4b19409c, 0x4b195b2c, 0x4b1975c2, 0x4b19905c, 0x4b19aafa, 0x4b19c59e,
    0x4b19e046, 0x4b19faf2, 0x4b1a15a3, 0x4b1a3059, 0x4b1a4b13, 0x4b1a65d2, 0x4b1a8096, 0x4b1a9b5e,
    0x4b1ab62b, 0x4b1ad0fd, 0x4b1aebd3, 0x4b1b06ae, 0x4b1b218d, 0x4b1b3c71, 0x4b1b575a, 0x4b1b7248,
    0x4b1b8d3a, 0x4b1ba831, 0x4b1bc32c, 0x4b1bde2c, 0x4b1bf931, 0x4b1c143b, 0x4b1c2f49, 0x4b1c4a5c,
    0x4b1c6573, 0x4b1c8090, 0x4b1c9bb1, 0x4b1cb6d6, 0x4b1cd201, 0x4b1ced30, 0x4b1d0864, 0x4b1d239c,
    0x4b1d3eda, 0x4b1d5a1c, 0x4b1d7562, 0x4b1d90ae, 0x4b1dabfe, 0x4b1dc753, 0x4b1de2ad, 0x4b1dfe0b,
    0x4b1e196e, 0x4b1e34d6, 0x4b1e5043, 0x4b1e6bb4, 0x4b1e872a, 0x4b1ea2a5, 0x4b1ebe25, 0x4b1ed9a9,
    0x4b1ef532, 0x4b1f10c0, 0x4b1f2c53, 0x4b1f47eb, 0x4b1f6387, 0x4b1f7f28, 0x4b1f9ace, 0x4b1fb679,
    0x4b1fd228, 0x4b1feddc, 0x4b200996, 0x4b202553, 0x4b204116, 0x4b205cde, 0x4b2078aa, 0x4b20947b,
    0x4b20b051, 0x4b20cc2c, 0x4b20e80b, 0x4b2103f0, 0x4b211fd9, 0x4b213bc7, 0x4b2157ba, 0x4b2173b2,
    0x4b218faf, 0x4b21abb0, 0x4b21c7b7, 0x4b21e3c2, 0x4b21ffd2, 0x4b221be7, 0x4b223801, 0x4b22541f,
    0x4b227043, 0x4b228c6b, 0x4b22a899, 0x4b22c4cb, 0x4b22e102, 0x4b22fd3e, 0x4b23197f, 0x4b2335c5,
    0x4b23520f, 0x4b236e5f, 0x4b238ab3, 0x4b23a70d, 0x4b23c36b, 0x4b23dfce, 0x4b23fc37, 0x4b2418a4,
    0x4b243516, 0x4b24518d, 0x4b246e08, 0x4b248a89, 0x4b24a70f, 0x4b24c39a, 0x4b24e029, 0x4b24fcbe,
    0x4b251958, 0x4b2535f6, 0x4b255299, 0x4b256f42, 0x4b258bef, 0x4b25a8a2, 0x4b25c559, 0x4b25e215,
    0x4b25fed7, 0x4b261b9d, 0x4b263868, 0x4b265538, 0x4b26720e, 0x4b268ee8, 0x4b26abc7, 0x4b26c8ac,
    0x4b26e595, 0x4b270283, 0x4b271f76, 0x4b273c6f, 0x4b27596c, 0x4b27766e, 0x4b279376, 0x4b27b082,
    0x4b27cd94, 0x4b27eaaa, 0x4b2807c6, 0x4b2824e6, 0x4b28420c, 0x4b285f37, 0x4b287c66, 0x4b28999b,
    0x4b28b6d5, 0x4b28d414, 0x4b28f158, 0x4b290ea1, 0x4b292bef, 0x4b294942, 0x4b29669b, 0x4b2983f8,
    0x4b29a15b, 0x4b29bec2, 0x4b29dc2f, 0x4b29f9a1, 0x4b2a1718, 0x4b2a3494, 0x4b2a5215, 0x4b2a6f9b,
    0x4b2a8d26, 0x4b2aaab7, 0x4b2ac84c, 0x4b2ae5e7, 0x4b2b0387, 0x4b2b212c, 0x4b2b3ed6, 0x4b2b5c85,
    0x4b2b7a3a, 0x4b2b97f3, 0x4b2bb5b2, 0x4b2bd376, 0x4b2bf13f, 0x4b2c0f0d, 0x4b2c2ce0, 0x4b2c4ab9,
    0x4b2c6897, 0x4b2c867a, 0x4b2ca462, 0x4b2cc24f, 0x4b2ce041, 0x4b2cfe39, 0x4b2d1c36, 0x4b2d3a38,
    0x4b2d583f, 0x4b2d764b, 0x4b2d945d, 0x4b2db274, 0x4b2dd090, 0x4b2deeb1, 0x4b2e0cd8, 0x4b2e2b03,
    0x4b2e4934, 0x4b2e676b, 0x4b2e85a6, 0x4b2ea3e7, 0x4b2ec22d, 0x4b2ee078, 0x4b2efec8, 0x4b2f1d1e,
    0x4b2f3b79, 0x4b2f59d9, 0x4b2f783e, 0x4b2f96a9, 0x4b2fb519, 0x4b2fd38e, 0x4b2ff209, 0x4b301089,
    0x4b302f0e, 0x4b304d98, 0x4b306c28, 0x4b308abd, 0x4b30a957, 0x4b30c7f7, 0x4b30e69c, 0x4b310546,
    0x4b3123f6, 0x4b3142aa, 0x4b316165, 0x4b318024, 0x4b319ee9, 0x4b31bdb3, 0x4b31dc83, 0x4b31fb57,
    0x4b321a32, 0x4b323911, 0x4b3257f6, 0x4b3276e0, 0x4b3295d0, 0x4b32b4c5, 0x4b32d3bf, 0x4b32f2bf,
    0x4b3311c4, 0x4b3330cf, 0x4b334fde, 0x4b336ef4, 0x4b338e0e, 0x4b33ad2e, 0x4b33cc54, 0x4b33eb7e,
    0x4b340aaf, 0x4b3429e4, 0x4b34491f, 0x4b346860, 0x4b3487a6, 0x4b34a6f1, 0x4b34c642, 0x4b34e598,
    0x4b3504f3, 0x4b352454, 0x4b3543bb, 0x4b356327, 0x4b358298, 0x4b35a20f, 0x4b35c18b, 0x4b35e10d,
    0x4b360094, 0x4b362020, 0x4b363fb2, 0x4b365f4a, 0x4b367ee7, 0x4b369e89, 0x4b36be31, 0x4b36dddf,
    0x4b36fd92, 0x4b371d4a, 0x4b373d08, 0x4b375ccc, 0x4b377c95, 0x4b379c63, 0x4b37bc37, 0x4b37dc11,
    0x4b37fbf0, 0x4b381bd4, 0x4b383bbe, 0x4b385bae, 0x4b387ba3, 0x4b389b9e, 0x4b38bb9e, 0x4b38dba4,
    0x4b38fbaf, 0x4b391bc0, 0x4b393bd7, 0x4b395bf3, 0x4b397c14, 0x4b399c3b, 0x4b39bc68, 0x4b39dc9a,
    0x4b39fcd2, 0x4b3a1d10, 0x4b3a3d53, 0x4b3a5d9b, 0x4b3a7dea, 0x4b3a9e3e, 0x4b3abe97, 0x4b3adef6,
    0x4b3aff5b, 0x4b3b1fc5, 0x4b3b4035, 0x4b3b60aa, 0x4b3b8126, 0x4b3ba1a6, 0x4b3bc22d, 0x4b3be2b9,
    0x4b3c034a, 0x4b3c23e2, 0x4b3c447f, 0x4b3c6521, 0x4b3c85ca, 0x4b3ca678, 0x4b3cc72b, 0x4b3ce7e5,
    0x4b3d08a4, 0x4b3d2968, 0x4b3d4a33, 0x4b3d6b03, 0x4b3d8bd8, 0x4b3dacb4, 0x4b3dcd95, 0x4b3dee7c,
    0x4b3e0f68, 0x4b3e305a, 0x4b3e5152, 0x4b3e7250, 0x4b3e9353, 0x4b3eb45c, 0x4b3ed56b, 0x4b3ef67f,
    0x4b3f179a, 0x4b3f38ba, 0x4b3f59df, 0x4b3f7b0b, 0x4b3f9c3c, 0x4b3fbd73, 0x4b3fdeb0, 0x4b3ffff2,
    0x4b40213b, 0x4b404289, 0x4b4063dc, 0x4b408536, 0x4b40a695, 0x4b40c7fb, 0x4b40e966, 0x4b410ad6,
    0x4b412c4d, 0x4b414dc9, 0x4b416f4b, 0x4b4190d3, 0x4b41b261, 0x4b41d3f5, 0x4b41f58e, 0x4b42172d,
    0x4b4238d2, 0x4b425a7d, 0x4b427c2e, 0x4b429de4, 0x4b42bfa1, 0x4b42e163, 0x4b43032b, 0x4b4324f9,
    0x4b4346cd, 0x4b4368a7, 0x4b438a86, 0x4b43ac6b, 0x4b43ce57, 0x4b43f048, 0x4b44123f, 0x4b44343c,
    0x4b44563f, 0x4b447848, 0x4b449a56, 0x4b44bc6b, 0x4b44de85, 0x4b4500a5, 0x4b4522cc, 0x4b4544f8,
    0x4b45672a, 0x4b458962, 0x4b45aba0, 0x4b45cde4, 0x4b45f02e, 0x4b46127e, 0x4b4634d3, 0x4b46572f,
    0x4b467991, 0x4b469bf8, 0x4b46be66, 0x4b46e0d9, 0x4b470353, 0x4b4725d2, 0x4b474858, 0x4b476ae3,
    0x4b478d75, 0x4b47b00c, 0x4b47d2aa, 0x4b47f54d, 0x4b4817f7, 0x4b483aa6, 0x4b485d5b, 0x4b488017,
    0x4b48a2d8, 0x4b48c5a0, 0x4b48e86d, 0x4b490b41, 0x4b492e1b, 0x4b4950fa, 0x4b4973e0, 0x4b4996cc,
    0x4b49b9be, 0x4b49dcb5, 0x4b49ffb3, 0x4b4a22b7, 0x4b4a45c1, 0x4b4a68d1, 0x4b4a8be8, 0x4b4aaf04,
    0x4b4ad226, 0x4b4af54f, 0x4b4b187d, 0x4b4b3bb2, 0x4b4b5eed, 0x4b4b822e, 0x4b4ba575, 0x4b4bc8c2,
    0x4b4bec15, 0x4b4c0f6e, 0x4b4c32ce, 0x4b4c5633, 0x4b4c799f, 0x4b4c9d11, 0x4b4cc089, 0x4b4ce407,
    0x4b4d078c, 0x4b4d2b16, 0x4b4d4ea7, 0x4b4d723d, 0x4b4d95da, 0x4b4db97e, 0x4b4ddd27, 0x4b4e00d6,
    0x4b4e248c, 0x4b4e4848, 0x4b4e6c0a, 0x4b4e8fd2, 0x4b4eb3a1, 0x4b4ed775, 0x4b4efb50, 0x4b4f1f31,
    0x4b4f4319, 0x4b4f6706, 0x4b4f8afa, 0x4b4faef4, 0x4b4fd2f4, 0x4b4ff6fb, 0x4b501b08, 0x4b503f1b,
    0x4b506334, 0x4b508753, 0x4b50ab79, 0x4b50cfa5, 0x4b50f3d7, 0x4b511810, 0x4b513c4f, 0x4b516094,
    0x4b5184df, 0x4b51a931, 0x4b51cd89, 0x4b51f1e7, 0x4b52164c, 0x4b523ab7, 0x4b525f28, 0x4b5283a0,
    0x4b52a81e, 0x4b52cca2, 0x4b52f12c, 0x4b5315bd, 0x4b533a54, 0x4b535ef2, 0x4b538396, 0x4b53a840,
    0x4b53ccf1, 0x4b53f1a8, 0x4b541665, 0x4b543b29, 0x4b545ff3, 0x4b5484c3, 0x4b54a99a, 0x4b54ce77,
    0x4b54f35b, 0x4b551845, 0x4b553d35, 0x4b55622c, 0x4b558729, 0x4b55ac2d, 0x4b55d137, 0x4b55f647,
    0x4b561b5e, 0x4b56407b, 0x4b56659f, 0x4b568ac9, 0x4b56affa, 0x4b56d531, 0x4b56fa6e, 0x4b571fb2,
    0x4b5744fd, 0x4b576a4e, 0x4b578fa5, 0x4b57b503, 0x4b57da67, 0x4b57ffd2, 0x4b582543, 0x4b584abb,
    0x4b587039, 0x4b5895be, 0x4b58bb49, 0x4b58e0db, 0x4b590673, 0x4b592c12, 0x4b5951b8, 0x4b597763,
    0x4b599d16, 0x4b59c2cf, 0x4b59e88e, 0x4b5a0e54, 0x4b5a3421, 0x4b5a59f4, 0x4b5a7fcd, 0x4b5aa5ae,
    0x4b5acb94, 0x4b5af182, 0x4b5b1776, 0x4b5b3d70, 0x4b5b6371, 0x4b5b8979, 0x4b5baf87, 0x4b5bd59c,
    0x4b5bfbb8, 0x4b5c21da, 0x4b5c4802, 0x4b5c6e32, 0x4b5c9468, 0x4b5cbaa4, 0x4b5ce0e7, 0x4b5d0731,
    0x4b5d2d82, 0x4b5d53d9, 0x4b5d7a36, 0x4b5da09b, 0x4b5dc706, 0x4b5ded77, 0x4b5e13f0, 0x4b5e3a6f,
    0x4b5e60f5, 0x4b5e8781, 0x4b5eae14, 0x4b5ed4ae, 0x4b5efb4e, 0x4b5f21f5, 0x4b5f48a3, 0x4b5f6f58,
    0x4b5f9613, 0x4b5fbcd5, 0x4b5fe39e, 0x4b600a6d, 0x4b603143, 0x4b605820, 0x4b607f03, 0x4b60a5ee,
    0x4b60ccdf, 0x4b60f3d7, 0x4b611ad5, 0x4b6141db, 0x4b6168e7, 0x4b618ffa, 0x4b61b713, 0x4b61de34,
    0x4b62055b, 0x4b622c89, 0x4b6253be, 0x4b627af9, 0x4b62a23c, 0x4b62c985, 0x4b62f0d5, 0x4b63182c,
    0x4b633f89, 0x4b6366ee, 0x4b638e59, 0x4b63b5cb, 0x4b63dd44, 0x4b6404c4, 0x4b642c4b, 0x4b6453d8,
    0x4b647b6d, 0x4b64a308, 0x4b64caaa, 0x4b64f253, 0x4b651a03, 0x4b6541b9, 0x4b656977, 0x4b65913c,
    0x4b65b907, 0x4b65e0d9, 0x4b6608b2, 0x4b663092, 0x4b665879, 0x4b668067, 0x4b66a85c, 0x4b66d058,
    0x4b66f85b, 0x4b672064, 0x4b674875, 0x4b67708c, 0x4b6798ab, 0x4b67c0d0, 0x4b67e8fd, 0x4b681130,
    0x4b68396a, 0x4b6861ac, 0x4b6889f4, 0x4b68b243, 0x4b68da99, 0x4b6902f7, 0x4b692b5b, 0x4b6953c6,
    0x4b697c38, 0x4b69a4b1, 0x4b69cd32, 0x4b69f5b9, 0x4b6a1e47, 0x4b6a46dd, 0x4b6a6f79, 0x4b6a981c,
    0x4b6ac0c7, 0x4b6ae978, 0x4b6b1231, 0x4b6b3af1, 0x4b6b63b7, 0x4b6b8c85, 0x4b6bb55a, 0x4b6bde36,
    0x4b6c0719, 0x4b6c3003, 0x4b6c58f4, 0x4b6c81ec, 0x4b6caaec, 0x4b6cd3f2, 0x4b6cfd00, 0x4b6d2614,
    0x4b6d4f30, 0x4b6d7853, 0x4b6da17d, 0x4b6dcaae, 0x4b6df3e7, 0x4b6e1d26, 0x4b6e466d, 0x4b6e6fbb,
    0x4b6e9910, 0x4b6ec26c, 0x4b6eebcf, 0x4b6f1539, 0x4b6f3eab, 0x4b6f6824, 0x4b6f91a4, 0x4b6fbb2b,
    0x4b6fe4ba, 0x4b700e4f, 0x4b7037ec, 0x4b706190, 0x4b708b3b, 0x4b70b4ee, 0x4b70dea8, 0x4b710868,
    0x4b713231, 0x4b715c00, 0x4b7185d7, 0x4b71afb5, 0x4b71d99a, 0x4b720386, 0x4b722d7a, 0x4b725775,
    0x4b728177, 0x4b72ab81, 0x4b72d592, 0x4b72ffaa, 0x4b7329c9, 0x4b7353f0, 0x4b737e1e, 0x4b73a853,
    0x4b73d290, 0x4b73fcd4, 0x4b74271f, 0x4b745172, 0x4b747bcc, 0x4b74a62d, 0x4b74d096, 0x4b74fb06,
    0x4b75257d, 0x4b754ffc, 0x4b757a82, 0x4b75a50f, 0x4b75cfa4, 0x4b75fa40, 0x4b7624e4, 0x4b764f8f,
    0x4b767a41, 0x4b76a4fb, 0x4b76cfbc, 0x4b76fa85, 0x4b772555, 0x4b77502d, 0x4b777b0b, 0x4b77a5f2,
    0x4b77d0df, 0x4b77fbd5, 0x4b7826d1, 0x4b7851d5, 0x4b787ce1, 0x4b78a7f4, 0x4b78d30e, 0x4b78fe30,
    0x4b79295a, 0x4b79548b, 0x4b797fc3, 0x4b79ab03, 0x4b79d64a, 0x4b7a0199, 0x4b7a2cf0, 0x4b7a584d,
    0x4b7a83b3, 0x4b7aaf20, 0x4b7ada94, 0x4b7b0610, 0x4b7b3194, 0x4b7b5d1f, 0x4b7b88b2, 0x4b7bb44c,
    0x4b7bdfed, 0x4b7c0b97, 0x4b7c3748, 0x4b7c6300, 0x4b7c8ec0, 0x4b7cba88, 0x4b7ce657, 0x4b7d122e,
    0x4b7d3e0c, 0x4b7d69f2, 0x4b7d95e0, 0x4b7dc1d5, 0x4b7dedd2, 0x4b7e19d6, 0x4b7e45e2, 0x4b7e71f6,
    0x4b7e9e11, 0x4b7eca34, 0x4b7ef65f, 0x4b7f2291, 0x4b7f4ecb, 0x4b7f7b0d, 0x4b7fa756, 0x4b7fd3a7,
], dtype=np.uint32).view(np.float32)
TAB_S = np.array([
    0x45b18179, 0x45b1a03e, 0x45b1bf08, 0x45b1ddd8, 0x45b1fcad, 0x45b21b87, 0x45b23a67, 0x45b2594c,
    0x45b27837, 0x45b29727, 0x45b2b61c, 0x45b2d516, 0x45b2f416, 0x45b3131c, 0x45b33226, 0x45b35137,
    0x45b3704c, 0x45b38f67, 0x45b3ae87, 0x45b3cdad, 0x45b3ecd8, 0x45b40c08, 0x45b42b3e, 0x45b44a79,
    0x45b469ba, 0x45b48900, 0x45b4a84c, 0x45b4c79c, 0x45b4e6f3, 0x45b5064f, 0x45b525b0, 0x45b54517,
    0x45b56483, 0x45b583f4, 0x45b5a36b, 0x45b5c2e8, 0x45b5e26a, 0x45b601f1, 0x45b6217e, 0x45b64110,
    0x45b660a8, 0x45b68045, 0x45b69fe8, 0x45b6bf90, 0x45b6df3e, 0x45b6fef1, 0x45b71eaa, 0x45b73e68,
    0x45b75e2c, 0x45b77df5, 0x45b79dc4, 0x45b7bd98, 0x45b7dd72, 0x45b7fd51, 0x45b81d36, 0x45b83d20,
    0x45b85d10, 0x45b87d05, 0x45b89d00, 0x45b8bd01, 0x45b8dd07, 0x45b8fd12, 0x45b91d23, 0x45b93d3a,
    0x45b95d56, 0x45b97d78, 0x45b99da0, 0x45b9bdcd, 0x45b9ddff, 0x45b9fe37, 0x45ba1e75, 0x45ba3eb8,
    0x45ba5f01, 0x45ba7f50, 0x45ba9fa4, 0x45babffd, 0x45bae05d, 0x45bb00c2, 0x45bb212c, 0x45bb419c,
    0x45bb6212, 0x45bb828d, 0x45bba30e, 0x45bbc395, 0x45bbe421, 0x45bc04b3, 0x45bc254b, 0x45bc45e8,
    0x45bc668b, 0x45bc8734, 0x45bca7e2, 0x45bcc896, 0x45bce94f, 0x45bd0a0e, 0x45bd2ad3, 0x45bd4b9e,
    0x45bd6c6e, 0x45bd8d44, 0x45bdae20, 0x45bdcf01, 0x45bdefe8, 0x45be10d5, 0x45be31c7, 0x45be52bf,
    0x45be73bd, 0x45be94c1, 0x45beb5ca, 0x45bed6d9, 0x45bef7ee, 0x45bf1908, 0x45bf3a29, 0x45bf5b4f,
    0x45bf7c7a, 0x45bf9dac, 0x45bfbee3, 0x45bfe020, 0x45c00163, 0x45c022ab, 0x45c043fa, 0x45c0654e,
    0x45c086a8, 0x45c0a807, 0x45c0c96d, 0x45c0ead8, 0x45c10c49, 0x45c12dc0, 0x45c14f3c, 0x45c170be,
    0x45c19247, 0x45c1b3d5, 0x45c1d569, 0x45c1f702, 0x45c218a2, 0x45c23a47, 0x45c25bf2, 0x45c27da3,
    0x45c29f5a, 0x45c2c117, 0x45c2e2d9, 0x45c304a1, 0x45c32670, 0x45c34844, 0x45c36a1e, 0x45c38bfd,
    0x45c3ade3, 0x45c3cfcf, 0x45c3f1c0, 0x45c413b7, 0x45c435b5, 0x45c457b8, 0x45c479c1, 0x45c49bcf,
    0x45c4bde4, 0x45c4dfff, 0x45c50220, 0x45c52446, 0x45c54673, 0x45c568a5, 0x45c58add, 0x45c5ad1b,
    0x45c5cf60, 0x45c5f1aa, 0x45c613fa, 0x45c63650, 0x45c658ac, 0x45c67b0e, 0x45c69d75, 0x45c6bfe3,
    0x45c6e257, 0x45c704d1, 0x45c72751, 0x45c749d6, 0x45c76c62, 0x45c78ef4, 0x45c7b18b, 0x45c7d429,
    0x45c7f6cd, 0x45c81977, 0x45c83c26, 0x45c85edc, 0x45c88198, 0x45c8a459, 0x45c8c721, 0x45c8e9ef,
    0x45c90cc3, 0x45c92f9d, 0x45c9527d, 0x45c97563, 0x45c9984f, 0x45c9bb41, 0x45c9de39, 0x45ca0137,
    0x45ca243b, 0x45ca4746, 0x45ca6a56, 0x45ca8d6c, 0x45cab089, 0x45cad3ac, 0x45caf6d4, 0x45cb1a03,
    0x45cb3d38, 0x45cb6073, 0x45cb83b4, 0x45cba6fc, 0x45cbca49, 0x45cbed9c, 0x45cc10f6, 0x45cc3456,
    0x45cc57bc, 0x45cc7b28, 0x45cc9e9a, 0x45ccc212, 0x45cce590, 0x45cd0915, 0x45cd2ca0, 0x45cd5031,
    0x45cd73c8, 0x45cd9765, 0x45cdbb08, 0x45cddeb2, 0x45ce0262, 0x45ce2618, 0x45ce49d4, 0x45ce6d96,
    0x45ce915f, 0x45ceb52d, 0x45ced902, 0x45cefcde, 0x45cf20bf, 0x45cf44a7, 0x45cf6894, 0x45cf8c88,
    0x45cfb083, 0x45cfd483, 0x45cff88a, 0x45d01c97, 0x45d040aa, 0x45d064c4, 0x45d088e4, 0x45d0ad0a,
    0x45d0d136, 0x45d0f568, 0x45d119a1, 0x45d13de0, 0x45d16226, 0x45d18671, 0x45d1aac3, 0x45d1cf1c,
    0x45d1f37a, 0x45d217df, 0x45d23c4a, 0x45d260bc, 0x45d28534, 0x45d2a9b2, 0x45d2ce36, 0x45d2f2c1,
    0x45d31752, 0x45d33bea, 0x45d36088, 0x45d3852c, 0x45d3a9d6, 0x45d3ce87, 0x45d3f33e, 0x45d417fc,
    0x45d43cc0, 0x45d4618a, 0x45d4865b, 0x45d4ab32, 0x45d4d00f, 0x45d4f4f3, 0x45d519de, 0x45d53ece,
    0x45d563c5, 0x45d588c3, 0x45d5adc7, 0x45d5d2d1, 0x45d5f7e2, 0x45d61cf9, 0x45d64216, 0x45d6673b,
    0x45d68c65, 0x45d6b196, 0x45d6d6cd, 0x45d6fc0b, 0x45d7214f, 0x45d7469a, 0x45d76beb, 0x45d79143,
    0x45d7b6a1, 0x45d7dc05, 0x45d80171, 0x45d826e2, 0x45d84c5a, 0x45d871d9, 0x45d8975e, 0x45d8bce9,
    0x45d8e27b, 0x45d90814, 0x45d92db3, 0x45d95359, 0x45d97905, 0x45d99eb7, 0x45d9c471, 0x45d9ea30,
    0x45da0ff7, 0x45da35c3, 0x45da5b97, 0x45da8171, 0x45daa751, 0x45dacd38, 0x45daf326, 0x45db191a,
    0x45db3f15, 0x45db6516, 0x45db8b1e, 0x45dbb12d, 0x45dbd742, 0x45dbfd5e, 0x45dc2380, 0x45dc49a9,
    0x45dc6fd9, 0x45dc960f, 0x45dcbc4c, 0x45dce28f, 0x45dd08d9, 0x45dd2f2a, 0x45dd5581, 0x45dd7bdf,
    0x45dda244, 0x45ddc8af, 0x45ddef21, 0x45de159a, 0x45de3c19, 0x45de629f, 0x45de892c, 0x45deafbf,
    0x45ded659, 0x45defcfa, 0x45df23a1, 0x45df4a50, 0x45df7104, 0x45df97c0, 0x45dfbe82, 0x45dfe54b,
    0x45e00c1b, 0x45e032f1, 0x45e059ce, 0x45e080b2, 0x45e0a79d, 0x45e0ce8e, 0x45e0f586, 0x45e11c85,
    0x45e1438b, 0x45e16a97, 0x45e191ab, 0x45e1b8c5, 0x45e1dfe5, 0x45e2070d, 0x45e22e3b, 0x45e25570,
    0x45e27cac, 0x45e2a3ef, 0x45e2cb38, 0x45e2f289, 0x45e319e0, 0x45e3413e, 0x45e368a2, 0x45e3900e,
    0x45e3b780, 0x45e3defa, 0x45e4067a, 0x45e42e01, 0x45e4558e, 0x45e47d23, 0x45e4a4bf, 0x45e4cc61,
    0x45e4f40a, 0x45e51bba, 0x45e54371, 0x45e56b2f, 0x45e592f4, 0x45e5bac0, 0x45e5e292, 0x45e60a6c,
    0x45e6324c, 0x45e65a34, 0x45e68222, 0x45e6aa17, 0x45e6d213, 0x45e6fa16, 0x45e72220, 0x45e74a31,
    0x45e77249, 0x45e79a67, 0x45e7c28d, 0x45e7eaba, 0x45e812ed, 0x45e83b28, 0x45e8636a, 0x45e88bb2,
    0x45e8b402, 0x45e8dc58, 0x45e904b6, 0x45e92d1a, 0x45e95586, 0x45e97df8, 0x45e9a672, 0x45e9cef2,
    0x45e9f77a, 0x45ea2009, 0x45ea489e, 0x45ea713b, 0x45ea99df, 0x45eac289, 0x45eaeb3b, 0x45eb13f4,
    0x45eb3cb4, 0x45eb657b, 0x45eb8e49, 0x45ebb71e, 0x45ebdffa, 0x45ec08de, 0x45ec31c8, 0x45ec5aba,
    0x45ec83b2, 0x45ecacb2, 0x45ecd5b9, 0x45ecfec6, 0x45ed27db, 0x45ed50f8, 0x45ed7a1b, 0x45eda345,
    0x45edcc77, 0x45edf5af, 0x45ee1eef, 0x45ee4836, 0x45ee7184, 0x45ee9ada, 0x45eec436, 0x45eeed9a,
    0x45ef1704, 0x45ef4076, 0x45ef69ef, 0x45ef9370, 0x45efbcf7, 0x45efe686, 0x45f0101c, 0x45f039b9,
    0x45f0635d, 0x45f08d09, 0x45f0b6bc, 0x45f0e076, 0x45f10a37, 0x45f13400, 0x45f15dcf, 0x45f187a6,
    0x45f1b185, 0x45f1db6a, 0x45f20557, 0x45f22f4b, 0x45f25946, 0x45f28349, 0x45f2ad53, 0x45f2d764,
    0x45f3017c, 0x45f32b9c, 0x45f355c3, 0x45f37ff1, 0x45f3aa27, 0x45f3d464, 0x45f3fea8, 0x45f428f4,
    0x45f45347, 0x45f47da1, 0x45f4a803, 0x45f4d26c, 0x45f4fcdc, 0x45f52754, 0x45f551d3, 0x45f57c59,
    0x45f5a6e7, 0x45f5d17c, 0x45f5fc19, 0x45f626bc, 0x45f65168, 0x45f67c1a, 0x45f6a6d5, 0x45f6d196,
    0x45f6fc5f, 0x45f7272f, 0x45f75207, 0x45f77ce6, 0x45f7a7cd, 0x45f7d2bb, 0x45f7fdb1, 0x45f828ae,
    0x45f853b2, 0x45f87ebe, 0x45f8a9d1, 0x45f8d4ec, 0x45f9000e, 0x45f92b38, 0x45f95669, 0x45f981a2,
    0x45f9ace2, 0x45f9d82a, 0x45fa0379, 0x45fa2ed0, 0x45fa5a2e, 0x45fa8594, 0x45fab101, 0x45fadc76,
    0x45fb07f2, 0x45fb3376, 0x45fb5f01, 0x45fb8a94, 0x45fbb62f, 0x45fbe1d1, 0x45fc0d7a, 0x45fc392c,
    0x45fc64e4, 0x45fc90a5, 0x45fcbc6d, 0x45fce83c, 0x45fd1413, 0x45fd3ff2, 0x45fd6bd8, 0x45fd97c6,
    0x45fdc3bc, 0x45fdefb9, 0x45fe1bbe, 0x45fe47ca, 0x45fe73de, 0x45fe9ffa, 0x45fecc1d, 0x45fef848,
    0x45ff247b, 0x45ff50b5, 0x45ff7cf7, 0x45ffa941, 0x45ffd592, 0x460000f6, 0x46001726, 0x46002d5a,
    0x46004392, 0x460059ce, 0x4600700e, 0x46008652, 0x46009c99, 0x4600b2e4, 0x4600c933, 0x4600df87,
    0x4600f5dd, 0x46010c38, 0x46012297, 0x460138fa, 0x46014f60, 0x460165ca, 0x46017c38, 0x460192ab,
    0x4601a921, 0x4601bf9a, 0x4601d618, 0x4601ec9a, 0x4602031f, 0x460219a9, 0x46023036, 0x460246c8,
    0x46025d5d, 0x460273f6, 0x46028a93, 0x4602a134, 0x4602b7d9, 0x4602ce82, 0x4602e52e, 0x4602fbdf,
    0x46031294, 0x4603294c, 0x46034009, 0x460356c9, 0x46036d8d, 0x46038456, 0x46039b22, 0x4603b1f2,
    0x4603c8c6, 0x4603df9e, 0x4603f67b, 0x46040d5b, 0x4604243f, 0x46043b27, 0x46045212, 0x46046902,
    0x46047ff6, 0x460496ee, 0x4604adea, 0x4604c4ea, 0x4604dbee, 0x4604f2f5, 0x46050a01, 0x46052111,
    0x46053825, 0x46054f3d, 0x46056658, 0x46057d78, 0x4605949c, 0x4605abc4, 0x4605c2f0, 0x4605da20,
    0x4605f154, 0x4606088b, 0x46061fc7, 0x46063707, 0x46064e4b, 0x46066593, 0x46067cdf, 0x4606942f,
    0x4606ab84, 0x4606c2dc, 0x4606da38, 0x4606f198, 0x460708fd, 0x46072065, 0x460737d1, 0x46074f42,
    0x460766b6, 0x46077e2f, 0x460795ac, 0x4607ad2c, 0x4607c4b1, 0x4607dc3a, 0x4607f3c7, 0x46080b58,
    0x460822ed, 0x46083a87, 0x46085224, 0x460869c5, 0x4608816b, 0x46089915, 0x4608b0c2, 0x4608c874,
    0x4608e02a, 0x4608f7e4, 0x46090fa2, 0x46092765, 0x46093f2b, 0x460956f6, 0x46096ec4, 0x46098697,
    0x46099e6e, 0x4609b649, 0x4609ce28, 0x4609e60b, 0x4609fdf3, 0x460a15de, 0x460a2dce, 0x460a45c2,
    0x460a5dba, 0x460a75b6, 0x460a8db7, 0x460aa5bb, 0x460abdc4, 0x460ad5d1, 0x460aede2, 0x460b05f7,
    0x460b1e10, 0x460b362e, 0x460b4e50, 0x460b6675, 0x460b7ea0, 0x460b96ce, 0x460baf00, 0x460bc737,
    0x460bdf72, 0x460bf7b1, 0x460c0ff4, 0x460c283c, 0x460c4087, 0x460c58d7, 0x460c712b, 0x460c8984,
    0x460ca1e0, 0x460cba41, 0x460cd2a6, 0x460ceb0f, 0x460d037c, 0x460d1bee, 0x460d3464, 0x460d4cde,
    0x460d655d, 0x460d7ddf, 0x460d9666, 0x460daef1, 0x460dc781, 0x460de014, 0x460df8ac, 0x460e1149,
    0x460e29e9, 0x460e428e, 0x460e5b37, 0x460e73e4, 0x460e8c95, 0x460ea54b, 0x460ebe05, 0x460ed6c4,
    0x460eef86, 0x460f084d, 0x460f2119, 0x460f39e8, 0x460f52bc, 0x460f6b94, 0x460f8471, 0x460f9d52,
    0x460fb637, 0x460fcf20, 0x460fe80e, 0x46100100, 0x461019f6, 0x461032f1, 0x46104bf0, 0x461064f3,
    0x46107dfb, 0x46109707, 0x4610b018, 0x4610c92c, 0x4610e245, 0x4610fb63, 0x46111485, 0x46112dab,
    0x461146d5, 0x46116004, 0x46117937, 0x4611926f, 0x4611abab, 0x4611c4eb, 0x4611de30, 0x4611f779,
    0x461210c7, 0x46122a18, 0x4612436f, 0x46125cc9, 0x46127628, 0x46128f8c, 0x4612a8f4, 0x4612c260,
    0x4612dbd1, 0x4612f546, 0x46130ebf, 0x4613283d, 0x461341bf, 0x46135b46, 0x461374d1, 0x46138e61,
    0x4613a7f5, 0x4613c18d, 0x4613db2a, 0x4613f4cb, 0x46140e71, 0x4614281b, 0x461441ca, 0x46145b7d,
    0x46147535, 0x46148ef1, 0x4614a8b1, 0x4614c276, 0x4614dc40, 0x4614f60e, 0x46150fe0, 0x461529b7,
    0x46154392, 0x46155d72, 0x46157756, 0x4615913f, 0x4615ab2c, 0x4615c51e, 0x4615df14, 0x4615f90f,
    0x4616130e, 0x46162d12, 0x4616471a, 0x46166127, 0x46167b38, 0x4616954e, 0x4616af69, 0x4616c987,
    0x4616e3ab, 0x4616fdd3, 0x461717ff, 0x46173230, 0x46174c66, 0x461766a0, 0x461780de, 0x46179b22,
    0x4617b569, 0x4617cfb6, 0x4617ea07, 0x4618045c, 0x46181eb6, 0x46183914, 0x46185378, 0x46186ddf,
    0x4618884c, 0x4618a2bc, 0x4618bd32, 0x4618d7ac, 0x4618f22a, 0x46190cae, 0x46192735, 0x461941c2,
    0x46195c53, 0x461976e8, 0x46199183, 0x4619ac21, 0x4619c6c5, 0x4619e16d, 0x4619fc1a, 0x461a16cb,
    0x461a3181, 0x461a4c3b, 0x461a66fb, 0x461a81be, 0x461a9c87, 0x461ab754, 0x461ad226, 0x461aecfc,
    0x461b07d7, 0x461b22b7, 0x461b3d9b, 0x461b5884, 0x461b7372, 0x461b8e64, 0x461ba95b, 0x461bc457,
    0x461bdf57, 0x461bfa5c, 0x461c1566, 0x461c3075, 0x461c4b88, 0x461c66a0, 0x461c81bc, 0x461c9cdd,
    0x461cb803, 0x461cd32e, 0x461cee5d, 0x461d0991, 0x461d24ca, 0x461d4007, 0x461d5b4a, 0x461d7691,
    0x461d91dc, 0x461dad2d, 0x461dc882, 0x461de3dc, 0x461dff3a, 0x461e1a9e, 0x461e3606, 0x461e5172,
    0x461e6ce4, 0x461e885a, 0x461ea3d6, 0x461ebf55, 0x461edada, 0x461ef663, 0x461f11f2, 0x461f2d85,
    0x461f491c, 0x461f64b9, 0x461f805a, 0x461f9c00, 0x461fb7ab, 0x461fd35b, 0x461fef0f, 0x46200ac9,
    0x46202687, 0x4620424a, 0x46205e11, 0x462079de, 0x462095af, 0x4620b185, 0x4620cd60, 0x4620e940,
    0x46210525, 0x4621210e, 0x46213cfd, 0x462158f0, 0x462174e8, 0x462190e5, 0x4621ace7, 0x4621c8ed,
    0x4621e4f9, 0x46220109, 0x46221d1e, 0x46223938, 0x46225557, 0x4622717b, 0x46228da3, 0x4622a9d1,
    0x4622c603, 0x4622e23b, 0x4622fe77, 0x46231ab8, 0x462336fe, 0x46235349, 0x46236f99, 0x46238bed,
    0x4623a847, 0x4623c4a6, 0x4623e109, 0x4623fd71, 0x462419df, 0x46243651, 0x462452c8, 0x46246f44,
    0x46248bc5, 0x4624a84b, 0x4624c4d6, 0x4624e166, 0x4624fdfb, 0x46251a94, 0x46253733, 0x462553d7,
    0x4625707f, 0x46258d2d, 0x4625a9e0, 0x4625c697, 0x4625e354, 0x46260015, 0x46261cdc, 0x462639a7,
    0x46265678, 0x4626734d, 0x46269028, 0x4626ad07, 0x4626c9ec, 0x4626e6d5, 0x462703c4, 0x462720b7,
    0x46273db0, 0x46275aad, 0x462777b0, 0x462794b7, 0x4627b1c4, 0x4627ced6, 0x4627ebec, 0x46280908,
    0x46282629, 0x4628434f, 0x4628607a, 0x46287daa, 0x46289adf, 0x4628b819, 0x4628d558, 0x4628f29c,
    0x46290fe6, 0x46292d34, 0x46294a87, 0x462967e0, 0x4629853e, 0x4629a2a0, 0x4629c008, 0x4629dd75,
    0x4629fae7, 0x462a185e, 0x462a35da, 0x462a535c, 0x462a70e2, 0x462a8e6e, 0x462aabfe, 0x462ac994,
    0x462ae72f, 0x462b04cf, 0x462b2274, 0x462b401f, 0x462b5dce, 0x462b7b83, 0x462b993d, 0x462bb6fc,
    0x462bd4c0, 0x462bf289, 0x462c1057, 0x462c2e2b, 0x462c4c04, 0x462c69e2, 0x462c87c5, 0x462ca5ad,
    0x462cc39a, 0x462ce18d, 0x462cff85, 0x462d1d82, 0x462d3b84, 0x462d598c, 0x462d7798, 0x462d95aa,
    0x462db3c1, 0x462dd1dd, 0x462defff, 0x462e0e26, 0x462e2c52, 0x462e4a83, 0x462e68b9, 0x462e86f5,
    0x462ea536, 0x462ec37c, 0x462ee1c7, 0x462f0018, 0x462f1e6e, 0x462f3cc9, 0x462f5b29, 0x462f798f,
    0x462f97fa, 0x462fb66a, 0x462fd4e0, 0x462ff35b, 0x463011db, 0x46303060, 0x46304eeb, 0x46306d7a,
    0x46308c10, 0x4630aaaa, 0x4630c94a, 0x4630e7ef, 0x4631069a, 0x46312549, 0x463143ff, 0x463162b9,
], dtype=np.uint32).view(np.float32)
R_MAX = np.float32(1.0 - 2.0 ** -24)  # the interpolation fraction is kept below 1
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


def kscale32(temperature: float) -> np.float32:
    """K = kappa * 1024 (exact: a power-of-two scaling), so that t = fl(x * K) = fl(x * kappa) * 1024."""
    return np.float32(kappa32(temperature) * np.float32(1024.0))


def sampled_row(temperature: float) -> bool:
    """A row samples when T > 0 and K is finite (T below ~4.3e-36 makes it greedy)."""
    return bool(f32(temperature) > 0) and bool(np.isfinite(kscale32(temperature)))


def t_units(x: torch.Tensor, temperature: float) -> torch.Tensor:
    """t = clamp(fl(x * K), -2^30, 2^30): x / T in units of 2^-10 powers of two (a = t / 1024 exactly)."""
    t = x.to(torch.float32) * torch.tensor(kscale32(temperature), dtype=torch.float32)
    return t.clamp(-T_CLAMP, T_CLAMP)


def exp2_table(t: torch.Tensor):
    """(q, mu) of t: q = floor(t) (n = q >> 10 = floor(a), fine bin = q >> 4 = floor(a * 64)) and
    mu = (uint32)(fl(fl(r * TAB_S[j]) + TAB_T[j])), j = q & 1023, r = min(fl(t - floor(t)), 1 - 2^-24):
    2^(a - n) * 2^23 to ~1.7e-7, in [2^23, 2^24]."""
    t = t.to(torch.float32)
    fl = torch.floor(t)
    q = fl.to(torch.int64)
    r = torch.minimum(t - fl, torch.tensor(R_MAX))
    j = q & 1023
    m = r * torch.from_numpy(TAB_S)[j]
    m = m + torch.from_numpy(TAB_T)[j]
    mu = m.to(torch.int64)
    return q, mu


def mantissa(t: torch.Tensor):
    """(n, mu): n = floor(a) = q >> 10, mu = 24-bit mantissa of 2^(a - n)."""
    q, mu = exp2_table(t)
    return q >> 10, mu


def min_p_cut(t_max: float, min_p: float) -> np.float32:
    """t_cut = fl((double)(t_max / 1024) + log2(min_p)) * 1024: min_p keeps t >= t_cut (a >= a_max + log2(min_p))."""
    a_max = float(np.float32(t_max) / np.float32(1024.0))
    return np.float32(np.float32(a_max + math.log2(float(f32(min_p)))) * np.float32(1024.0))


@dataclass
class RowResult:
    token: int
    kept: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int64))     # kept token ids, rank order
    weights: list = field(default_factory=list)                                 # their weights (python ints)
    S2: int = 0
    greedy: bool = False

    def probs(self) -> dict:
        return {int(i): (w / self.S2) for i, w in zip(self.kept, self.weights) if w > 0}


def _prefix_first(ws, target: int, strict: bool) -> int:
    """First position j with inclusive prefix sum of ws (non-negative ints < 2^62) >= target (strict=False)
    or > target (strict=True).  Exact: prefix sums in two 31-bit halves (int64), compared as python ints."""
    w = np.asarray(ws, dtype=np.int64)
    clo, chi = np.cumsum(w & 0x7FFFFFFF), np.cumsum(w >> 31)
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


def _exact_sum(w: np.ndarray) -> int:
    """Exact sum of non-negative int64 values < 2^62 (two 31-bit halves)."""
    w = np.asarray(w, dtype=np.int64)
    return int((w & 0x7FFFFFFF).sum()) + (int((w >> 31).sum()) << 31)


def distribution(x: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0, min_p: float = 0.0):
    """Kept candidates of a processed row in rank order with their weights: (ids int64 [n], weights list[int], S2)."""
    cand = torch.nonzero(x != -math.inf).flatten()
    if cand.numel() == 0:
        return None
    xc = x[cand]
    order = rank_order(xc, cand)
    ids = cand[order]
    t = t_units(x[ids], temperature)
    if f32(min_p) > 0:
        keep = t >= torch.tensor(min_p_cut(float(t[0]), min_p))
        ids, t = ids[keep], t[keep]
    if top_k > 0 and top_k < ids.numel():
        ids, t = ids[:top_k], t[:top_k]
    n, mu = mantissa(t)
    N = int(n[0])
    sh = n - N + D_EXP
    w_t = torch.where(sh >= 0, mu << sh.clamp_min(0), torch.zeros_like(mu)).numpy()
    S = _exact_sum(w_t)
    tp = f32(top_p)
    if tp < f32(1.0):
        TP = math.floor(float(tp) * 2 ** 32)
        thr = -((-TP * S) >> 32)
        j = _prefix_first(w_t, thr, strict=False)
        ids, w_t = ids[: j + 1], w_t[: j + 1]
    return ids.numpy(), w_t.tolist(), _exact_sum(w_t)


def draw_index_order(ids: np.ndarray, ws: Sequence[int], S2: int, u24: int) -> int:
    """Inverse CDF in index order: the smallest kept id whose prefix sum exceeds floor(u24 * S2 / 2^24)."""
    t = (int(u24) * int(S2)) >> 24
    o = np.argsort(ids, kind="stable")
    j = _prefix_first(np.asarray(ws, dtype=np.int64)[o], t, strict=True)
    return int(ids[o[j]])


def sample_row(logits: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0, min_p: float = 0.0,
               seed: int = 0, position: int = 0, stream: int = ST_FIRST, row_key: int = 0,
               procs: Optional[RowProcs] = None, drafts_before: Sequence[int] = ()) -> RowResult:
    """One row: processors, then greedy (temperature <= 0) or the sampled token."""
    x = process(logits, procs, drafts_before)
    if not sampled_row(temperature):
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
    """floor(q * S2) exactly for an fp32 probability q (NaN and q <= 0 count as 0, q >= 1 as 1)."""
    qd = float(f32(q))
    if not qd > 0.0:
        return 0
    if qd >= 1.0:
        return int(S2)
    m, e = math.frexp(qd)  # qd = m * 2^e, m in [0.5, 1)
    M = int(m * (1 << 53))
    s = 53 - e
    return (M * S2) >> s if s >= 0 else (M * S2) << (-s)


@dataclass
class VerifyResult:
    tokens: list
    accepted: int   # emitted tokens = accepted drafts + 1


def draft_params(temperature: float, top_k: int, top_p: float, draft_sample: int = 1, draft_temperature: float = 0.0,
                 draft_top_k: int = 0, draft_top_p: float = 0.0):
    """The drafter's (temperature, top_k, top_p) of make_sampp (engine/src/mtp_sample.cu:379-383): the draft values
    where set, else the target's; top_k = 1 (q = the point mass at the argmax) unless draft_sample; no min_p
    (k_topk2 applies min_p to the target rows only, :159)."""
    t = draft_temperature if draft_temperature > 0 else temperature
    k = (draft_top_k if draft_top_k > 0 else top_k) if draft_sample else 1
    return t, k, (draft_top_p if draft_top_p > 0 else top_p)


def verify_seq(target_logits: torch.Tensor, draft_probs: torch.Tensor, idmap: np.ndarray, drafts: Sequence[int],
               temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0, min_p: float = 0.0, seed: int = 0,
               position: int = 0, row_key: int = 0, procs: Optional[RowProcs] = None, test_flags: int = 0,
               n_chain: Optional[int] = None) -> VerifyResult:
    """One sequence: target rows [K+1][V], draft probabilities [K][Vd] over the reduced vocabulary with
    token ids idmap[Vd], draft tokens d_1..d_K (engine/src/mtp_sample.cu:227-258).  Drafts t >= n_chain are delta
    proposals (k_delta_q, engine/src/mtp_sample.cu:286-296: q = 1 at the draft, 0 elsewhere; their draft_probs
    rows are not read), so they are accepted with probability p(d) and a rejection draws from p without d."""
    K = len(drafts)
    inv = {int(t): j for j, t in enumerate(np.asarray(idmap).tolist())}
    out = []
    for t in range(K + 1):
        x = process(target_logits[t], procs, list(drafts[:t]))
        if not bool((x != -math.inf).any()):
            d = None
        elif not sampled_row(temperature):  # a greedy row is p = the argmax with weight 1
            d = (np.array([greedy(x)], dtype=np.int64), [1], 1)
        else:
            d = distribution(x, temperature, top_k, top_p, min_p)
        if d is None:  # no candidate
            out.append(greedy(x))
            return VerifyResult(out, len(out))
        ids, ws, S2 = d
        r = philox(position, ST_ACCEPT + t, row_key, 0, seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)
        u_acc, u_res = int(r[0] >> np.uint64(8)), int(r[1] >> np.uint64(8))
        if t == K:  # every draft accepted: bonus token from the last row
            out.append(draw_index_order(ids, ws, S2, u_res))
            return VerifyResult(out, len(out))
        dt = int(drafts[t])
        delta = n_chain is not None and t >= n_chain
        qrow = None if delta else draft_probs[t].numpy()

        def qof(i):
            if delta:
                return 1.0 if int(i) == dt else 0.0
            return float(qrow[inv[int(i)]]) if int(i) in inv else 0.0
        qd = qof(dt)
        wd = 0
        pos = np.nonzero(ids == dt)[0]
        if len(pos):
            wd = ws[int(pos[0])]
        if u_acc * q_fix(qd, S2) < wd * (1 << 24):
            out.append(dt)
            continue
        res = ws
        if not (test_flags & 1):
            res = [max(0, w - q_fix(qof(i), S2)) for i, w in zip(ids, ws)]
            if sum(res) == 0:
                res = ws
        out.append(draw_index_order(ids, res, sum(res), u_res))
        return VerifyResult(out, len(out))
    raise AssertionError("unreachable")
