"""Host side of the MI355X sampling stage: the reference's Python-facing sampling contract over libqws.

Mirrors, with the same names, argument meanings and error behaviour:
  * Sampling / make_sampling               engine/spec.py:40-46
  * Procs / make_procs                     engine/spec.py:49-67
  * GenParams.procs (processor gating)     server/smk_runner.py:52-76
  * check_supported (request validation)   server/smk_core_client.py:37-72
  * SeqSampler.set_sampling / set_procs / proc_state / test_draw
                                           engine/spec.py:276-311 (SpecEngine's sampling surface)
  * Runner._begin's parameter mapping      server/smk_runner.py:597-607
and adds the batched entry the server's batch loop calls once per decode step (Sampler.sample), which
replaces the reference's per-sequence kernel launches (engine/src/batch.cu:210-246).

Device work is one qws_sample call on the current torch stream; nothing here computes a token on the CPU.
"""
from __future__ import annotations

import ctypes as C
import math
import random
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import (DTYPE_BF16, DTYPE_F32, MASK_ALLOWED, MASK_BANNED, MASK_NONE, ST_ACCEPT, ST_DRAFT, ST_DRAW, ST_FIRST, TF_BROKEN, TF_RESCAN, TF_SPLIT_SELECT, TF_STAGED_DRAW,
                   Batch, Procs, Row, Sampling, VerifyBatch, check)

VOCAB = 248320
LOGIT_BIAS_MAX = 1024     # server/smk_core_client.py:33
REF_MAX_TOP_K = 64        # server/smk_runner.py:48 (the reference sampler's cap; see GenParams.cap64)
HIST_MAX = 65535          # generated tokens + drafts per row the per-chunk tables count
BIAS_MAX_ROW = 2047       # bias entries per row


class ValidationError(ValueError):
    """A rejected request parameter (the reference answers HTTP 400 naming it: server/smk_core_client.py:37-72)."""

    def __init__(self, msg, parameter=None, value=None):
        super().__init__(msg)
        self.parameter, self.value = parameter, value


# ---------------------------------------------------------------------------------------------- reference structs
def make_sampling(temperature=0.0, top_k=20, top_p=1.0, draft_sample=1, draft_temperature=0.0, draft_top_k=0, draft_top_p=0.0, seed=0,
                  test_flags=0, min_p=0.0) -> Sampling:
    """engine/spec.py:45-46."""
    return Sampling(temperature, top_k, top_p, draft_sample, draft_temperature, draft_top_k, draft_top_p, test_flags, seed, min_p)


def make_procs(prompt=(), presence=0.0, frequency=0.0, repetition=1.0, min_tokens=0, bias=None, allowed=None, stop=()):
    """engine/spec.py:56-67: returns (Procs, keepalive); bias = {token id: value}, allowed = token ids
    (None / empty: unrestricted), stop = ids masked by min_tokens."""
    def ints(x):
        a = np.ascontiguousarray(np.asarray(list(x), dtype=np.int32))
        return a, a.ctypes.data_as(C.POINTER(C.c_int)), len(a)

    pr, bi, al, st = ints(prompt), ints((bias or {}).keys()), ints(allowed or ()), ints(stop)
    bv = np.ascontiguousarray(np.asarray(list((bias or {}).values()), dtype=np.float32))
    keep = [pr[0], bi[0], al[0], st[0], bv]
    p = Procs(presence, frequency, repetition, min_tokens, pr[1], pr[2], bi[1], bv.ctypes.data_as(C.POINTER(C.c_float)), bi[2], al[1], al[2], st[1], st[2])
    return p, keep


# ---------------------------------------------------------------------------------------------- request parameters
@dataclass
class GenParams:
    """server/smk_runner.py:52-76 (the sampling part).  cap64 = True reproduces the reference sampler's
    top-k semantics (top_k <= 0 means its 64 best candidates; top_k > 64 is rejected); the default is the
    full-vocabulary vLLM semantics (top_k <= 0 = no top-k filter)."""
    max_tokens: int = 16
    eos: Optional[int] = None
    stop_ids: frozenset = frozenset()
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    seed: Optional[int] = None
    min_p: float = 0.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    min_tokens: int = 0
    min_tokens_ids: frozenset = frozenset()
    logit_bias: Optional[dict] = None
    allowed_token_ids: Optional[tuple] = None
    cap64: bool = False

    def procs(self, prompt_ids):
        """make_procs arguments of the elementwise processors, None when none is active (min_p is a sampler parameter)."""
        if not (self.presence_penalty or self.frequency_penalty or self.repetition_penalty != 1.0 or self.min_tokens or self.logit_bias
                or self.allowed_token_ids):
            return None
        return dict(prompt=prompt_ids, presence=self.presence_penalty, frequency=self.frequency_penalty, repetition=self.repetition_penalty,
                    min_tokens=self.min_tokens, bias=self.logit_bias, allowed=self.allowed_token_ids, stop=sorted(self.min_tokens_ids))


def _bias_ids(lb):
    """logit_bias keys as token ids (JSON gives strings); None when one is not an integer."""
    try:
        return [int(t) for t in lb]
    except (TypeError, ValueError):
        return None


def check_supported(p: GenParams, vocab: int = VOCAB):
    """server/smk_core_client.py:37-72: rejects what the sampler cannot do, naming the parameter, plus the request
    limits the reference documents (docs/USAGE.md:80-87) and its server answers with HTTP 400
    (tests/test_sampling_params.py:209-226, tests/test_server_seed.py:10-11)."""
    if p.cap64 and p.top_k > REF_MAX_TOP_K:
        raise ValidationError(f"top_k must be <= {REF_MAX_TOP_K} (0 or -1 = no top-k filter), got {p.top_k}", "top_k", p.top_k)
    if p.top_k < -1:
        raise ValidationError(f"top_k must be -1 or 0 (no top-k filter) or at least 1, got {p.top_k}", "top_k", p.top_k)
    if not (p.temperature >= 0.0 and math.isfinite(p.temperature)):
        raise ValidationError(f"temperature must be finite and >= 0, got {p.temperature}", "temperature", p.temperature)
    if not (0.0 < p.top_p <= 1.0):
        raise ValidationError(f"top_p must be in (0, 1], got {p.top_p}", "top_p", p.top_p)
    if not (0.0 <= p.min_p <= 1.0):
        raise ValidationError(f"min_p must be in [0, 1], got {p.min_p}", "min_p", p.min_p)
    for name in ("presence_penalty", "frequency_penalty"):
        v = getattr(p, name)
        if not -2.0 <= v <= 2.0:
            raise ValidationError(f"{name} must be in [-2, 2], got {v}", name, v)
    if not (p.repetition_penalty > 0.0 and math.isfinite(p.repetition_penalty)):
        raise ValidationError(f"repetition_penalty must be > 0, got {p.repetition_penalty}", "repetition_penalty", p.repetition_penalty)
    if p.min_tokens < 0:
        raise ValidationError(f"min_tokens must be >= 0, got {p.min_tokens}", "min_tokens", p.min_tokens)
    if p.max_tokens is not None and p.min_tokens > p.max_tokens:
        raise ValidationError(f"min_tokens must be <= max_tokens ({p.max_tokens}), got {p.min_tokens}", "min_tokens", p.min_tokens)
    lb = p.logit_bias
    if lb:
        if len(lb) > LOGIT_BIAS_MAX:
            raise ValidationError(f"logit_bias has {len(lb)} entries, at most {LOGIT_BIAS_MAX} are supported", "logit_bias", len(lb))
        ids = _bias_ids(lb)
        if ids is None or any(not 0 <= t < vocab for t in ids) or any(not math.isfinite(v) for v in lb.values()):
            raise ValidationError(f"logit_bias: token ids must be integers in [0, {vocab}) and values finite", "logit_bias", len(lb))
    al = p.allowed_token_ids
    if al is not None and len(al) == 0:
        raise ValidationError("allowed_token_ids must not be empty", "allowed_token_ids", 0)
    if al:
        if len(al) > vocab or any(not 0 <= int(t) < vocab for t in al):
            raise ValidationError(f"allowed_token_ids: at most {vocab} ids, each in [0, {vocab})", "allowed_token_ids", len(al))
        if p.min_tokens and set(al) <= set(p.min_tokens_ids):
            raise ValidationError("min_tokens masks the stop tokens, but every allowed_token_ids entry is a stop token: nothing could be generated",
                                  "min_tokens", p.min_tokens)


# ---------------------------------------------------------------------------------------------- rows
@dataclass
class RowSpec:
    """One logits row of a batched call: sampling parameters, Philox counter and processor state (include/qws.h qws_row)."""
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    seed: int = 0
    position: int = 0
    stream: int = ST_FIRST
    row_key: int = 0
    presence: float = 0.0
    frequency: float = 0.0
    repetition: float = 1.0
    min_tokens: int = 0
    prompt: Sequence[int] = ()
    gen: Sequence[int] = ()
    ngen: Optional[int] = None
    drafts: Sequence[int] = ()
    bias: Optional[dict] = None
    allowed: Optional[Sequence[int]] = None
    banned: Optional[np.ndarray] = None
    stop: Sequence[int] = ()
    test_flags: int = 0
    draw_word: int = 0  # Philox output word of the row's draw (1 for verify rows: the residual / bonus word)
    state_slot: int = -1  # >= 0: the prompt set and generated counts come from this slot of the batch's ProcState

    def procs_on(self) -> bool:
        """engine/src/proc.cu:149 (any elementwise processor active), plus the banned bitmask."""
        return bool(self.presence != 0.0 or self.frequency != 0.0 or self.repetition != 1.0 or self.min_tokens > 0 or self.bias
                    or (self.allowed is not None and len(self.allowed) > 0) or self.banned is not None)


def row_from_params(p: GenParams, prompt_ids=(), gen_ids=(), position=0, row_key=0, seed=None) -> RowSpec:
    """server/smk_runner.py:597-607: a request's GenParams -> the row the sampler runs.  Greedy with
    processors is the argmax of the processed logits (the reference runs it as top_k = 1 sampling)."""
    check_supported(p)
    pr = p.procs(list(prompt_ids)) or {}
    if p.temperature > 0:
        s = p.seed if p.seed is not None else (seed if seed is not None else random.getrandbits(62))
        top_k = p.top_k if p.top_k > 0 else (REF_MAX_TOP_K if p.cap64 else 0)
        r = RowSpec(temperature=p.temperature, top_k=top_k, top_p=p.top_p, min_p=p.min_p, seed=s)
    else:
        r = RowSpec(temperature=0.0)
    r.position, r.row_key, r.gen = position, row_key, list(gen_ids)
    if pr:
        r.prompt, r.presence, r.frequency, r.repetition = list(pr["prompt"]), pr["presence"], pr["frequency"], pr["repetition"]
        r.min_tokens, r.allowed, r.stop = pr["min_tokens"], pr["allowed"], list(pr["stop"])
        # integer ids, values clamped to [-100, 100] (docs/USAGE.md:84)
        r.bias = {int(t): min(max(float(v), -100.0), 100.0) for t, v in pr["bias"].items()} if pr["bias"] else None
    return r


def draft_row(temperature=0.0, top_k=20, top_p=1.0, draft_sample=1, draft_temperature=0.0, draft_top_k=0, draft_top_p=0.0, seed=0, j=1,
              position=0, row_key=0) -> RowSpec:
    """The drafter's row for draft j of a cycle (make_sampp's draft parameters, engine/src/mtp_sample.cu:375-387, and
    k_draft_pick's stream ST_DRAFT + j, :280-284): temperature = draft_temperature, else temperature; top_k =
    draft_top_k, else top_k, when draft_sample (1 otherwise: q is the point mass at the argmax); top_p = draft_top_p,
    else top_p; no min_p and no processors (they apply to the target rows only).  include/qws.h qws_row_init_pick
    (QWS_PICK_DRAFT) fills the C row the same way."""
    t = draft_temperature if draft_temperature > 0 else temperature
    k = (draft_top_k if draft_top_k > 0 else top_k) if draft_sample else 1
    p = draft_top_p if draft_top_p > 0 else top_p
    return RowSpec(temperature=t, top_k=k, top_p=p, min_p=0.0, seed=seed, position=position, stream=ST_DRAFT + int(j), row_key=row_key)


def _ids(ids, V, name) -> np.ndarray:
    """Token ids (a list, tuple, set, dict keys, numpy array or tensor) as one int64 array in iteration order, converted
    once; ValidationError unless every id is an integer in [0, V) (a float or bool array is refused, not truncated)."""
    if isinstance(ids, torch.Tensor):
        if ids.numel() and (ids.dtype == torch.bool or ids.dtype.is_floating_point or ids.dtype.is_complex):  # empty: any dtype
            raise ValidationError(f"{name}: token ids must be integers, got a {ids.dtype} tensor", name)
        a = ids.detach().reshape(-1).to("cpu", torch.int64).numpy()
    elif isinstance(ids, np.ndarray):
        if ids.size and not np.issubdtype(ids.dtype, np.integer):  # empty: any dtype
            raise ValidationError(f"{name}: token ids must be integers, got a {ids.dtype} array", name)
        a = ids.reshape(-1).astype(np.int64, copy=False)
    else:
        # the element types checked once per distinct type (a C-speed pass), then one conversion
        seq = ids if isinstance(ids, (list, tuple)) else list(ids)
        if not all(_int_type(tp) for tp in set(map(type, seq))):
            raise ValidationError(f"{name}: token ids must be integers", name)
        try:
            a = np.fromiter(seq, dtype=np.int64, count=len(seq))
        except (TypeError, ValueError, OverflowError):
            raise ValidationError(f"{name}: token ids must be integers", name) from None
    if a.size and (a.min() < 0 or a.max() >= V):
        raise ValidationError(f"{name}: token ids must be in [0, {V})", name)
    return a


def _int_type(tp) -> bool:
    """The type of one id of a Python container: an int or a numpy integer (not a bool, a float or a string)."""
    return issubclass(tp, (int, np.integer)) and not issubclass(tp, (bool, np.bool_))


def penalties_need_state(r: "RowSpec") -> bool:
    """A row whose penalties count generated tokens (repetition, presence or frequency active) and whose history is
    not a state slot: a step taken on the device (advance, qws_finish_rows) cannot extend its CSR history, so its
    counts would miss the drawn tokens."""
    return r.procs_on() and int(r.state_slot) < 0 and (r.repetition != 1.0 or r.presence != 0.0 or r.frequency != 0.0)


class PackedBatch:
    """Rows packed into device arrays (CSR histories, bias, stop ids, masks) and the qws_batch struct.  Rows with a
    state_slot take their prompt set and generated counts from `state` (a ProcState) instead of a CSR history:
    their prompt / gen lists are not packed, and ngen (for min_tokens) is r.ngen, else len(r.gen)."""

    def __init__(self, rows: Sequence[RowSpec], V: int, device, state: Optional["ProcState"] = None):
        self.B, self.V = len(rows), V
        self.state = state
        if state is not None and state.V != V:
            raise ValidationError(f"the ProcState holds V={state.V}, the batch V={V}", "state")
        W = (V + 31) // 32
        hr, hist, drafts, bids, bvals, stops, masks = [], [], [], [], [], [], []
        nh = nd = 0  # entries of hist and drafts so far
        for r in rows:
            if not (r.repetition > 0.0) or r.min_tokens < 0:
                raise ValidationError("repetition must be > 0 and min_tokens >= 0", "repetition_penalty", r.repetition)
            if not (0.0 < r.top_p <= 1.0) or not (0.0 <= r.min_p <= 1.0):
                raise ValidationError("top_p must be in (0, 1] and min_p in [0, 1]", "top_p", r.top_p)
            prompt, gen, rdrafts, rstop = (_ids(r.prompt, V, "prompt"), _ids(r.gen, V, "gen"), _ids(r.drafts, V, "drafts"),
                                           _ids(r.stop, V, "stop"))
            allowed = _ids(r.allowed, V, "allowed") if r.allowed is not None else None
            if allowed is not None and allowed.size == 0:
                allowed = None  # an empty allowed list masks nothing
            bkeys = _ids((r.bias or {}).keys(), V, "logit_bias")
            ng = len(gen) if r.ngen is None else int(r.ngen)
            st = int(r.state_slot)
            if st >= 0 and (state is None or st >= state.slots):
                raise ValidationError(f"state_slot {st} needs a ProcState with more than {st} slots", "state_slot", st)
            if len(gen) + len(rdrafts) > HIST_MAX:
                raise ValidationError(f"history longer than {HIST_MAX} tokens", "history", len(gen) + len(rdrafts))
            nb = len(r.bias or {})
            if nb > BIAS_MAX_ROW:
                raise ValidationError(f"logit_bias has {nb} entries, at most {BIAS_MAX_ROW} per row", "logit_bias", nb)
            row = Row()
            on = r.procs_on()
            row.temperature, row.top_k, row.top_p, row.min_p = r.temperature, r.top_k, r.top_p, r.min_p
            row.log2_min_p = math.log2(float(np.float32(r.min_p))) if r.min_p > 0 else 0.0
            row.seed, row.position, row.stream, row.row_key = int(r.seed) & (2 ** 64 - 1), r.position & 0xFFFFFFFF, r.stream, r.row_key & 0xFFFFFFFF
            row.proc_on = int(on)
            row.presence, row.frequency, row.repetition, row.min_tokens, row.ngen = r.presence, r.frequency, r.repetition, r.min_tokens, ng
            row.test_flags, row.draw_word = r.test_flags, r.draw_word
            row.state_slot = st if st >= 0 else -1
            if on:
                row.hist_off = nh
                if st < 0:
                    row.n_prompt, row.n_gen = len(prompt), len(gen)
                    hist += [prompt, gen]
                    nh += len(prompt) + len(gen)
                row.draft_off, row.n_drafts = nd, len(rdrafts)
                drafts.append(rdrafts)
                nd += len(rdrafts)
                row.bias_off, row.n_bias = len(bids), nb
                bids += bkeys.tolist()
                bvals += [float(v) for v in (r.bias or {}).values()]
                row.stop_off, row.n_stop = len(stops), len(rstop)
                stops += rstop.tolist()
                if allowed is not None:
                    m = np.zeros(W, np.uint32)
                    a = allowed
                    np.bitwise_or.at(m, a >> 5, (np.uint32(1) << (a & 31).astype(np.uint32)))
                    if r.banned is not None:
                        m &= ~np.asarray(r.banned, dtype=np.uint32)[:W]
                    row.mask_mode, row.mask_row = MASK_ALLOWED, len(masks)
                    masks.append(m)
                elif r.banned is not None:
                    row.mask_mode, row.mask_row = MASK_BANNED, len(masks)
                    masks.append(np.asarray(r.banned, dtype=np.uint32)[:W])
            hr.append(row)
        dev = torch.device(device)

        def arr(a, dt):  # one element at least, so that every array has a device address
            return np.concatenate(a).astype(dt) if a and isinstance(a[0], np.ndarray) else (np.asarray(a, dtype=dt) if len(a) else np.zeros(1, dt))

        # every array in one host buffer (256-byte aligned parts) and one host-to-device copy; the device arrays are
        # views of it
        parts = [np.frombuffer((Row * self.B)(*hr), dtype=np.uint8), arr(hist, np.int32), arr(drafts, np.int32), arr(bids, np.int32),
                 arr(bvals, np.float32), arr(stops, np.int32), np.stack(masks).astype(np.uint32) if masks else np.zeros(0, np.uint32)]
        offs, n = [], 0
        for a in parts:
            offs.append(n)
            n += (a.nbytes + 255) & ~255
        buf = np.zeros(max(n, 256), np.uint8)
        for a, o in zip(parts, offs):
            buf[o:o + a.nbytes] = a.reshape(-1).view(np.uint8)
        self.dev_buf = torch.from_numpy(buf).to(dev)
        view = [self.dev_buf[o:o + a.nbytes] for a, o in zip(parts, offs)]
        self.rows_t = view[0]
        self.hist_t, self.drafts_t, self.bids_t = view[1].view(torch.int32), view[2].view(torch.int32), view[3].view(torch.int32)
        self.bvals_t, self.stops_t = view[4].view(torch.float32), view[5].view(torch.int32)
        self.masks_t = view[6].view(torch.int32).reshape(len(masks), W) if masks else None
        self.W = W
        self.host_rows = hr
        self.specs = list(rows)

    def check_advance(self):
        """The rows may take their decode step on the device (qws_batch.advance, qws_finish_rows): distinct state slots,
        and penalties that count generated tokens kept in a state slot (penalties_need_state)."""
        slots = [r.state_slot for r in self.host_rows if r.state_slot >= 0]
        if len(set(slots)) != len(slots):
            raise ValidationError("advance needs distinct state slots across the batch's rows", "state_slot")
        if any(penalties_need_state(r) for r in self.specs):
            raise ValidationError("a row whose penalties count generated tokens must keep them in a state slot (ProcState) to take its "
                                  "step on the device: its CSR history would miss the drawn tokens", "state_slot")

    def batch(self, logits: torch.Tensor, out_tokens: torch.Tensor, out_logits=None, out_probs=None, out_info=None, row_stride=None,
              advance: bool = False) -> Batch:
        """The call's qws_batch.  advance=True: every row that draws a token also takes the step on the device (the token
        noted in its state slot, its ngen and position incremented in this batch's device row array, include/qws.h
        qws_batch.advance); the rows' state slots must then be distinct."""
        if advance:
            self.check_advance()
        b = Batch()
        b.logits = logits.data_ptr()
        b.dtype = DTYPE_BF16 if logits.dtype == torch.bfloat16 else DTYPE_F32
        b.B, b.V = self.B, self.V
        b.row_stride = logits.stride(0) if row_stride is None else row_stride
        b.rows, b.hist, b.drafts = self.rows_t.data_ptr(), self.hist_t.data_ptr(), self.drafts_t.data_ptr()
        b.bias_ids, b.bias_vals, b.stop_ids = self.bids_t.data_ptr(), self.bvals_t.data_ptr(), self.stops_t.data_ptr()
        b.masks = self.masks_t.data_ptr() if self.masks_t is not None else None
        b.mask_words = self.W
        b.out_tokens = out_tokens.data_ptr()
        b.out_logits = out_logits.data_ptr() if out_logits is not None else None
        b.out_probs = out_probs.data_ptr() if out_probs is not None else None
        b.out_info = out_info.data_ptr() if out_info is not None else None
        if self.state is not None:
            b.state_mem, b.state_slots = self.state.mem.data_ptr(), self.state.slots
        b.advance = int(bool(advance))
        return b


class ProcState:
    """Device-resident per-request processor state (include/qws.h qws_state_*): the reference's proc_begin /
    proc_note (engine/src/proc.cu:72-103, engine/src/proc.h:52-56) kept on the GPU across decode steps.  Each of
    `slots` slots holds one request's prompt set and generated-token counts as touched-token tables per 8,192-token
    block, so a sampling call reads its block's entries instead of the request's whole history.  A row names its
    slot in RowSpec.state_slot; the PackedBatch is built with state=this."""

    def __init__(self, slots: int, V: int = VOCAB, device="cuda"):
        self.lib = _lib.load()
        self.slots, self.V = int(slots), int(V)
        n = self.lib.qws_state_bytes(self.slots, self.V)
        if n == 0:
            raise ValidationError(f"no state arena for slots={slots}, V={V}", "slots")
        self.device = torch.device(device)
        self.mem = torch.empty(n, dtype=torch.uint8, device=self.device)

    def _stream(self):
        return C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def begin(self, slot: int, prompt=(), gen=()):
        """engine/src/proc.cu:72-103 for the penalties' state: slot <- the prompt set and the counts of `gen`
        (ids validated as ids_ok, engine/src/proc.cu:55-59)."""
        if not 0 <= slot < self.slots:
            raise ValidationError(f"slot must be in [0, {self.slots}), got {slot}", "slot", slot)
        prompt, gen = _ids(prompt, self.V, "prompt"), _ids(gen, self.V, "gen")
        if len(gen) > HIST_MAX - 64:
            raise ValidationError(f"at most {HIST_MAX - 64} generated tokens per slot", "gen", len(gen))
        pr = torch.as_tensor(prompt.astype(np.int32) if len(prompt) else np.zeros(1, np.int32)).to(self.device)
        ge = torch.as_tensor(gen.astype(np.int32) if len(gen) else np.zeros(1, np.int32)).to(self.device)
        check(self.lib.qws_state_begin(self.mem.data_ptr(), self.slots, self.V, int(slot), pr.data_ptr(), len(prompt), ge.data_ptr(), len(gen),
                                       self._stream()), "qws_state_begin")

    def note(self, slots, tokens: torch.Tensor):
        """engine/src/proc.h:52-56: adds tokens[b] (int32 [B] or [B, T] on the GPU, entries outside [0, V) skipped:
        the -1 after a verify call's emitted tokens) to slot slots[b] (distinct slots, or -1 to skip a row)."""
        if tokens.dtype != torch.int32 or tokens.device.type != "cuda":
            raise ValidationError("tokens must be an int32 CUDA tensor", "tokens")
        tok = tokens.reshape(tokens.shape[0], -1).contiguous()
        B, T = tok.shape
        if not isinstance(slots, torch.Tensor):
            sl = [int(v) for v in slots]
            if len(sl) != B or len({v for v in sl if v >= 0}) != sum(1 for v in sl if v >= 0):
                raise ValidationError("slots must name one distinct slot (or -1) per row", "slots")
            slots = torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(self.device)
        check(self.lib.qws_state_note(self.mem.data_ptr(), self.slots, self.V, slots.data_ptr(), B, tok.data_ptr(), T, self._stream()),
              "qws_state_note")

    def read(self, slot: int):
        """The slot's state as dense device arrays (include/qws.h qws_state_read; the reference's smk_engine_read what = 3,
        engine/include/engine.h:173-176): (generated-token counts int32 [V], prompt-set flags uint8 [V])."""
        if not 0 <= slot < self.slots:
            raise ValidationError(f"slot must be in [0, {self.slots}), got {slot}", "slot", slot)
        counts = torch.empty(self.V, dtype=torch.int32, device=self.device)
        flags = torch.empty(self.V, dtype=torch.uint8, device=self.device)
        check(self.lib.qws_state_read(self.mem.data_ptr(), self.slots, self.V, int(slot), counts.data_ptr(), flags.data_ptr(), self._stream()),
              "qws_state_read")
        return counts, flags


class Sampler:
    """Batched sampling stage: B rows of logits [B, V] (fp32 or bf16, on the GPU) -> B tokens.
    One qws_sample call (two kernel launches) on the current stream; the workspace is kept per shape."""

    def __init__(self, device="cuda"):
        self.lib = _lib.load()
        self.device = torch.device(device)
        self._ws = {}

    def workspace(self, B, V):
        key = (B, V)
        if key not in self._ws:
            n = self.lib.qws_sample_ws_bytes(B, V)
            self._ws[key] = torch.empty(n, dtype=torch.uint8, device=self.device)
        return self._ws[key]

    def run(self, packed: PackedBatch, logits: torch.Tensor, out_tokens=None, out_logits=None, out_probs=None, out_info=None, row_stride=None,
            advance: bool = False):
        if logits.dim() != 2 or logits.shape[1] != packed.V or (row_stride != 0 and logits.shape[0] != packed.B):
            raise ValidationError(f"logits shape {tuple(logits.shape)} does not match B={packed.B}, V={packed.V}", "logits")
        if logits.dtype not in (torch.float32, torch.bfloat16) or logits.device.type != "cuda" or logits.stride(1) != 1:
            raise ValidationError("logits must be a CUDA fp32 / bf16 tensor with contiguous rows", "logits")
        if out_tokens is None:
            out_tokens = torch.empty(packed.B, dtype=torch.int32, device=logits.device)
        ws = self.workspace(packed.B, packed.V)
        b = packed.batch(logits, out_tokens, out_logits, out_probs, out_info, row_stride, advance)
        st = torch.cuda.current_stream(logits.device).cuda_stream
        check(self.lib.qws_sample(C.byref(b), ws.data_ptr(), ws.numel(), C.c_void_p(st)), "qws_sample")
        return out_tokens

    def broadcast(self, row: RowSpec, positions, V: int, device) -> PackedBatch:
        """One row description replicated with per-row Philox positions (row-stride-0 calls: many draws
        from the same logits row, as the reference's smk_test_draw)."""
        one = PackedBatch([row], V, device)
        pos = np.asarray(positions, dtype=np.int64) & 0xFFFFFFFF
        n = len(pos)
        rec = np.frombuffer(bytes(one.host_rows[0]), dtype=np.uint8)
        arr = np.tile(rec, (n, 1))
        off = Row.position.offset
        arr[:, off:off + 4] = pos.astype(np.uint32).view(np.uint8).reshape(n, 4)
        one.B = n
        one.rows_t = torch.from_numpy(arr.reshape(-1).copy()).to(torch.device(device))
        return one

    # ------------------------------------------------------------------------------------------ speculative verify
    def verify_map(self, idmap: torch.Tensor, V: int) -> torch.Tensor:
        """The inverse of a drafter's reduced-vocabulary id table (idmap [Vd] int32 target ids, on the GPU):
        int32 [V] holding each target id's reduced index or -1.  Build once per table."""
        if idmap.dtype != torch.int32 or idmap.device.type != "cuda" or idmap.dim() != 1 or not idmap.is_contiguous():
            raise ValidationError("idmap must be a contiguous CUDA int32 vector", "idmap")
        inv = torch.empty(V, dtype=torch.int32, device=idmap.device)
        st = torch.cuda.current_stream(idmap.device).cuda_stream
        check(self.lib.qws_verify_map(idmap.data_ptr(), idmap.numel(), V, inv.data_ptr(), C.c_void_p(st)), "qws_verify_map")
        return inv

    @staticmethod
    def verify_rows(seqs: Sequence[RowSpec], drafts) -> list:
        """The K + 1 target rows of each sequence (engine/src/mtp_sample.cu:227-258 over the rows of
        engine/src/proc.cu:8-29): row t counts d_1..d_t as generated and draws with rng(ctr, ACCEPT + t).y."""
        rows = []
        for r, d in zip(seqs, drafts):
            d = [int(v) for v in d]
            for t in range(len(d) + 1):
                rt = RowSpec(**{k: getattr(r, k) for k in RowSpec.__dataclass_fields__})
                rt.stream, rt.draw_word, rt.drafts = ST_ACCEPT + t, 1, d[:t]
                rt.ngen = len(r.gen) if r.ngen is None else r.ngen
                rows.append(rt)
        return rows

    def verify(self, target_logits: torch.Tensor, draft_probs: torch.Tensor, inv_map: torch.Tensor, drafts: torch.Tensor,
               seqs: Sequence[RowSpec], packed: Optional[PackedBatch] = None, state: Optional[ProcState] = None,
               n_chain: Optional[torch.Tensor] = None, out_probs: Optional[torch.Tensor] = None, out_logits: Optional[torch.Tensor] = None):
        """Speculative verify of B sequences: target_logits [B, K + 1, V] (fp32 / bf16), draft_probs [B, K, Vd] fp32,
        inv_map [V] (verify_map), drafts [B, K] int32 target ids, seqs[b] = sequence b's sampling parameters and
        history (its Philox stream fields are set per row).  Returns (tokens int32 [B, K + 1], -1 past n; n int32 [B]
        = accepted drafts + 1).  One qws_verify call on the current stream.  state: the ProcState of seqs' state_slot.
        n_chain (optional int32 [B] on the GPU): drafts t >= n_chain[b] are delta proposals (prompt-lookup tail tokens:
        q = 1 at the draft, engine/src/mtp_sample.cu:286-296); their draft_probs rows are not read.  out_probs /
        out_logits (optional fp32 [B, K + 1, V] on the GPU): each verify row's sampling distribution / processed logits,
        row t with d_1..d_t counted as generated (the reference's smk_spec_read what = 2, engine/include/mtp.h:57-59)."""
        B, K1, V = target_logits.shape
        K = K1 - 1
        if draft_probs.shape[:2] != (B, K) or draft_probs.dtype != torch.float32 or drafts.shape != (B, K) or drafts.dtype != torch.int32:
            raise ValidationError("draft_probs must be fp32 [B, K, Vd] and drafts int32 [B, K]", "draft_probs")
        if inv_map.dtype != torch.int32 or inv_map.numel() != V or len(seqs) != B:
            raise ValidationError("inv_map must be int32 [V] and seqs hold B rows", "inv_map")
        for t in (target_logits, draft_probs, inv_map, drafts):
            if t.device.type != "cuda" or not t.is_contiguous():
                raise ValidationError("verify tensors must be contiguous CUDA tensors", "target_logits")
        if packed is None:
            packed = PackedBatch(self.verify_rows(seqs, drafts.cpu().tolist()), V, target_logits.device, state)
        if n_chain is not None and (n_chain.dtype != torch.int32 or n_chain.numel() != B or n_chain.device.type != "cuda"):
            raise ValidationError("n_chain must be a CUDA int32 [B] tensor", "n_chain")
        for name, t in (("out_probs", out_probs), ("out_logits", out_logits)):
            if t is not None and (t.shape != (B, K1, V) or t.dtype != torch.float32 or t.device.type != "cuda" or not t.is_contiguous()):
                raise ValidationError(f"{name} must be a contiguous CUDA fp32 [B, K + 1, V] tensor", name)
        vb, ws, out, n = self.verify_call(target_logits, draft_probs, inv_map, drafts, packed, n_chain, out_probs, out_logits)
        st = torch.cuda.current_stream(target_logits.device).cuda_stream
        check(self.lib.qws_verify(C.byref(vb), ws.data_ptr(), ws.numel(), C.c_void_p(st)), "qws_verify")
        return out, n

    def verify_call(self, target_logits: torch.Tensor, draft_probs: torch.Tensor, inv_map: torch.Tensor, drafts: torch.Tensor,
                    packed: PackedBatch, n_chain: Optional[torch.Tensor] = None, out_probs: Optional[torch.Tensor] = None,
                    out_logits: Optional[torch.Tensor] = None):
        """The arguments of one qws_verify call over checked tensors: (VerifyBatch, workspace, out tokens [B, K + 1],
        out n [B]).  A caller that repeats the call on the same buffers builds them once (the batch loop, bench.py)."""
        B, K1, V = target_logits.shape
        K = K1 - 1
        flat = target_logits.view(B * K1, V)
        key = ("verify", B, K, V)
        if key not in self._ws:
            self._ws[key] = torch.empty(self.lib.qws_verify_ws_bytes(B, K, V), dtype=torch.uint8, device=self.device)
        ws = self._ws[key]
        out = torch.empty(B, K1, dtype=torch.int32, device=target_logits.device)
        n = torch.empty(B, dtype=torch.int32, device=target_logits.device)
        vb = VerifyBatch()
        vb.target = packed.batch(flat, out, out_logits=out_logits, out_probs=out_probs)  # target.out_tokens is not used by qws_verify
        vb.B, vb.K, vb.Vd = B, K, draft_probs.shape[2]
        vb.draft_tokens, vb.draft_probs, vb.inv_map = drafts.data_ptr(), draft_probs.data_ptr(), inv_map.data_ptr()
        vb.out_tokens, vb.out_n = out.data_ptr(), n.data_ptr()
        vb.n_chain = n_chain.data_ptr() if n_chain is not None else None
        return vb, ws, out, n

    def draft_pick(self, draft_logits: torch.Tensor, rows: Sequence[RowSpec], idmap: torch.Tensor):
        """The drafter's picks (include/qws.h qws_draft_pick): draft-head logits [B, Vd] over the reduced vocabulary,
        rows from draft_row (stream ST_DRAFT + j), idmap int32 [Vd] (reduced index -> target id) on the GPU.  Returns
        (target ids int32 [B], q fp32 [B, Vd] = the draft_probs rows verify takes, reduced indices int32 [B])."""
        B, Vd = draft_logits.shape
        if idmap.dtype != torch.int32 or idmap.numel() != Vd or idmap.device.type != "cuda" or not idmap.is_contiguous():
            raise ValidationError("idmap must be a contiguous CUDA int32 [Vd] tensor", "idmap")
        packed = PackedBatch(rows, Vd, draft_logits.device)
        red = torch.empty(B, dtype=torch.int32, device=draft_logits.device)
        ids = torch.empty(B, dtype=torch.int32, device=draft_logits.device)
        q = torch.empty(B, Vd, dtype=torch.float32, device=draft_logits.device)  # every entry written by the call
        ws = self.workspace(B, Vd)
        b = packed.batch(draft_logits, red, out_probs=q, row_stride=draft_logits.stride(0))
        st = torch.cuda.current_stream(draft_logits.device).cuda_stream
        check(self.lib.qws_draft_pick(C.byref(b), idmap.data_ptr(), ids.data_ptr(), ws.data_ptr(), ws.numel(), C.c_void_p(st)), "qws_draft_pick")
        return ids, q, red

    def sample(self, logits: torch.Tensor, rows: Sequence[RowSpec], state: Optional[ProcState] = None) -> torch.Tensor:
        packed = PackedBatch(rows, logits.shape[1], logits.device, state)
        return self.run(packed, logits)

    def processed_logits(self, logits: torch.Tensor, rows: Sequence[RowSpec], state: Optional[ProcState] = None) -> torch.Tensor:
        packed = PackedBatch(rows, logits.shape[1], logits.device, state)
        out = torch.empty(logits.shape, dtype=torch.float32, device=logits.device)
        self.run(packed, logits, out_logits=out)
        return out

    def probs(self, logits: torch.Tensor, rows: Sequence[RowSpec]):
        """(tokens, dense probabilities [B, V] (0 outside the kept set), info [B])."""
        packed = PackedBatch(rows, logits.shape[1], logits.device)
        probs = torch.zeros(logits.shape, dtype=torch.float32, device=logits.device)
        info = torch.empty(packed.B, dtype=torch.int32, device=logits.device)
        tok = self.run(packed, logits, out_probs=probs, out_info=info)
        return tok, probs, info


class SeqSampler:
    """One sequence's sampling state with the reference's SpecEngine surface (engine/spec.py:276-311):
    set_sampling / set_procs per request, note() the emitted tokens (proc_note, engine/src/proc.h:52-56),
    row() for the next decode position."""

    def __init__(self, sampler: Optional[Sampler] = None, row_key=0):
        self.sampler = sampler or Sampler()
        self.row_key = row_key
        self.cfg = dict(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, seed=0)
        self.pr = {}
        self.gen = []
        self.position = 0

    def set_sampling(self, temperature=0.0, top_k=20, top_p=1.0, draft_sample=1, draft_temperature=0.0, draft_top_k=0, draft_top_p=0.0, seed=0,
                     test_flags=0, min_p=0.0):
        self.cfg = dict(temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p, seed=seed, test_flags=test_flags)
        self.draft_cfg = dict(temperature=temperature, top_k=top_k, top_p=top_p, draft_sample=draft_sample, draft_temperature=draft_temperature,
                              draft_top_k=draft_top_k, draft_top_p=draft_top_p, seed=seed)
        self.sampling = temperature > 0

    def set_procs(self, prompt=(), presence=0.0, frequency=0.0, repetition=1.0, min_tokens=0, bias=None, allowed=None, stop=()):
        self.pr = dict(prompt=list(prompt), presence=presence, frequency=frequency, repetition=repetition, min_tokens=min_tokens, bias=bias,
                       allowed=allowed, stop=list(stop))
        self.gen = []

    def note(self, tokens):
        self.gen += [int(t) for t in tokens]
        self.position += len(tokens)

    def proc_state(self):
        """(generated-token counts int32 [V], tokens generated so far) -- engine/spec.py:288-292."""
        c = torch.bincount(torch.as_tensor(self.gen, dtype=torch.long), minlength=VOCAB).to(torch.int32) if self.gen else torch.zeros(VOCAB, dtype=torch.int32)
        return c, len(self.gen)

    def row(self, stream=ST_FIRST, position=None) -> RowSpec:
        """The target row at the next position.  The sampling config's test_flags bit0 (broken verify) carries over;
        bit1 keeps the engine's argmax as the first token (k_first_pick, engine/src/mtp_sample.cu:298-311): the
        ST_FIRST row is then greedy."""
        c = self.cfg
        tf = c.get("test_flags", 0)
        temp = 0.0 if (stream == ST_FIRST and tf & 2) else c["temperature"]
        return RowSpec(temperature=temp, top_k=c["top_k"], top_p=c["top_p"], min_p=c["min_p"], seed=c["seed"],
                       test_flags=tf & TF_BROKEN, position=self.position if position is None else position, stream=stream,
                       row_key=self.row_key, gen=list(self.gen), **self.pr)

    def draft_row(self, j: int, position=None) -> RowSpec:
        """The drafter's row for draft j at the next position (draft_row over this sequence's sampling config)."""
        return draft_row(**getattr(self, "draft_cfg", dict(temperature=self.cfg["temperature"], top_k=self.cfg["top_k"], top_p=self.cfg["top_p"],
                                                              seed=self.cfg["seed"])),
                         j=j, position=self.position if position is None else position, row_key=self.row_key)

    def test_draw(self, logits_row: torch.Tensor, n: int, ctr0: int = 0) -> torch.Tensor:
        """n independent draws from the processed distribution of one logits row (counter ctr0 + i, stream
        ST_DRAW): engine/include/mtp.h:118-119 (smk_test_draw).  Rows share the logits (row stride 0)."""
        packed = self.sampler.broadcast(self.row(stream=ST_DRAW), np.arange(ctr0, ctr0 + n), logits_row.shape[-1], logits_row.device)
        return self.sampler.run(packed, logits_row.reshape(1, -1).expand(n, -1), row_stride=0)
