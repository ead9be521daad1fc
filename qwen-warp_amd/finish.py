"""Host side of the device decode-step bookkeeping (include/qws.h qws_finish): the reference's spec_finish
(engine/src/mtp_sample.h:65-92) for many sequences per launch, fused with proc_note (ProcState) and the PLD
history append (DevicePld)."""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import Seq, check
from .sampling import ProcState, ValidationError

SEQ_WORDS = C.sizeof(Seq) // 4


class StepBook:
    """`nseq` sequences' bookkeeping (qws_seq) and output rings of `ring_len` tokens, on the GPU."""

    def __init__(self, nseq: int, ring_len: int = 4096, device="cuda"):
        self.lib = _lib.load()
        self.nseq, self.ring_len = int(nseq), int(ring_len)
        self.device = torch.device(device)
        self.seqs = torch.zeros(self.nseq, SEQ_WORDS, dtype=torch.int32, device=self.device)
        self.rings = torch.full((self.nseq, self.ring_len), -1, dtype=torch.int32, device=self.device)

    def start(self, seq: int, pos: int, last: int):
        """A sequence starts at position `pos` after token `last` (its counters and ring cleared)."""
        row = torch.zeros(SEQ_WORDS, dtype=torch.int32)
        row[0], row[1] = int(pos), int(last)
        self.seqs[seq] = row.to(self.device)
        self.rings[seq].fill_(-1)

    def finish(self, row_seqs, tokens: torch.Tensor, counts: Optional[torch.Tensor] = None, state: Optional[ProcState] = None, pld=None,
               rows=None, rows_per_entry: int = 1, force: Optional[torch.Tensor] = None):
        """tokens int32 [B, T <= 64] (or [B]) on the GPU, a sampling or verify call's output; counts int32 [B] (a verify
        call's out_n) or None (tokens before the first negative one).  rows: the next call's rows (a PackedBatch, or its
        device row array) to advance on the GPU (qws_finish_rows: counter word 0 += 1, ngen += a for the rows_per_entry
        rows of each entry), so the step needs nothing from the host.  force (int32 [n] on the GPU): the reference's
        forced-acceptance schedule (smk_spec_set_force, engine/include/mtp.h:49-50): a sequence's step keeps
        min(a, force[cycles % n]) tokens (qws_finish_forced)."""
        if tokens.dtype != torch.int32 or tokens.device.type != "cuda":
            raise ValidationError("tokens must be an int32 CUDA tensor", "tokens")
        tok = tokens.reshape(tokens.shape[0], -1).contiguous()
        B, T = tok.shape
        if isinstance(row_seqs, torch.Tensor):
            rs = row_seqs.to(device=self.device, dtype=torch.int32).contiguous()
        else:
            sl = [int(v) for v in row_seqs]
            if len(sl) != B or len({v for v in sl if v >= 0}) != sum(1 for v in sl if v >= 0):
                raise ValidationError("one distinct sequence (or -1) per row", "row_seqs")
            rs = torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(self.device)
        if counts is not None and (counts.dtype != torch.int32 or counts.numel() != B or counts.device.type != "cuda"):
            raise ValidationError("counts must be an int32 CUDA tensor [B]", "counts")
        st = C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        args = (self.seqs.data_ptr(), self.nseq, self.rings.data_ptr(), self.ring_len, rs.data_ptr(), B, tok.data_ptr(),
                counts.data_ptr() if counts is not None else None, T,
                state.mem.data_ptr() if state is not None else None, state.slots if state is not None else 0, state.V if state is not None else 0,
                pld.mem.data_ptr() if pld is not None else None, pld.seqs if pld is not None else 0, pld.max_len if pld is not None else 0)
        rt = None
        if rows is not None:
            if hasattr(rows, "check_advance"):
                rows.check_advance()
            rt = rows.rows_t if hasattr(rows, "rows_t") else rows
            if rt.device.type != "cuda" or rt.numel() < B * rows_per_entry * C.sizeof(_lib.Row):
                raise ValidationError(f"rows must hold {B} x {rows_per_entry} device rows", "rows")
        if force is not None:
            if force.dtype != torch.int32 or force.device.type != "cuda" or force.dim() != 1 or not force.is_contiguous():
                raise ValidationError("force must be a contiguous CUDA int32 vector", "force")
            check(self.lib.qws_finish_forced(*args, rt.data_ptr() if rt is not None else None, rows_per_entry, force.data_ptr(), force.numel(), st),
                  "qws_finish_forced")
        elif rt is None:
            check(self.lib.qws_finish(*args, st), "qws_finish")
        else:
            check(self.lib.qws_finish_rows(*args, rt.data_ptr(), rows_per_entry, st), "qws_finish_rows")

    def read(self, seq: int) -> dict:
        r = self.seqs[seq].cpu().tolist()
        return dict(pos=r[0], last=r[1], outn=r[2], cycles=r[3], hist=r[4:12])
