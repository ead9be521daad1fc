"""Host side of the device prompt-lookup (PLD) tail proposer (include/qws.h qws_pld_*).

Mirrors the reference's proposer handle (engine/include/pld.h:22-39: create / reset / append / propose) for many
sequences at once, with the histories on the GPU: `reset` per sequence at admission, `append` with the tokens a
sampling or verify call emitted (device tensors, -1 padding ignored), `propose` after the drafts of a cycle.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import PldCfg, check
from .sampling import ValidationError


def default_cfg() -> PldCfg:
    """engine/src/pld.cu:45-52 (smk_pld_default_cfg)."""
    c = PldCfg()
    _lib.load().qws_pld_default_cfg(C.byref(c))
    return c


class DevicePld:
    """`seqs` PLD histories of at most `max_len` tokens each, in one device arena."""

    def __init__(self, seqs: int, max_len: int = 1 << 17, cfg: Optional[PldCfg] = None, device="cuda"):
        self.lib = _lib.load()
        self.seqs, self.max_len = int(seqs), int(max_len)
        n = self.lib.qws_pld_bytes(self.seqs, self.max_len)
        if n == 0:
            raise ValidationError(f"no PLD arena for seqs={seqs}, max_len={max_len}", "seqs")
        self.cfg = cfg if cfg is not None else default_cfg()
        self.device = torch.device(device)
        self.mem = torch.empty(n, dtype=torch.uint8, device=self.device)

    def _stream(self):
        return C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def _slots(self, seqs, B):
        if isinstance(seqs, torch.Tensor):
            return seqs.to(device=self.device, dtype=torch.int32).contiguous()
        sl = [int(v) for v in seqs]
        if len(sl) != B:
            raise ValidationError("one sequence (or -1) per row", "seqs")
        return torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(self.device)

    def reset(self, seq: int, ctx: Sequence[int]):
        """engine/src/pld.cu:64-69: the history of `seq` <- ctx (its last token is the anchor)."""
        if not 0 <= seq < self.seqs:
            raise ValidationError(f"seq must be in [0, {self.seqs}), got {seq}", "seq", seq)
        if len(ctx) > self.max_len:
            raise ValidationError(f"context longer than {self.max_len} tokens", "ctx", len(ctx))
        t = torch.as_tensor(np.asarray(list(ctx) or [0], dtype=np.int32)).to(self.device)
        check(self.lib.qws_pld_reset(self.mem.data_ptr(), self.seqs, self.max_len, int(seq), t.data_ptr(), len(ctx), self._stream()), "qws_pld_reset")

    def append(self, seqs, tokens: torch.Tensor):
        """engine/src/pld.cu:71-76: tokens int32 [B] or [B, T <= 64] on the GPU, each row up to its first negative value."""
        if tokens.dtype != torch.int32 or tokens.device.type != "cuda":
            raise ValidationError("tokens must be an int32 CUDA tensor", "tokens")
        tok = tokens.reshape(tokens.shape[0], -1).contiguous()
        B, T = tok.shape
        sl = self._slots(seqs, B)
        check(self.lib.qws_pld_append(self.mem.data_ptr(), self.seqs, self.max_len, sl.data_ptr(), B, tok.data_ptr(), T, self._stream()),
              "qws_pld_append")

    def propose(self, seqs, drafts: Optional[torch.Tensor] = None, max_tail: Optional[int] = None, min_len: Optional[int] = None):
        """engine/src/pld.cu:88-121 for every row: drafts int32 [B, nd] on the GPU (None: nd = 0).  Returns
        (tails int32 [B, 8], -1 after each tail; lengths int32 [B]; agreement lengths int32 [B])."""
        B = len(seqs) if not isinstance(seqs, torch.Tensor) else seqs.numel()
        sl = self._slots(seqs, B)
        if drafts is None:
            nd, dp = 0, None
        else:
            if drafts.dtype != torch.int32 or drafts.device.type != "cuda" or drafts.dim() != 2 or drafts.shape[0] != B:
                raise ValidationError("drafts must be an int32 CUDA tensor [B, nd]", "drafts")
            drafts = drafts.contiguous()
            nd, dp = drafts.shape[1], drafts.data_ptr()
        mt = self.cfg.max_tail if max_tail is None else int(max_tail)
        ml = self.cfg.min_len if min_len is None else int(min_len)
        out = torch.empty(B, 8, dtype=torch.int32, device=self.device)
        n = torch.empty(B, dtype=torch.int32, device=self.device)
        l = torch.empty(B, dtype=torch.int32, device=self.device)
        check(self.lib.qws_pld_propose(self.mem.data_ptr(), self.seqs, self.max_len, C.byref(self.cfg), sl.data_ptr(), B, dp, nd, mt, ml,
                                       out.data_ptr(), n.data_ptr(), l.data_ptr(), self._stream()), "qws_pld_propose")
        return out, n, l
