"""Host side of the candidate select + exact rescore over a quantised head's approximate logits
(include/qws.h qws_head_select_rescore): the reference's smk_headq_select_rescore(_ids)
(engine/include/head_q.h:29-38, engine/src/head_q.cu:124-302) on torch tensors."""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import _lib
from ._lib import check
from .sampling import ValidationError


class HeadSelect:
    """Keeps the workspace (qws_head_ws_bytes) of one device."""

    def __init__(self, device="cuda"):
        self.lib = _lib.load()
        self.device = torch.device(device)
        self.ws = torch.empty(self.lib.qws_head_ws_bytes(), dtype=torch.uint8, device=self.device)

    def __call__(self, logits: torch.Tensor, w_bf16: torch.Tensor, x: torch.Tensor, R: int, ids: Optional[torch.Tensor] = None):
        """logits fp32 [T, N] (updated in place at the candidates), w_bf16 [rows, K], x bf16 [T, K], ids int32 [N]
        (ascending token ids of the logits rows) or None.  Returns (out_tok int32 [T], out_val fp32 [T],
        candidates int32 [T, R] in rank order (-1 past the last), their exact logits fp32 [T, R])."""
        if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_contiguous():
            raise ValidationError("logits must be a contiguous fp32 [T, N] tensor", "logits")
        if w_bf16.dtype != torch.bfloat16 or x.dtype != torch.bfloat16 or not (w_bf16.is_contiguous() and x.is_contiguous()):
            raise ValidationError("w and x must be contiguous bf16 tensors", "w_bf16")
        T, N = logits.shape
        K = w_bf16.shape[1]
        if x.shape != (T, K):
            raise ValidationError("x must be [T, K]", "x")
        if ids is not None and (ids.dtype != torch.int32 or ids.numel() != N):
            raise ValidationError("ids must be int32 [N]", "ids")
        tok = torch.empty(T, dtype=torch.int32, device=self.device)
        val = torch.empty(T, dtype=torch.float32, device=self.device)
        st = C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        check(self.lib.qws_head_select_rescore(logits.data_ptr(), w_bf16.data_ptr(), x.data_ptr(), N, K, T, int(R), tok.data_ptr(), val.data_ptr(),
                                               self.ws.data_ptr(), st, ids.data_ptr() if ids is not None else None), "qws_head_select_rescore")
        base = self.ws.data_ptr()
        oc = self.lib.qws_head_ws_cand(base) - base
        oe = self.lib.qws_head_ws_exact(base) - base
        cand = self.ws[oc:oc + 16 * 64 * 4].view(torch.int32).view(16, 64)[:T, :R]
        exact = self.ws[oe:oe + 16 * 64 * 4].view(torch.float32).view(16, 64)[:T, :R]
        return tok, val, cand, exact
