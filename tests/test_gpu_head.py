"""Candidate select + exact rescore over approximate head logits (qws_head_select_rescore through the C ABI) against
the CPU oracle (oracle/head.py): candidate sets and their rank order bit-exact (the select is deterministic given
the logits), exact logits within the fp32 accumulation bound, the logits buffer changed exactly at the candidates,
and the argmax equal to the argmax of the returned exact logits (and to the float64 one wherever the top two are
further apart than the bound).  Cases: the full head shape (N = 248,320, K = 5,120), NaN / tied / flat rows (ties at a
tile's threshold key resolved by index), ragged N, R = 1 and 64, T = 16, and a sub-vocabulary (ids)."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import head as H
from qwen_warp_amd import _lib

pytestmark = pytest.mark.gpu


def run(lib, logits, w, x, R, ids=None):
    T, N = logits.shape
    K = w.shape[1]
    lg = logits.clone().cuda()
    ws = torch.empty(lib.qws_head_ws_bytes(), dtype=torch.uint8, device="cuda")
    tok = torch.empty(T, dtype=torch.int32, device="cuda")
    val = torch.empty(T, dtype=torch.float32, device="cuda")
    idd = ids.cuda() if ids is not None else None
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.qws_head_select_rescore(lg.data_ptr(), w.data_ptr(), x.data_ptr(), N, K, T, R, tok.data_ptr(), val.data_ptr(), ws.data_ptr(),
                                           C.c_void_p(st), idd.data_ptr() if idd is not None else None), "qws_head_select_rescore")
    torch.cuda.synchronize()
    cptr = lib.qws_head_ws_cand(ws.data_ptr())
    eptr = lib.qws_head_ws_exact(ws.data_ptr())
    off_c, off_e = cptr - ws.data_ptr(), eptr - ws.data_ptr()
    wsh = ws.cpu()
    cand = wsh[off_c:off_c + 16 * 64 * 4].view(torch.int32).view(16, 64)
    exact = wsh[off_e:off_e + 16 * 64 * 4].view(torch.float32).view(16, 64)
    return lg.cpu(), tok.cpu(), val.cpu(), cand, exact


def check(lib, logits, w, x, R, ids=None, label=""):
    """w, x on the GPU (bf16); logits on the CPU (fp32)."""
    T, N = logits.shape
    lg, tok, val, cand, exact = run(lib, logits, w, x, R, ids)
    ids_np = ids.numpy() if ids is not None else None
    want = H.select_rescore(logits.numpy(), _RowsOnDemand(w), x.cpu(), R, ids_np)
    for t in range(T):
        wc, wex, wtol = want[t]
        got = cand[t, :R].numpy().astype(np.int64)
        assert (got == wc).all(), f"{label} row {t}: candidates {got[:8]}... != {wc[:8]}..."
        n = int((wc >= 0).sum())
        gex = exact[t, :n].numpy().astype(np.float64)
        assert (np.abs(gex - wex) <= wtol + 1e-30).all(), f"{label} row {t}: exact logits off by {np.abs(gex - wex).max()}"
        # the logits buffer: exact values at the candidates' rows, unchanged elsewhere
        rows = np.where(wc >= 0, wc, -1)[:n] if ids is None else np.searchsorted(ids_np, wc[:n])
        ref = logits[t].clone()
        ref[torch.as_tensor(rows, dtype=torch.long)] = exact[t, :n]
        assert torch.equal(lg[t].view(torch.int32), ref.view(torch.int32)), f"{label} row {t}: logits buffer (bit patterns)"
        if n == 0:
            assert int(tok[t]) == 0
            continue
        order = sorted(range(n), key=lambda i: (-float(exact[t, i]), int(wc[i])))
        assert int(tok[t]) == int(wc[order[0]]) and float(val[t]) == float(exact[t, order[0]]), f"{label} row {t}: argmax"
        o64 = np.argsort(-wex, kind="stable")
        if n > 1 and wex[o64[0]] - wex[o64[1]] > 2 * (wtol[o64[0]] + wtol[o64[1]]):
            assert int(tok[t]) == int(wc[o64[0]]), f"{label} row {t}: float64 argmax"


class _RowsOnDemand:
    """Indexable view of a GPU bf16 head that copies only the requested rows to the CPU."""

    def __init__(self, w):
        self.w = w

    def __getitem__(self, idx):
        return self.w[idx.cuda()].cpu()


def _head(N, K, g, dev="cuda"):
    return (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)


def test_full_head_shape():
    lib = _lib.load()
    g = torch.Generator().manual_seed(1)
    N, K, T = 248320, 5120, 2
    w = (torch.randn(N, K, device="cuda") * 0.02).to(torch.bfloat16)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    approx = (w.float() @ x.float().T).T.cpu() + torch.randn(T, N, generator=g) * 0.01  # a noisy quantised-head stand-in
    for R in (1, 20, 64):
        check(lib, approx.contiguous(), w, x, R, label=f"full R={R}")


@pytest.mark.parametrize("case", ["nan_ties", "flat", "ragged", "few"])
def test_edge_rows(case):
    lib = _lib.load()
    g = torch.Generator().manual_seed(2)
    K = 512
    if case == "ragged":
        N, T = 4096 * 5 + 12, 3
    elif case == "few":
        N, T = 40, 2
    else:
        N, T = 65536, 4
    w = _head(N, K, g)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    lg = torch.randn(T, N, generator=g)
    if case == "nan_ties":
        lg[0, ::7] = float("nan")
        lg[1, :] = torch.round(lg[1, :] * 4) / 4          # many exact ties: lower index first
        lg[2, 100:20000] = 3.0                            # a tied cluster above the rest (the flat paths)
        lg[3, 5] = -0.0
        lg[3, 6] = 0.0
        lg[3, 7:] = -1.0
    elif case == "flat":
        lg[:] = 1.0                                       # every chunk's survivors exceed the counting limit
        lg[1, 12345] = 1.5
    elif case == "few":
        lg[1, 3:] = float("nan")                          # only 3 candidates in row 1
    for R in (1, 7, 64):
        check(lib, lg.contiguous(), w, x, R, label=f"{case} R={R}")


def test_sixteen_rows_and_sub_vocabulary():
    lib = _lib.load()
    g = torch.Generator().manual_seed(3)
    V, K, N, T = 100000, 256, 32768, 16
    w = _head(V, K, g)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    ids = torch.sort(torch.randperm(V, generator=g)[:N]).values.to(torch.int32)
    lg = torch.randn(T, N, generator=g) * 2.0
    check(lib, lg.contiguous(), w, x, 64, ids=ids, label="ids T=16")
    check(lib, lg.contiguous(), w, x, 33, label="T=16")
