"""qws_sample_noalloc (the entry point that allocates nothing: its workspace is the library's own device array)
against qws_sample with a caller workspace, through the C ABI: tokens, probabilities and the info word identical on
two calls in a row, the second smaller; a batch past the array's size is rejected."""
import ctypes as C

import pytest
import torch

import qwen_warp_amd as q
from qwen_warp_amd import _lib, workloads

pytestmark = pytest.mark.gpu


def _run(lib, packed, logits, noalloc):
    B = packed.B
    tok = torch.full((B,), -5, dtype=torch.int32, device="cuda")
    probs = torch.zeros(logits.shape, dtype=torch.float32, device="cuda")
    info = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    b = packed.batch(logits, tok, out_probs=probs, out_info=info)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        _lib.check(lib.qws_sample_noalloc(C.byref(b), st), "qws_sample_noalloc")
    else:
        ws = torch.empty(lib.qws_sample_ws_bytes(B, packed.V), dtype=torch.uint8, device="cuda")
        _lib.check(lib.qws_sample(C.byref(b), C.c_void_p(ws.data_ptr()), ws.numel(), st), "qws_sample")
    torch.cuda.synchronize()
    return tok.cpu(), probs.cpu(), info.cpu()


def test_noalloc_matches_workspace_entry_point():
    lib = _lib.load()
    torch.cuda.set_device(0)
    # first call: C4's parameters at the array's largest batch (15 rows x 31 blocks at V = 248,320); second call: three
    # bf16 rows of config 5 (bias, min_tokens, banned bits), a smaller input in a shorter vocabulary slice
    w1 = workloads.c4(B=15)
    w2 = workloads.c5(B=3)
    cases = [(w1.logits.cuda(), q.PackedBatch(w1.rows, w1.logits.shape[1], "cuda")),
             (w2.logits[:, :100000].contiguous().cuda(), None)]
    rows2 = []
    for r in w2.rows:
        r2 = q.RowSpec(temperature=r.temperature, top_k=r.top_k, top_p=0.9, min_tokens=r.min_tokens, ngen=r.ngen, stop=[5, 77],
                       bias={k: v for k, v in r.bias.items() if k < 100000}, seed=r.seed, row_key=r.row_key)
        rows2.append(r2)
    cases[1] = (cases[1][0], q.PackedBatch(rows2, 100000, "cuda"))
    for i, (lg, packed) in enumerate(cases):
        want = _run(lib, packed, lg, noalloc=False)
        got = _run(lib, packed, lg, noalloc=True)
        assert torch.equal(got[0], want[0]), f"call {i}: tokens differ"
        assert torch.equal(got[1], want[1]), f"call {i}: probabilities differ"
        assert torch.equal(got[2], want[2]), f"call {i}: info differs"
        assert int((want[0] < 0).sum()) == 0


def test_noalloc_rejects_batches_past_the_array():
    lib = _lib.load()
    w = workloads.c4(B=16)  # 16 x 31 records exceed 16 MiB
    assert lib.qws_sample_ws_bytes(16, w.logits.shape[1]) > _lib.NOALLOC_SCRATCH_BYTES
    packed = q.PackedBatch(w.rows, w.logits.shape[1], "cuda")
    lg = w.logits.cuda()
    tok = torch.empty(16, dtype=torch.int32, device="cuda")
    b = packed.batch(lg, tok)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.qws_sample_noalloc(C.byref(b), st) == _lib.ERR_NOT_SUPPORTED
