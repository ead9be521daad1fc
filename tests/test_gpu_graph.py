"""qws_sample and qws_verify inside a captured HIP graph (torch.cuda.CUDAGraph over the current stream): the calls
allocate nothing and launch only kernels, so a captured step replays to the same tokens as the eager call.  The
replays run several times, with eager work and synchronisations between them, and every replay is checked."""
import pytest
import torch

import qwen_warp_amd as q
from qwen_warp_amd import workloads

pytestmark = pytest.mark.gpu


def test_sample_graph_replays():
    sm = q.Sampler("cuda")
    w = workloads.c5(B=8)
    packed = q.PackedBatch(w.rows, w.logits.shape[1], "cuda")
    lg = w.logits.cuda()
    want = sm.run(packed, lg).clone()
    torch.cuda.synchronize()
    out = torch.full((packed.B,), -7, dtype=torch.int32, device="cuda")
    sm.workspace(packed.B, packed.V)  # allocated before capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        sm.run(packed, lg, out_tokens=out)  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            sm.run(packed, lg, out_tokens=out)
    torch.cuda.synchronize()
    for rep in range(4):
        out.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}: {out.tolist()} != {want.tolist()}"
        _ = sm.run(packed, lg)  # eager work between replays
        torch.cuda.synchronize()


def test_verify_graph_replays():
    sm = q.Sampler("cuda")
    w = workloads.c3(B=2, K=4, Vd=4096)
    x = w.extra
    tl, dp = w.logits.cuda(), x["draft_probs"].cuda()
    inv = sm.verify_map(x["idmap"].cuda(), tl.shape[2])
    d = x["drafts"].cuda()
    want_t, want_n = sm.verify(tl, dp, inv, d, w.rows)
    torch.cuda.synchronize()
    packed = q.PackedBatch(sm.verify_rows(w.rows, x["drafts"].tolist()), tl.shape[2], "cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        sm.verify(tl, dp, inv, d, w.rows, packed=packed)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            got_t, got_n = sm.verify(tl, dp, inv, d, w.rows, packed=packed)
    torch.cuda.synchronize()
    for rep in range(3):
        got_t.fill_(-9)
        got_n.fill_(-9)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got_t, want_t) and torch.equal(got_n, want_n), f"replay {rep}"
